"""CPU checker for rvllm_amd.attn_model.HipBackend (test infrastructure):
the same attention-only decoder computed with the oracle - f16 paged cache,
oracle attn_prep, float64 paged prefill/decode attention, numpy f32 GEMMs,
the oracle's greedy argmax - and a lock-step backend that runs both on every
forward, compares the logits and returns the GPU's tokens."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np

from oracle import oracle as orc
from rvllm_amd.attn_model import logit_scale, padded_tables
from rvllm_amd.rope import rope_cos_sin


class OracleBackend:
    def __init__(self, cfg, weights, num_blocks, block_size):
        self.cfg, self.w = cfg, weights
        self.config = SimpleNamespace(context_length=cfg.context_length)
        self.caches = [orc.KvCache(num_blocks, block_size, cfg.n_kv_heads,
                                   cfg.head_dim, orc.F16)
                       for _ in range(cfg.n_layers)]
        self.last_logits = None

    def release(self, seq_id):
        pass

    def copy_blocks(self, src, dst):
        for c in self.caches:
            c.copy_blocks(np.asarray(src, np.uint32),
                          np.asarray(dst, np.uint32))

    def forward_sample(self, items, last_only, samplers):
        c, w = self.cfg, self.w
        H, KV, hd = c.n_heads, c.n_kv_heads, c.head_dim
        toks = np.concatenate([np.asarray(it.tokens, np.int64)
                               for it in items])
        pos = np.concatenate([it.position_offset + np.arange(len(it.tokens))
                              for it in items])
        slots = np.array([p for it in items for p in it.write_positions],
                         np.uint32).reshape(-1, 2)
        rows = len(toks)
        cos, sin = rope_cos_sin(c.rope_theta, hd, pos)
        tables = padded_tables(items)
        mb = tables.shape[1]
        x = w["embed"][toks].astype(np.float32)
        decode = not last_only and all(len(it.tokens) == 1 for it in items)
        for l in range(c.n_layers):
            q = (x @ w[f"wq{l}"]).reshape(rows, H, hd)
            k = (x @ w[f"wk{l}"]).reshape(rows, KV, hd)
            v = (x @ w[f"wv{l}"]).reshape(rows, KV, hd)
            qr = orc.attn_prep(self.caches[l], q, k, v, cos, sin, slots[:, 0],
                               slots[:, 1], w.get(f"bq{l}"), w.get(f"bk{l}"),
                               w.get(f"bv{l}"), w.get(f"qn{l}"),
                               w.get(f"kn{l}"), c.eps)
            if decode:
                att = orc.paged_decode_f64(
                    self.caches[l], qr, tables.reshape(-1), mb,
                    [it.read_num_tokens for it in items], window=c.window)
            else:
                att = np.empty_like(qr)
                r0 = 0
                for i, it in enumerate(items):
                    n = len(it.tokens)
                    att[r0:r0 + n] = orc.paged_prefill_f64(
                        self.caches[l], qr[r0:r0 + n].reshape(1, n, H, hd),
                        tables[i], mb, [it.position_offset],
                        [it.read_num_tokens], window=c.window)[0]
                    r0 += n
            x = x + att.reshape(rows, H * hd) @ w[f"wo{l}"]
        last = np.cumsum([len(it.tokens) for it in items]) - 1
        logits = (x[last] @ w["embed"].T) * np.float32(logit_scale(c))
        self.last_logits = logits.astype(np.float32)
        return orc.argmax_rows(self.last_logits).tolist()


class LockstepBackend:
    """Runs the GPU and the CPU backend on every call; records the worst
    logit difference and any token the two pick differently (allowed only
    where the oracle's top-2 margin is within the tolerance)."""

    def __init__(self, gpu, cpu, atol=2e-3, rtol=2e-3):
        self.gpu, self.cpu = gpu, cpu
        self.config = gpu.config
        self.atol, self.rtol = atol, rtol
        self.worst = 0.0
        self.calls = 0
        self.close_calls = []  # (margin, gpu token, cpu token)

    def release(self, seq_id):
        self.gpu.release(seq_id)
        self.cpu.release(seq_id)

    def copy_blocks(self, src, dst):
        self.gpu.copy_blocks(src, dst)
        self.cpu.copy_blocks(src, dst)

    def forward_sample(self, items, last_only, samplers):
        g = self.gpu.forward_sample(items, last_only, samplers)
        c = self.cpu.forward_sample(items, last_only, samplers)
        gl = self.gpu.last_logits.cpu().numpy()
        cl = self.cpu.last_logits
        tol = self.atol + self.rtol * float(np.abs(cl).max())
        err = float(np.abs(gl - cl).max())
        self.worst = max(self.worst, err / tol)
        assert err <= tol, (err, tol)
        # The GPU argmax must be exactly the greedy scan of its own logits.
        assert g == orc.argmax_rows(gl).tolist()
        for r, (a, b) in enumerate(zip(g, c)):
            if a != b:
                top = np.sort(cl[r])[-2:]
                self.close_calls.append((float(top[1] - top[0]), a, b))
                assert top[1] - top[0] <= 2 * tol
        self.calls += 1
        return g
