"""Continuous-batching decode driver over the native block manager.

Drives the paged KV path the way rvllm's engine does (src/engine.rs:344-490)
for the gemma-3-270m churn workload:
- every step a fraction of the running sequences finishes, and their blocks
  return to a seeded-shuffled, fragmented free list;
- the same number of new sequences is admitted with short prompts, whose
  K/V rows of every layer are appended in one launch (prefill append,
  rvkv_append_layers);
- then every running sequence decodes one token: its slot comes from
  logical_to_physical(num_tokens) (rvkv_bm_append_slots), and one fused
  rvkv_decode_step per layer runs under a decode plan rebuilt from the
  host-side token counts (the per-forward GatherPlan).

Host bookkeeping of the next steps overlaps the GPU work of step s. The
host arrays go through pinned staging used in turn (three sets, as the
decode plan's own staging) and non-blocking uploads.
K/V/q contents are synthetic (seeded device RNG); only the bookkeeping and
the data movement are real.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import RVKV_F32, check
from .block_manager import BlockManager
from .kv_storage import HipDecodePlan, HipKvStorage
from .workloads import Config, Rng, append_bytes

NSTAGE = 3  # host staging sets (the decode plan keeps as many)


class ChurnDriver:
    def __init__(self, cfg: Config, batch: int, init_ctx: int,
                 prompt_len: int = 64, churn: float = 0.10,
                 pool_factor: float = 1.25, steps: int = 200,
                 seed: int = 0, fill: bool = True):
        self.cfg, self.batch, self.prompt_len = cfg, batch, prompt_len
        bs = cfg.block_size
        self.n_churn = int(round(churn * batch))
        live = batch * -(-init_ctx // bs)
        self.num_blocks = int(np.ceil(pool_factor * live))
        # Longest possible sequence: an initial one that survives every step.
        self.max_blocks = -(-(init_ctx + steps + 1) // bs)
        self.rng = Rng(seed or cfg.seed)
        self.bm = BlockManager(self.num_blocks, bs)
        self.bm.shuffle_free(self.rng.u64())
        self.st = HipKvStorage(cfg.n_layers, self.num_blocks, bs,
                               cfg.n_kv_heads, cfg.head_dim)
        dev = self.st.device
        g = torch.Generator(device="cuda")
        g.manual_seed(cfg.seed)
        if fill:
            self._fill(g)
        # Sequences hold init_ctx - 1 tokens; the first step appends one.
        self.running = np.array([self.bm.add_seq(init_ctx - 1)
                                 for _ in range(batch)], np.int64)
        L, H, KV, hd = cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        self.q = [torch.randn((batch, H, hd), generator=g, device=dev)
                  for _ in range(L)]
        self.nk = [torch.randn((batch, KV, hd), generator=g, device=dev)
                   for _ in range(L)]
        self.nv = [torch.randn((batch, KV, hd), generator=g, device=dev)
                   for _ in range(L)]
        n_prompt = max(1, self.n_churn * prompt_len)
        # Each layer's rows of the admitted prompts (f32, as a prefill's
        # projections leave them).
        self.pk = torch.randn((L, n_prompt, KV, hd), generator=g, device=dev)
        self.pv = torch.randn((L, n_prompt, KV, hd), generator=g, device=dev)
        self.out = [torch.empty_like(self.q[0]) for _ in range(L)]
        P = ctypes.c_void_p
        self._q_p = [P(t.data_ptr()) for t in self.q]
        self._nk_p = [P(t.data_ptr()) for t in self.nk]
        self._nv_p = [P(t.data_ptr()) for t in self.nv]
        self._out_p = [P(t.data_ptr()) for t in self.out]
        # Pinned staging + device copies of the step arrays, NSTAGE sets used
        # in turn, so the host can prepare a few steps ahead of the device.
        # Each set is one buffer (arrays at 256-byte offsets), moved by one
        # copy a step: six copies a step left ~5 us of dispatch gap each.
        mb = self.max_blocks
        shapes = {"tables": (batch, mb), "ctx": (batch,), "sb": (batch,),
                  "so": (batch,), "pb": (n_prompt,), "po": (n_prompt,)}
        offs, n = {}, 0
        for k, s in shapes.items():
            offs[k] = n
            n += -(-int(np.prod(s)) // 64) * 64
        self.host_flat = [torch.empty(n, dtype=torch.int32, pin_memory=True)
                          for _ in range(NSTAGE)]
        self.dev_flat = [torch.empty(n, dtype=torch.int32, device=dev)
                         for _ in range(NSTAGE)]

        def views(flat):
            return {k: flat[offs[k]:offs[k] + int(np.prod(s))].view(s)
                    for k, s in shapes.items()}

        self.host = [views(f) for f in self.host_flat]
        self.devb = [views(f) for f in self.dev_flat]
        self.copied = [torch.cuda.Event() for _ in range(NSTAGE)]
        self.plan = None
        self.step_index = 0
        self.bytes_moved = 0
        self.last = None  # host copy of the last step's decode inputs

    def _fill(self, g) -> None:
        st = self.st
        bs, nkv, hd = st.block_size, st.n_kv_heads, st.head_dim
        total = st.num_blocks * bs
        chunk = max(1, (1 << 28) // (nkv * hd * 2))
        for layer in range(st.n_layers):
            for t0 in range(0, total, chunk):
                n = min(chunk, total - t0)
                s = torch.arange(t0, t0 + n, device="cuda", dtype=torch.int64)
                k = torch.randn((n, nkv, hd), generator=g, device="cuda",
                                dtype=torch.float16)
                v = torch.randn((n, nkv, hd), generator=g, device="cuda",
                                dtype=torch.float16)
                st.write_tokens(layer, (s // bs).to(torch.int32),
                                (s % bs).to(torch.int32), k, v)
        torch.cuda.synchronize()

    def step(self) -> None:
        """One engine step: finish + admit (prefill append), then decode."""
        c, bm, st = self.cfg, self.bm, self.st
        i = self.step_index % NSTAGE
        hb, db = self.host[i], self.devb[i]
        self.copied[i].synchronize()  # staging i is free again
        bs = c.block_size
        n_prompt_tok = 0
        if self.step_index > 0 and self.n_churn:
            # Finish a seeded random subset, admit as many new prompts in
            # their places.
            idx = self.rng.np.choice(self.batch, self.n_churn, replace=False)
            bm.free_seqs(self.running[idx])
            new = bm.add_seqs(np.full(len(idx), self.prompt_len, np.uint32))
            self.running[idx] = new
            tabs, _ = bm.fill_tables(new, -(-self.prompt_len // bs))
            pos = np.arange(self.prompt_len)
            pb = tabs[:, pos // bs].reshape(-1)
            po = np.tile(pos % bs, len(new))
            n_prompt_tok = len(pb)
            hb["pb"][:n_prompt_tok].numpy().view(np.uint32)[:] = pb
            hb["po"][:n_prompt_tok].numpy().view(np.uint32)[:] = po
        blocks, offs, cs, cd = bm.append_slots(self.running)
        tables = hb["tables"].numpy().view(np.uint32)
        lens = hb["ctx"].numpy().view(np.uint32)
        bm.fill_tables(self.running, self.max_blocks, out=tables,
                       lens_out=lens)
        hb["sb"].numpy().view(np.uint32)[:] = blocks
        hb["so"].numpy().view(np.uint32)[:] = offs
        self.dev_flat[i].copy_(self.host_flat[i], non_blocking=True)
        self.copied[i].record()
        if len(cs):
            st.copy_blocks(torch.from_numpy(cs.view(np.int32)).cuda(),
                           torch.from_numpy(cd.view(np.int32)).cuda())
        if self.plan is None:
            self.plan = HipDecodePlan(st, lens, c.n_heads, window=c.window)
        else:
            self.plan.update(lens)
        self._layers(db, n_prompt_tok)
        self.bytes_moved += c.n_layers * (
            self.decode_bytes(lens) + append_bytes(self.batch, c)
            + append_bytes(n_prompt_tok, c))
        self.last = (tables.copy(), lens.copy(), blocks.copy(), offs.copy())
        # This step's prompt slots (rows pk/pv[:n] went there), for checks.
        self.last_prompt = (
            hb["pb"][:n_prompt_tok].numpy().view(np.uint32).copy(),
            hb["po"][:n_prompt_tok].numpy().view(np.uint32).copy())
        self.step_index += 1

    def _layers(self, db, n_prompt_tok) -> None:
        """The per-layer launches (prompt append, fused decode step) through
        the C ABI with arguments validated once here; the same calls as
        HipKvStorage.write_tokens / decode_step without their per-call
        Python checks."""
        c, st, L = self.cfg, self.st, self.st._L
        P = ctypes.c_void_p
        plan, ws = self.plan, self.plan.ws
        ws_p = P(ws.data_ptr()) if ws is not None else None
        ws_n = ws.numel() if ws is not None else 0
        pb, po = P(db["pb"].data_ptr()), P(db["po"].data_ptr())
        sb, so = P(db["sb"].data_ptr()), P(db["so"].data_ptr())
        tables, ctx = P(db["tables"].data_ptr()), P(db["ctx"].data_ptr())
        pk, pv = P(self.pk.data_ptr()), P(self.pv.data_ptr())
        scale = 1.0 / np.sqrt(c.head_dim)
        if n_prompt_tok:
            # The admitted prompts' rows of every layer in one launch.
            check(L.rvkv_append_layers(
                st._pool, 0, c.n_layers, pk, pv, RVKV_F32,
                self.pk.shape[1] * c.n_kv_heads * c.head_dim, pb, po,
                n_prompt_tok))
        for layer in range(c.n_layers):
            check(L.rvkv_decode_step(
                st._pool, plan._plan, layer, self._nk_p[layer],
                self._nv_p[layer], RVKV_F32, sb, so, self._q_p[layer], tables,
                ctx, self.batch, self.max_blocks, c.n_heads, 0, scale,
                c.window, self._out_p[layer], ws_p, ws_n))

    def close(self) -> None:
        """Frees the plan and the pool (the block manager frees with the
        object)."""
        if self.plan is not None:
            self.plan.close()
            self.plan = None
        self.st.close()

    def decode_bytes(self, lens) -> int:
        """Algorithmic bytes of one decode launch at these lengths."""
        c = self.cfg
        kv = int(lens.astype(np.int64).sum()) * c.n_kv_heads * c.head_dim * 4
        qo = self.batch * c.n_heads * c.head_dim * 8
        tables = 4 * int((-(-lens.astype(np.int64) // c.block_size)).sum())
        return kv + qo + tables + 4 * self.batch
