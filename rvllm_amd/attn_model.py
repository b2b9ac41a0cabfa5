"""A synthetic attention-only decoder and its GPU backend for the engine.

This is the harness that drives the paged KV path the way rvllm's forward
does (src/model.rs:600-644 per layer; the CUDA backend's forward_sample,
src/cuda/engine.rs:339-404): token embedding, then per layer the Q/K/V
projection (one fused QKV GEMM), attention prep with the K/V append
(rvkv_attn_prep_qkv),
attention straight over the paged cache (rvkv_paged_prefill for a prefill
item, rvkv_paged_decode_planned under a per-forward decode plan for a decode
batch) and the output projection with
a residual add; then tied-embedding logits and the greedy pick on the GPU
(rvkv_argmax). The MLP, norms and real checkpoints are outside the KV path
and left out: the weights are seeded random. The projections are plain
library GEMMs (torch on the GPU); every KV-path step is this library's HIP
code.

Sampling is greedy only (the GPU argmax), like the reference's CUDA
backend fast path for SamplingParams::GREEDY (src/cuda/engine.rs:96-125).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Dict, List

import numpy as np
import torch

from . import _lib
from ._lib import check
from .kv_storage import HipDecodePlan, HipKvStorage
from .rope import rope_cos_sin


@dataclass
class AttnModelConfig:
    vocab: int = 1024
    hidden: int = 256
    n_layers: int = 2
    n_heads: int = 8
    n_kv_heads: int = 2
    head_dim: int = 64
    qkv_bias: bool = False
    qk_norm: bool = False
    rope_theta: float = 10000.0
    eps: float = 1e-6
    context_length: int = 4096
    window: int = 0
    seed: int = 1234


def init_weights(cfg: AttnModelConfig) -> Dict[str, np.ndarray]:
    """Seeded f32 weights (host). Projections are scaled so q/k/v and the
    attention output keep unit-order magnitudes."""
    rng = np.random.default_rng(cfg.seed)
    D, H, KV, hd = cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    f = lambda *s, scale=1.0: (rng.standard_normal(s) * scale).astype(
        np.float32)
    w = {"embed": f(cfg.vocab, D)}
    for l in range(cfg.n_layers):
        w[f"wq{l}"] = f(D, H * hd, scale=1 / math.sqrt(D))
        w[f"wk{l}"] = f(D, KV * hd, scale=1 / math.sqrt(D))
        w[f"wv{l}"] = f(D, KV * hd, scale=1 / math.sqrt(D))
        w[f"wo{l}"] = f(H * hd, D, scale=1 / math.sqrt(H * hd))
        if cfg.qkv_bias:
            w[f"bq{l}"] = f(H * hd, scale=0.5)
            w[f"bk{l}"] = f(KV * hd, scale=0.5)
            w[f"bv{l}"] = f(KV * hd, scale=0.5)
        if cfg.qk_norm:
            w[f"qn{l}"] = (1.0 + f(hd, scale=0.2)).astype(np.float32)
            w[f"kn{l}"] = (1.0 + f(hd, scale=0.2)).astype(np.float32)
    return w


def logit_scale(cfg: AttnModelConfig) -> float:
    return 1.0 / math.sqrt(cfg.hidden)


def padded_tables(items) -> np.ndarray:
    """[batch, max_blocks] u32 block tables, padded with each row's last
    block (GatherPlan's padding, src/kv_storage.rs:50-75)."""
    mb = max(1, max(len(it.read_blocks) for it in items))
    t = np.zeros((len(items), mb), np.uint32)
    for i, it in enumerate(items):
        r = list(it.read_blocks) or [0]
        t[i, :len(r)] = r
        t[i, len(r):] = r[-1]
    return t


class HipBackend:
    """Engine backend (forward_sample / release / copy_blocks) on one GPU."""

    def __init__(self, cfg: AttnModelConfig, weights: Dict[str, np.ndarray],
                 num_blocks: int, block_size: int, device: str = "cuda"):
        self.cfg = cfg
        self.config = SimpleNamespace(context_length=cfg.context_length)
        self.dev = torch.device(device)
        self.w = {k: torch.from_numpy(v).to(self.dev) for k, v in
                  weights.items()}
        # One fused QKV projection per layer (Q heads, then K, then V),
        # consumed in place by rvkv_attn_prep_qkv.
        for l in range(cfg.n_layers):
            self.w[f"wqkv{l}"] = torch.cat(
                [self.w[f"wq{l}"], self.w[f"wk{l}"], self.w[f"wv{l}"]],
                dim=1).contiguous()
            if cfg.qkv_bias:
                self.w[f"bqkv{l}"] = torch.cat(
                    [self.w[f"bq{l}"], self.w[f"bk{l}"], self.w[f"bv{l}"]])
        self.st = HipKvStorage(cfg.n_layers, num_blocks, block_size,
                               cfg.n_kv_heads, cfg.head_dim)
        self._L = _lib.load()
        self.last_logits = None
        self.forwards = 0
        self._plans = {}

    def _u32(self, a) -> torch.Tensor:
        arr = np.ascontiguousarray(np.asarray(a, np.uint32)).view(np.int32)
        return torch.from_numpy(arr.copy()).to(self.dev)

    def release(self, seq_id: int) -> None:
        pass  # the KV path keeps no per-sequence device state

    def copy_blocks(self, src, dst) -> None:
        self.st.copy_blocks(self._u32(src), self._u32(dst))

    def forward_sample(self, items, last_only: bool, samplers) -> List[int]:
        c, w, st = self.cfg, self.w, self.st
        H, KV, hd = c.n_heads, c.n_kv_heads, c.head_dim
        toks = np.concatenate([np.asarray(it.tokens, np.int64)
                               for it in items])
        pos = np.concatenate([it.position_offset + np.arange(len(it.tokens))
                              for it in items])
        slots = np.array([p for it in items for p in it.write_positions],
                         np.uint32).reshape(-1, 2)
        rows = len(toks)
        cos, sin = (torch.from_numpy(a).to(self.dev)
                    for a in rope_cos_sin(c.rope_theta, hd, pos))
        sb, so = self._u32(slots[:, 0]), self._u32(slots[:, 1])
        tables = self._u32(padded_tables(items))
        offs = self._u32([it.position_offset for it in items])
        reads = self._u32([it.read_num_tokens for it in items])
        x = w["embed"][torch.from_numpy(toks).to(self.dev)]
        scale = 1.0 / math.sqrt(hd)
        decode = not last_only and all(len(it.tokens) == 1 for it in items)
        if decode:
            # One decode plan per forward, shared by every layer (rvllm's
            # GatherPlan); kept per batch size and updated in place.
            lens = [it.read_num_tokens for it in items]
            plan = self._plans.get(len(items))
            if plan is None:
                plan = HipDecodePlan(st, lens, H, window=c.window)
                self._plans[len(items)] = plan
            else:
                plan.update(lens)
        for l in range(c.n_layers):
            qkv = x @ w[f"wqkv{l}"]
            qr = st.attn_prep_qkv(l, qkv, H, cos, sin, sb, so,
                                  bias=w.get(f"bqkv{l}"),
                                  q_norm=w.get(f"qn{l}"),
                                  k_norm=w.get(f"kn{l}"), eps=c.eps)
            if decode:
                att = st.paged_decode_planned(l, plan, qr, tables, reads,
                                              scale=scale)
            else:
                att = torch.empty_like(qr)
                r0 = 0
                for i, it in enumerate(items):  # one prefill item at a time
                    n = len(it.tokens)
                    st.paged_prefill(l, qr[r0:r0 + n].view(1, n, H, hd),
                                     tables[i:i + 1], offs[i:i + 1],
                                     reads[i:i + 1],
                                     out=att[r0:r0 + n].view(1, n, H, hd),
                                     scale=scale, window=c.window)
                    r0 += n
            x = x + att.view(rows, H * hd) @ w[f"wo{l}"]
        last = np.cumsum([len(it.tokens) for it in items]) - 1
        xs = x[torch.from_numpy(last).to(self.dev)]
        logits = (xs @ w["embed"].T) * logit_scale(c)
        logits = logits.contiguous()
        ids = torch.empty(len(items), dtype=torch.int32, device=self.dev)
        check(self._L.rvkv_argmax(ctypes.c_void_p(logits.data_ptr()),
                                  len(items), c.vocab,
                                  ctypes.c_void_p(ids.data_ptr()),
                                  ctypes.c_void_p(st.stream.cuda_stream)))
        self.last_logits = logits
        self.forwards += 1
        return ids.cpu().numpy().view(np.uint32).tolist()
