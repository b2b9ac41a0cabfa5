"""TEST INFRASTRUCTURE ONLY: numpy-facing wrapper of the CPU oracle.

The oracle (``rvkv_oracle.c``) restates rvllm's CPU KV path; only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg use it, always as the checker or the timed CPU baseline, never as the
product. Each wrapper names the reference function it restates.

Parity status of each function (how the oracle itself is pinned):
  * f32_to_f16 / f16_to_f32   - numpy float16 (library routine), closed form
                                special cases (tests/test_oracle.py)
  * write_tokens / gather     - reference KATs src/kv_storage.rs:193-255,
                                src/cuda/ops.rs:1070-1259 (tests/golden)
  * gather_plan               - src/kv_storage.rs:50-75 padding rule KAT
                                (src/cuda/ops.rs:1222-1226: [0,1,2,2])
  * batch_mask                - src/model.rs:1184-1197 KAT
  * gqa_attention             - src/model.rs:879-923 hand-computed KAT,
                                naive per-head + torch SDPA (CPU) cross-check
  * paged_decode_f64          - src/metal/ops.rs:676-766 cases, brute force
                                vs torch SDPA in float64
  * copy_blocks / checksums   - parity unpinned (no reference behaviour):
                                pinned by invariants (dst == src, others
                                untouched) and an independent numpy FNV-1a
  * decode_step               - composition of the pinned parts above
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_rvkv.so")
F16, F32 = 1, 2

_lib = None


def build() -> str:
    """Compiles the oracle with its Makefile (gcc); returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle_rvkv.so"],
                   check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        u32, i32, sz, f32, f64 = (ctypes.c_uint32, ctypes.c_int32,
                                  ctypes.c_size_t, ctypes.c_float,
                                  ctypes.c_double)
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [f32]
        L.orc_f16_to_f32.restype = f32
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16_array.argtypes = [P, P, sz]
        L.orc_f16_to_f32_array.argtypes = [P, P, sz]
        L.orc_write_tokens.restype = ctypes.c_int
        L.orc_write_tokens.argtypes = [P, P, ctypes.c_int, u32, u32, u32, u32,
                                       P, P, u32, P, P]
        L.orc_write_tokens_f16src.restype = ctypes.c_int
        L.orc_write_tokens_f16src.argtypes = [P, P, u32, u32, u32, u32, P, P,
                                              u32, P, P]
        L.orc_gather_plan.argtypes = [u32, P, P, P, P, P, P]
        L.orc_gather.argtypes = [P, ctypes.c_int, u32, u32, u32, u32, P, u32,
                                 u32, u32, P]
        L.orc_batch_mask.argtypes = [u32, P, P, u32, u32, i32, P]
        L.orc_gqa_attention.argtypes = [P, P, P, P, u32, u32, u32, u32, u32,
                                        u32, P]
        L.orc_paged_decode_f64.argtypes = [P, P, ctypes.c_int, u32, u32, u32,
                                           P, P, u32, P, u32, u32, f64, i32, P]
        L.orc_paged_prefill_f64.argtypes = [P, P, ctypes.c_int, u32, u32,
                                            u32, P, P, u32, P, P, u32, u32,
                                            u32, f64, i32, P]
        L.orc_copy_blocks.argtypes = [P, ctypes.c_int, u32, u32, u32, P, P,
                                      u32]
        L.orc_block_checksums.argtypes = [P, u32, u32, u32, P, u32, P]
        L.orc_decode_step.restype = ctypes.c_int
        L.orc_decode_step.argtypes = [P, P, ctypes.c_int, u32, u32, u32, u32,
                                      P, P, P, P, P, u32, P, u32, u32, P, P,
                                      u32]
        L.orc_rope_cos_sin.argtypes = [f32, P, u32, P, u32, P, P]
        L.orc_rms_norm.argtypes = [P, P, u32, u32, f32, P]
        L.orc_rope_apply.argtypes = [P, P, P, u32, u32, P]
        L.orc_attn_prep.restype = ctypes.c_int
        L.orc_attn_prep.argtypes = [P, P, P, u32, u32, u32, u32, P, P, P, P,
                                    P, f32, P, P, P, P, P, P, ctypes.c_int,
                                    u32, u32, P]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def f32_to_f16_bits(x) -> np.ndarray:
    """IEEE f32 -> f16 round-to-nearest-even, as uint16 bit patterns."""
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(np.asarray(h, dtype=np.uint16))
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


class KvCache:
    """One layer of rvllm's KvStorage (src/kv_storage.rs:9-13, 84-104):
    zeroed K and V of logical shape [num_blocks, block_size, n_kv, hd] with
    f32 cells (the reference's dtype) or f16 cells (uint16 bit patterns)."""

    def __init__(self, num_blocks, block_size, n_kv, hd, dtype=F16):
        self.num_blocks, self.bs, self.n_kv, self.hd = (num_blocks, block_size,
                                                        n_kv, hd)
        self.dtype = dtype
        shape = (num_blocks, block_size, n_kv, hd)
        np_dt = np.uint16 if dtype == F16 else np.float32
        self.k = np.zeros(shape, dtype=np_dt)
        self.v = np.zeros(shape, dtype=np_dt)

    def write_tokens(self, blocks, offsets, k, v) -> None:
        """KvStorage::write_tokens (src/kv_storage.rs:116-150); k, v f32
        [n_tokens, n_kv, hd]."""
        blocks, offsets = _u32(blocks), _u32(offsets)
        k, v = _f32(k), _f32(v)
        n = blocks.size
        assert k.shape == (n, self.n_kv, self.hd) and v.shape == k.shape
        rc = lib().orc_write_tokens(_p(self.k), _p(self.v), self.dtype,
                                    self.num_blocks, self.bs, self.n_kv,
                                    self.hd, _p(blocks), _p(offsets), n,
                                    _p(k), _p(v))
        if rc:
            raise ValueError("write_tokens: slot out of range")

    def write_tokens_f16(self, blocks, offsets, k_bits, v_bits) -> None:
        """f16-source append: bits copied unchanged."""
        assert self.dtype == F16
        blocks, offsets = _u32(blocks), _u32(offsets)
        k_bits = np.ascontiguousarray(k_bits, dtype=np.uint16)
        v_bits = np.ascontiguousarray(v_bits, dtype=np.uint16)
        rc = lib().orc_write_tokens_f16src(_p(self.k), _p(self.v),
                                           self.num_blocks, self.bs,
                                           self.n_kv, self.hd, _p(blocks),
                                           _p(offsets), blocks.size,
                                           _p(k_bits), _p(v_bits))
        if rc:
            raise ValueError("write_tokens: slot out of range")

    def gather(self, block_idx, batch, max_blocks, ctx_len):
        """KvStorage::gather (src/kv_storage.rs:157-173): f32 K and V of
        shape [batch, n_kv, ctx_len, hd] through the padded plan."""
        block_idx = _u32(block_idx)
        assert block_idx.size == batch * max_blocks
        outs = []
        for cache in (self.k, self.v):
            out = np.empty((batch, self.n_kv, ctx_len, self.hd), np.float32)
            lib().orc_gather(_p(cache), self.dtype, self.num_blocks, self.bs,
                             self.n_kv, self.hd, _p(block_idx), batch,
                             max_blocks, ctx_len, _p(out))
            outs.append(out)
        return outs[0], outs[1]

    def copy_blocks(self, src, dst) -> None:
        """CoW block copy (no reference counterpart; invariants only)."""
        src, dst = _u32(src), _u32(dst)
        for cache in (self.k, self.v):
            lib().orc_copy_blocks(_p(cache), self.dtype, self.bs, self.n_kv,
                                  self.hd, _p(src), _p(dst), src.size)

    def checksums(self, which: int, blocks) -> np.ndarray:
        """FNV-1a 64 of each block's logical little-endian bytes (an f32
        cell hashes as its two 16-bit halves, low first)."""
        blocks = _u32(blocks)
        out = np.empty(blocks.size, np.uint64)
        cache = (self.k if which == 0 else self.v).view(np.uint16)
        words = self.hd * (1 if self.dtype == F16 else 2)
        lib().orc_block_checksums(_p(cache), self.bs, self.n_kv, words,
                                  _p(blocks), blocks.size, _p(out))
        return out

    def as_f32(self, which: int) -> np.ndarray:
        cache = self.k if which == 0 else self.v
        return f16_bits_to_f32(cache) if self.dtype == F16 else cache.copy()


def gather_plan(tables, n_tokens):
    """GatherPlan::new (src/kv_storage.rs:50-75): (padded idx
    [batch*max_blocks], max_blocks, ctx_len)."""
    lens = _u32([len(t) for t in tables])
    flat = _u32(np.concatenate([np.asarray(t, np.uint32) for t in tables])
                if len(tables) and lens.sum() else np.zeros(0, np.uint32))
    n_tokens = _u32(n_tokens)
    mb, cl = ctypes.c_uint32(0), ctypes.c_uint32(0)
    L = lib()
    L.orc_gather_plan(len(tables), _p(lens), _p(flat), _p(n_tokens), None,
                      ctypes.byref(mb), ctypes.byref(cl))
    idx = np.zeros(len(tables) * mb.value, np.uint32)
    if idx.size:
        L.orc_gather_plan(len(tables), _p(lens), _p(flat), _p(n_tokens),
                          _p(idx), ctypes.byref(mb), ctypes.byref(cl))
    return idx, mb.value, cl.value


def batch_mask(position_offset, read_num_tokens, q_len, ctx_len, window=0):
    """batch_mask (src/model.rs:346-369): [batch, 1, q_len, ctx_len]."""
    po, rn = _u32(position_offset), _u32(read_num_tokens)
    batch = po.size
    m = np.empty((batch, 1, q_len, ctx_len), np.float32)
    lib().orc_batch_mask(batch, _p(po), _p(rn), q_len, ctx_len,
                         int(window or 0), _p(m))
    return m


def gqa_attention(q, k, v, mask):
    """gqa_attention (src/model.rs:377-415), f32."""
    q, k, v, mask = _f32(q), _f32(k), _f32(v), _f32(mask)
    batch, n_heads, q_len, hd = q.shape
    _, n_kv, ctx_len, _ = k.shape
    out = np.empty_like(q)
    lib().orc_gqa_attention(_p(q), _p(k), _p(v), _p(mask), batch, n_heads,
                            n_kv, q_len, ctx_len, hd, _p(out))
    return out


def paged_decode_f64(cache: KvCache, q, tables, max_blocks, ctx_lens,
                     scale=None, window=0):
    """Float64 decode attention straight over the paged cache
    (src/metal/ops.rs:719-745 restated for q_len 1). q [batch, n_heads,
    hd] f32 -> out f32."""
    q = _f32(q)
    batch, n_heads, hd = q.shape
    tables, ctx_lens = _u32(tables), _u32(ctx_lens)
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    out = np.empty_like(q)
    lib().orc_paged_decode_f64(_p(cache.k), _p(cache.v), cache.dtype,
                               cache.bs, cache.n_kv, cache.hd, _p(q),
                               _p(tables), max_blocks, _p(ctx_lens), batch,
                               n_heads, float(scale), int(window or 0),
                               _p(out))
    return out


def paged_prefill_f64(cache: KvCache, q, tables, max_blocks, pos_offset,
                      read_num, scale=None, window=0):
    """Float64 paged attention for q_len >= 1 rows per sequence with
    batch_mask's causal/window rule (src/model.rs:346-369; the Metal test
    reference src/metal/ops.rs:719-745). q [batch, q_len, n_heads, hd]
    token-major f32 -> out of the same shape."""
    q = _f32(q)
    batch, q_len, n_heads, hd = q.shape
    tables, pos_offset, read_num = _u32(tables), _u32(pos_offset), \
        _u32(read_num)
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    out = np.empty_like(q)
    lib().orc_paged_prefill_f64(_p(cache.k), _p(cache.v), cache.dtype,
                                cache.bs, cache.n_kv, cache.hd, _p(q),
                                _p(tables), max_blocks, _p(pos_offset),
                                _p(read_num), batch, q_len, n_heads,
                                float(scale), int(window or 0), _p(out))
    return out


def decode_step(cache: KvCache, slot_block, slot_off, new_k, new_v,
                block_idx, max_blocks, read_num_tokens, q, n_threads=1):
    """One decode step of one layer as rvllm's CPU path runs it
    (src/model.rs:628-644): append, padded gather, mask, gqa_attention.
    Mutates ``cache``; returns out [batch, n_heads, hd]."""
    q = _f32(q)
    batch, n_heads, hd = q.shape
    sb, so = _u32(slot_block), _u32(slot_off)
    nk, nv = _f32(new_k), _f32(new_v)
    bi, rn = _u32(block_idx), _u32(read_num_tokens)
    out = np.empty_like(q)
    rc = lib().orc_decode_step(_p(cache.k), _p(cache.v), cache.dtype,
                               cache.num_blocks,
                               cache.bs, cache.n_kv, cache.hd, _p(sb), _p(so),
                               _p(nk), _p(nv), _p(bi), max_blocks, _p(rn),
                               batch, n_heads, _p(q), _p(out), n_threads)
    if rc:
        raise ValueError("decode_step: slot out of range")
    return out


# ---- attention prep (bias, QK RMS norm, RoPE) + append ------
def rope_cos_sin(rope_theta, head_dim, positions, factors=None):
    """rope_cos_sin (src/model.rs:224-250): f32 cos, sin [n, hd/2]."""
    pos = _u32(positions)
    half = head_dim // 2
    c = np.empty((pos.size, half), np.float32)
    s = np.empty((pos.size, half), np.float32)
    fac = _f32(factors) if factors is not None else None
    lib().orc_rope_cos_sin(float(rope_theta), _p(fac) if fac is not None
                           else None, head_dim, _p(pos), pos.size, _p(c),
                           _p(s))
    return c, s


def rms_norm(x, w, eps):
    """rms_norm over the last dim (src/model.rs:200-215)."""
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    dim = x.shape[-1]
    lib().orc_rms_norm(_p(x), _p(w), x.size // dim, dim, float(eps), _p(out))
    return out


def rope_apply(x, cos, sin):
    """rope_apply, rotate-half (src/model.rs:252-264); x [rows, hd]."""
    x, cos, sin = _f32(x), _f32(cos), _f32(sin)
    out = np.empty_like(x)
    lib().orc_rope_apply(_p(x), _p(cos), _p(sin), x.shape[0], x.shape[1],
                         _p(out))
    return out


def attn_prep(cache: KvCache, q_in, k_in, v_in, cos, sin, slot_block,
              slot_off, q_bias=None, k_bias=None, v_bias=None, q_norm=None,
              k_norm=None, eps=1e-6):
    """The prep segment of Attention::forward (src/model.rs:600-626) plus
    write_tokens: returns q_out, mutates the cache (f16 or f32 cells)."""
    q_in, k_in, v_in = _f32(q_in), _f32(k_in), _f32(v_in)
    rows, n_heads, hd = q_in.shape
    n_kv = k_in.shape[1]
    opt = [None if a is None else _f32(a) for a in
           (q_bias, k_bias, v_bias, q_norm, k_norm)]
    cos, sin = _f32(cos), _f32(sin)
    sb, so = _u32(slot_block), _u32(slot_off)
    q_out = np.empty_like(q_in)
    rc = lib().orc_attn_prep(
        _p(q_in), _p(k_in), _p(v_in), rows, n_heads, n_kv, hd,
        *[None if a is None else _p(a) for a in opt], float(eps), _p(cos),
        _p(sin), _p(sb), _p(so), _p(cache.k), _p(cache.v), cache.dtype,
        cache.num_blocks,
        cache.bs, _p(q_out))
    if rc:
        raise ValueError("attn_prep: slot out of range")
    return q_out


def argmax_rows(logits) -> np.ndarray:
    """Greedy token per row as Sampler::sample_slice scans it
    (src/sampler.rs:64-75): first maximum wins, NaN is never a maximum, a
    row with nothing above -inf gives 0 (numpy's argmax returns the first
    occurrence, and index 0 for an all -inf row)."""
    x = np.asarray(logits, np.float32)
    x = np.where(np.isnan(x), -np.inf, x)
    return np.argmax(x, axis=-1).astype(np.uint32)
