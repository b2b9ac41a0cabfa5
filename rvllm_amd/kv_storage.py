"""Host-side mirror of rvllm's device KV storage API over librvkv.so.

``HipKvStorage`` / ``HipGatherPlan`` keep the names, argument meaning and
error strings of ``CudaKvStorage`` / ``CudaGatherPlan``
(src/cuda/kv_storage.rs:17-164) and of the validating wrappers
``kv_write_wrapper`` / ``kv_gather_wrapper`` (src/cuda/ops.rs:313-445), and
add the fused paged decode attention and the copy-on-write block copy. Device
buffers are torch tensors on the GPU, used only as memory: every byte of
work runs in the HIP kernels of librvkv.so. Length checks the C ABI cannot
see (it gets raw pointers) are done here, before the call, with the
reference's messages.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import RVKV_F16, RVKV_F32, RvkvError, check

_DT = {torch.float32: RVKV_F32, torch.float16: RVKV_F16}


def _ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise RvkvError(msg)


def _dev_u32(x, device) -> torch.Tensor:
    """u32 data as an int32 device tensor (same bits)."""
    if isinstance(x, torch.Tensor):
        t = x.to(device=device)
        if t.dtype != torch.int32:
            t = t.to(torch.int64).to(torch.int32)
        return t.contiguous()
    import numpy as np
    arr = np.asarray(x, dtype=np.uint32).view(np.int32)
    return torch.from_numpy(arr.copy()).to(device)


class HipGatherPlan:
    """CudaGatherPlan::new (src/cuda/kv_storage.rs:26-54): each sequence's
    block table padded to max_blocks with its own last block, uploaded once
    per forward and shared by all layers. items: [(blocks, n_tokens)]."""

    def __init__(self, items: Sequence[Tuple[Sequence[int], int]], device=None):
        device = device or torch.device("cuda", torch.cuda.current_device())
        self.batch = len(items)
        self.ctx_len = max((n for _, n in items), default=0)
        self.max_blocks = max((len(b) for b, _ in items), default=0)
        idx = []
        for blocks, _ in items:
            blocks = [int(x) for x in blocks]
            pad = blocks[-1] if blocks else 0
            idx.extend(blocks + [pad] * (self.max_blocks - len(blocks)))
        self.block_idx = _dev_u32(idx, device)


class HipDecodePlan:
    """Per-forward decode plan (rvkv_decode_plan_create): built from the
    host-side context lengths (rvllm's read_num_tokens) and shared by every
    layer's paged_decode_planned, like GatherPlan (src/kv_storage.rs:50-75).
    """

    def __init__(self, store: "HipKvStorage", ctx_lens, n_heads: int,
                 window: int = 0):
        import numpy as np
        self._L = store._L
        lens = np.ascontiguousarray(np.asarray(ctx_lens, dtype=np.uint32))
        self.batch = int(lens.size)
        self.n_heads = n_heads
        self.window = int(window or 0)
        self.ctx_lens_host = lens
        handle = ctypes.c_void_p()
        check(self._L.rvkv_decode_plan_create(
            store._pool, lens.ctypes.data_as(ctypes.c_void_p), self.batch,
            n_heads, self.window, ctypes.byref(handle)))
        self._plan = handle
        # The native plan reaches its pool's stream when destroyed, so the
        # pool must outlive it: hold the storage.
        self._store = store
        self._device = store.device
        self.ws = None
        self._sync()

    def _sync(self) -> None:
        self.workspace_bytes = self._L.rvkv_decode_plan_workspace_bytes(
            self._plan)
        self.items = self._L.rvkv_decode_plan_items(self._plan)
        have = self.ws.numel() if self.ws is not None else 0
        if self.workspace_bytes > have:
            self.ws = torch.empty(self.workspace_bytes + (1 << 20),
                                  dtype=torch.uint8, device=self._device)

    def update(self, ctx_lens, tables=None) -> None:
        """rvkv_decode_plan_update: this step's context lengths; with the
        host copy of the padded block tables ([batch, max_blocks]), items
        of sequences sharing prefix blocks are ordered back to back
        (rvkv_decode_plan_update_tables)."""
        import numpy as np
        lens = np.ascontiguousarray(np.asarray(ctx_lens, dtype=np.uint32))
        if tables is None:
            check(self._L.rvkv_decode_plan_update(
                self._plan, lens.ctypes.data_as(ctypes.c_void_p), lens.size))
        else:
            tab = np.ascontiguousarray(np.asarray(tables, dtype=np.uint32))
            _need(tab.ndim == 2 and tab.shape[0] == lens.size,
                  "decode_plan: tables must be [batch, max_blocks]")
            check(self._L.rvkv_decode_plan_update_tables(
                self._plan, lens.ctypes.data_as(ctypes.c_void_p),
                tab.ctypes.data_as(ctypes.c_void_p), tab.shape[1],
                lens.size))
        self.batch = int(lens.size)
        self.ctx_lens_host = lens
        self._sync()

    def close(self) -> None:
        if getattr(self, "_plan", None):
            self._L.rvkv_decode_plan_destroy(self._plan)
            self._plan = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipKvStorage:
    """CudaKvStorage (src/cuda/kv_storage.rs:65-164) on MI355X: one zeroed
    pool for all layers' K and V, owned by librvkv. Cells are f16 (the
    default) or, with dtype=torch.float32, f32 like rvllm's own cache (every
    operation). On an f32 pool, decode at head_dim 32/64/128/256 with
    power-of-two blocks runs the tuned decode_f32_kernel (split partials and
    a reduction, as on f16); prefill, attn_prep and decode at other shapes
    run the generic kernels."""

    def __init__(self, n_layers: int, num_blocks: int, block_size: int,
                 n_kv_heads: int, head_dim: int, stream=None,
                 dtype: torch.dtype = torch.float16):
        self._L = _lib.load()
        self.n_layers, self.num_blocks = n_layers, num_blocks
        self.block_size, self.n_kv_heads, self.head_dim = (block_size,
                                                           n_kv_heads,
                                                           head_dim)
        self.device = torch.device("cuda", torch.cuda.current_device())
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        self.stream = stream
        _need(dtype in _DT, "pool_create: cache dtype must be float16 or "
              "float32")
        self.dtype = dtype
        handle = ctypes.c_void_p()
        check(self._L.rvkv_pool_create(n_layers, num_blocks, block_size,
                                       n_kv_heads, head_dim, _DT[dtype],
                                       ctypes.c_void_p(stream.cuda_stream),
                                       ctypes.byref(handle)))
        self._pool = handle

    # -- lifetime ---------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_pool", None):
            self._L.rvkv_pool_destroy(self._pool)
            self._pool = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream) -> None:
        """Rebinds the pool to another stream (e.g. a graph-capture stream);
        later calls enqueue there."""
        check(self._L.rvkv_pool_set_stream(
            self._pool, ctypes.c_void_p(stream.cuda_stream)))
        self.stream = stream

    @property
    def nbytes(self) -> int:
        return self._L.rvkv_pool_bytes(self._pool)

    # -- append ---------------------------------------------------------
    def write_tokens(self, layer: int, block_ids: torch.Tensor,
                     offsets: torch.Tensor, k: torch.Tensor,
                     v: torch.Tensor) -> None:
        """CudaKvStorage::write_tokens -> kv_write_wrapper
        (src/cuda/ops.rs:313-373). k, v: [n_tokens, n_kv, hd] f32 (rounded
        to f16, nearest-even) or f16 (copied); block_ids/offsets: one u32
        per token (int32 device tensors carrying the same bits)."""
        _need(k.numel() == v.numel(), "kv_write: k and v have different lengths")
        n = k.numel()
        _need(n != 0, "kv_write: k/v len is 0")
        per_token = self.n_kv_heads * self.head_dim
        _need(n % per_token == 0,
              "kv_write: k/v length is not a multiple of n_kv_heads * head_dim")
        n_tokens = n // per_token
        _need(block_ids.numel() == n_tokens and offsets.numel() == n_tokens,
              "kv_write: block_ids/offsets length must equal n_tokens")
        _need(k.dtype == v.dtype and k.dtype in _DT,
              "kv_write: k/v must both be float32 or float16")
        _need(k.is_contiguous() and v.is_contiguous() and
              block_ids.is_contiguous() and offsets.is_contiguous(),
              "kv_write: inputs must be contiguous")
        check(self._L.rvkv_append(self._pool, layer, _ptr(k), _ptr(v),
                                  _DT[k.dtype], _ptr(block_ids),
                                  _ptr(offsets), n_tokens))

    def write_tokens_layers(self, layer0: int, block_ids: torch.Tensor,
                            offsets: torch.Tensor, k: torch.Tensor,
                            v: torch.Tensor) -> None:
        """write_tokens for layers layer0 .. layer0 + k.shape[0] - 1 with one
        slot list, in one launch (rvkv_append_layers). k, v:
        [n_layers, n_tokens, n_kv, hd] f32 or f16."""
        _need(k.shape == v.shape and k.dim() == 4,
              "kv_write: k/v must be [n_layers, n_tokens, n_kv_heads, "
              "head_dim] of one shape")
        n_layers, n_tokens = int(k.shape[0]), int(k.shape[1])
        _need(n_tokens != 0 and n_layers != 0, "kv_write: k/v len is 0")
        _need(tuple(k.shape[2:]) == (self.n_kv_heads, self.head_dim),
              "kv_write: k/v rows must be [n_kv_heads, head_dim]")
        _need(block_ids.numel() == n_tokens and offsets.numel() == n_tokens,
              "kv_write: block_ids/offsets length must equal n_tokens")
        _need(k.dtype == v.dtype and k.dtype in _DT,
              "kv_write: k/v must both be float32 or float16")
        _need(k.is_contiguous() and v.is_contiguous() and
              block_ids.is_contiguous() and offsets.is_contiguous(),
              "kv_write: inputs must be contiguous")
        check(self._L.rvkv_append_layers(
            self._pool, layer0, n_layers, _ptr(k), _ptr(v), _DT[k.dtype],
            n_tokens * self.n_kv_heads * self.head_dim, _ptr(block_ids),
            _ptr(offsets), n_tokens))

    # -- gather ---------------------------------------------------------
    def gather(self, layer: int, plan: HipGatherPlan, out_k: torch.Tensor,
               out_v: torch.Tensor) -> None:
        """CudaKvStorage::gather -> kv_gather_wrapper
        (src/cuda/ops.rs:381-445): [batch, n_kv, ctx_len, hd] into
        caller-owned outputs (f32, or f16 for raw bits)."""
        _need(plan.batch > 0 and plan.max_blocks > 0 and plan.ctx_len > 0,
              "kv_gather: batch/max_blocks/ctx_len/block_size/n_kv_heads/"
              "head_dim must be positive")
        _need(plan.block_idx.numel() == plan.batch * plan.max_blocks,
              "kv_gather: block_idx length must equal batch * max_blocks")
        n = plan.batch * self.n_kv_heads * plan.ctx_len * self.head_dim
        _need(out_k.numel() == n and out_v.numel() == n,
              "kv_gather: output length must equal batch * n_kv_heads * "
              "ctx_len * head_dim")
        _need(plan.ctx_len <= plan.max_blocks * self.block_size,
              "kv_gather: ctx_len must not exceed max_blocks * block_size")
        _need(out_k.dtype == out_v.dtype and out_k.dtype in _DT,
              "kv_gather: outputs must both be float32 or float16")
        check(self._L.rvkv_gather(self._pool, layer, _ptr(plan.block_idx),
                                  plan.batch, plan.max_blocks, plan.ctx_len,
                                  _ptr(out_k), _ptr(out_v), _DT[out_k.dtype]))

    # -- paged decode attention -----------------------------------
    def decode_workspace_bytes(self, batch: int, n_heads: int,
                               max_ctx_len: int) -> int:
        return self._L.rvkv_decode_workspace_bytes(self._pool, batch, n_heads,
                                                   max_ctx_len)

    def decode_partition_tokens(self, batch: int, n_heads: int,
                                max_ctx_len: int) -> int:
        return self._L.rvkv_decode_partition_tokens(self._pool, batch,
                                                    n_heads, max_ctx_len)

    def alloc_workspace(self, batch: int, n_heads: int,
                        max_ctx_len: int) -> torch.Tensor:
        nbytes = self.decode_workspace_bytes(batch, n_heads, max_ctx_len)
        return torch.empty(max(nbytes, 256), dtype=torch.uint8,
                           device=self.device)

    def paged_decode(self, layer: int, q: torch.Tensor,
                     block_tables: torch.Tensor, ctx_lens: torch.Tensor,
                     max_ctx_len: int, out: Optional[torch.Tensor] = None,
                     ws: Optional[torch.Tensor] = None,
                     scale: Optional[float] = None,
                     window: int = 0) -> torch.Tensor:
        """One decode step of attention for every sequence (q_len 1), read
        straight through the block tables: the fused replacement of
        kv_gather + attention_scores + mask_add_broadcast + softmax +
        attention_apply (src/cuda/model.rs:528-569). q: [batch, n_heads,
        hd] f32; block_tables: [batch, max_blocks] u32; ctx_lens: [batch]
        u32 (read_num_tokens, including this step's token)."""
        _need(q.dim() == 3 and q.shape[2] == self.head_dim,
              "paged_decode: q must be [batch, n_heads, head_dim]")
        _need(q.dtype == torch.float32 and q.is_contiguous(),
              "paged_decode: q must be contiguous float32")
        batch, n_heads, hd = q.shape
        _need(block_tables.dim() == 2 and block_tables.shape[0] == batch,
              "paged_decode: block_tables must be [batch, max_blocks]")
        _need(ctx_lens.numel() == batch,
              "paged_decode: ctx_lens length must equal batch")
        max_blocks = block_tables.shape[1]
        if out is None:
            out = torch.empty_like(q)
        _need(out.shape == q.shape and out.dtype == torch.float32 and
              out.is_contiguous(), "paged_decode: out must match q")
        need = self.decode_workspace_bytes(batch, n_heads, max_ctx_len)
        if ws is None and need:
            ws = self.alloc_workspace(batch, n_heads, max_ctx_len)
        if scale is None:
            scale = 1.0 / math.sqrt(hd)
        check(self._L.rvkv_paged_decode(
            self._pool, layer, _ptr(q), _ptr(block_tables), _ptr(ctx_lens),
            batch, max_blocks, n_heads, max_ctx_len, float(scale),
            int(window or 0), _ptr(out), _ptr(ws),
            ws.numel() if ws is not None else 0))
        return out

    def paged_prefill(self, layer: int, q: torch.Tensor,
                      block_tables: torch.Tensor, pos_offset: torch.Tensor,
                      read_num_tokens: torch.Tensor,
                      out: Optional[torch.Tensor] = None,
                      scale: Optional[float] = None,
                      window: int = 0) -> torch.Tensor:
        """Prefill / chunked-prefill attention (q_len >= 1 rows per
        sequence, batch_mask's causal and window rule) straight over the
        paged cache: the replacement of kv_gather + batch_mask +
        gqa_attention (src/model.rs:346-415, 628-644). q: [batch, q_len,
        n_heads, hd] f32 token-major; block_tables [batch, max_blocks],
        pos_offset and read_num_tokens [batch] u32."""
        _need(q.dim() == 4 and q.shape[3] == self.head_dim,
              "paged_prefill: q must be [batch, q_len, n_heads, head_dim]")
        _need(q.dtype == torch.float32 and q.is_contiguous(),
              "paged_prefill: q must be contiguous float32")
        batch, q_len, n_heads, hd = q.shape
        _need(block_tables.dim() == 2 and block_tables.shape[0] == batch,
              "paged_prefill: block_tables must be [batch, max_blocks]")
        _need(pos_offset.numel() == batch and read_num_tokens.numel() == batch,
              "paged_prefill: pos_offset/read_num_tokens length must equal "
              "batch")
        if out is None:
            out = torch.empty_like(q)
        _need(out.shape == q.shape and out.dtype == torch.float32 and
              out.is_contiguous(), "paged_prefill: out must match q")
        if scale is None:
            scale = 1.0 / math.sqrt(hd)
        check(self._L.rvkv_paged_prefill(
            self._pool, layer, _ptr(q), _ptr(block_tables), _ptr(pos_offset),
            _ptr(read_num_tokens), batch, q_len, block_tables.shape[1],
            n_heads, float(scale), int(window or 0), _ptr(out)))
        return out

    def paged_decode_planned(self, layer: int, plan: HipDecodePlan,
                             q: torch.Tensor, block_tables: torch.Tensor,
                             ctx_lens: torch.Tensor,
                             out: Optional[torch.Tensor] = None,
                             scale: Optional[float] = None) -> torch.Tensor:
        """paged_decode driven by a per-forward HipDecodePlan (ragged
        batches): same inputs and result."""
        _need(q.dim() == 3 and q.shape[0] == plan.batch and
              q.shape[1] == plan.n_heads and q.shape[2] == self.head_dim,
              "paged_decode: q must be [batch, n_heads, head_dim] of the plan")
        _need(q.dtype == torch.float32 and q.is_contiguous(),
              "paged_decode: q must be contiguous float32")
        _need(block_tables.dim() == 2 and block_tables.shape[0] == plan.batch,
              "paged_decode: block_tables must be [batch, max_blocks]")
        _need(ctx_lens.numel() == plan.batch,
              "paged_decode: ctx_lens length must equal batch")
        if out is None:
            out = torch.empty_like(q)
        _need(out.shape == q.shape and out.dtype == torch.float32 and
              out.is_contiguous(), "paged_decode: out must match q")
        if scale is None:
            scale = 1.0 / math.sqrt(self.head_dim)
        ws = plan.ws
        check(self._L.rvkv_paged_decode_planned(
            self._pool, plan._plan, layer, _ptr(q), _ptr(block_tables),
            _ptr(ctx_lens), block_tables.shape[1], float(scale), _ptr(out),
            _ptr(ws), ws.numel() if ws is not None else 0))
        return out

    def decode_step(self, layer: int, k: torch.Tensor, v: torch.Tensor,
                    slot_block: torch.Tensor, slot_off: torch.Tensor,
                    q: torch.Tensor, block_tables: torch.Tensor,
                    ctx_lens: torch.Tensor, max_ctx_len: int = 0,
                    plan: Optional[HipDecodePlan] = None,
                    out: Optional[torch.Tensor] = None,
                    ws: Optional[torch.Tensor] = None,
                    scale: Optional[float] = None,
                    window: int = 0) -> torch.Tensor:
        """One layer of a decode step in one launch (rvkv_decode_step):
        append each sequence's new K/V row (k, v: [batch, n_kv, hd]) at its
        slot, then attend over ctx_lens keys including it. Equivalent to
        write_tokens + paged_decode(_planned)."""
        _need(q.dim() == 3 and q.shape[2] == self.head_dim and
              q.dtype == torch.float32 and q.is_contiguous(),
              "decode_step: q must be contiguous float32 [batch, n_heads, "
              "head_dim]")
        batch, n_heads, hd = q.shape
        _need(k.shape == (batch, self.n_kv_heads, hd) and v.shape == k.shape
              and k.dtype == v.dtype and k.dtype in _DT and
              k.is_contiguous() and v.is_contiguous(),
              "decode_step: k/v must be contiguous [batch, n_kv_heads, "
              "head_dim] float32 or float16")
        _need(slot_block.numel() == batch and slot_off.numel() == batch,
              "decode_step: block_ids/offsets length must equal batch")
        _need(block_tables.dim() == 2 and block_tables.shape[0] == batch and
              ctx_lens.numel() == batch,
              "decode_step: block_tables/ctx_lens must have batch rows")
        if out is None:
            out = torch.empty_like(q)
        if scale is None:
            scale = 1.0 / math.sqrt(hd)
        if plan is not None:
            ws = plan.ws
            window = plan.window
        elif ws is None:
            need = self.decode_workspace_bytes(batch, n_heads, max_ctx_len)
            if need:
                ws = self.alloc_workspace(batch, n_heads, max_ctx_len)
        check(self._L.rvkv_decode_step(
            self._pool, plan._plan if plan is not None else None, layer,
            _ptr(k), _ptr(v), _DT[k.dtype], _ptr(slot_block), _ptr(slot_off),
            _ptr(q), _ptr(block_tables), _ptr(ctx_lens), batch,
            block_tables.shape[1], n_heads, max_ctx_len, float(scale),
            int(window or 0), _ptr(out), _ptr(ws),
            ws.numel() if ws is not None else 0))
        return out

    # -- attention prep + append ------------------------------------
    def attn_prep(self, layer: int, q_in: torch.Tensor, k_in: torch.Tensor,
                  v_in: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                  slot_block: torch.Tensor, slot_off: torch.Tensor,
                  q_bias=None, k_bias=None, v_bias=None, q_norm=None,
                  k_norm=None, eps: float = 1e-6,
                  q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """rvkv_attn_prep: bias, per-head RMS norm and RoPE for q and k
        (src/model.rs:600-626), q returned, k/v appended at their slots."""
        rows, n_heads, hd = q_in.shape
        _need(hd == self.head_dim and k_in.shape == (rows, self.n_kv_heads,
                                                      hd)
              and v_in.shape == k_in.shape,
              "attn_prep: q/k/v must be [rows, heads, head_dim]")
        for t in (q_in, k_in, v_in, cos, sin, q_bias, k_bias, v_bias, q_norm,
                  k_norm):
            _need(t is None or (t.dtype == torch.float32 and
                                t.is_contiguous()),
                  "attn_prep: float tensors must be contiguous float32")
        _need(cos.shape == (rows, hd // 2) and sin.shape == cos.shape,
              "attn_prep: cos/sin must be [rows, head_dim / 2]")
        _need(slot_block.numel() == rows and slot_off.numel() == rows,
              "attn_prep: block_ids/offsets length must equal rows")
        if q_out is None:
            q_out = torch.empty_like(q_in)
        check(self._L.rvkv_attn_prep(
            self._pool, layer, _ptr(q_in), _ptr(k_in), _ptr(v_in), rows,
            n_heads, _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(q_norm),
            _ptr(k_norm), float(eps), _ptr(cos), _ptr(sin), _ptr(slot_block),
            _ptr(slot_off), _ptr(q_out)))
        return q_out

    def attn_prep_qkv(self, layer: int, qkv: torch.Tensor, n_heads: int,
                      cos: torch.Tensor, sin: torch.Tensor,
                      block_ids: torch.Tensor, offsets: torch.Tensor,
                      bias=None, q_norm=None, k_norm=None, eps: float = 1e-5,
                      q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """rvkv_attn_prep_qkv: attn_prep over one fused QKV buffer [rows,
        (n_heads + 2 n_kv) * hd] with a fused bias, as the reference's
        fused attn_prep takes them (src/metal/ops.rs:357-420); returns q
        [rows, n_heads, hd]."""
        hd, kv = self.head_dim, self.n_kv_heads
        width = (n_heads + 2 * kv) * hd
        _need(qkv.dim() == 2 and qkv.shape[1] == width,
              "attn_prep: qkv length is not a multiple of the QKV width")
        rows = qkv.shape[0]
        for t in (qkv, cos, sin, bias, q_norm, k_norm):
            _need(t is None or (t.dtype == torch.float32 and
                                t.is_contiguous()),
                  "attn_prep: float tensors must be contiguous float32")
        _need(bias is None or bias.numel() == width,
              "attn_prep: bias must be [QKV width]")
        _need(cos.shape == (rows, hd // 2) and sin.shape == cos.shape,
              "attn_prep: cos/sin must be [rows, head_dim / 2]")
        _need(block_ids.numel() == rows and offsets.numel() == rows,
              "attn_prep: block_ids/offsets must hold one entry per row")
        if q_out is None:
            q_out = torch.empty((rows, n_heads, hd), dtype=torch.float32,
                                device=qkv.device)
        check(self._L.rvkv_attn_prep_qkv(
            self._pool, layer, _ptr(qkv), rows, n_heads, _ptr(bias),
            _ptr(q_norm), _ptr(k_norm), float(eps), _ptr(cos), _ptr(sin),
            _ptr(block_ids), _ptr(offsets), _ptr(q_out)))
        return q_out

    # -- copy-on-write -------------------------------------------------
    def copy_blocks(self, src: torch.Tensor, dst: torch.Tensor) -> None:
        """Copies src[i] -> dst[i] for all layers, K and V."""
        _need(src.numel() == dst.numel(),
              "copy_blocks: src and dst have different lengths")
        check(self._L.rvkv_copy_blocks(self._pool, _ptr(src), _ptr(dst),
                                       src.numel()))

    # -- inspection ---------------------------------------------------------
    def read_blocks(self, layer: int, which: int,
                    block_ids: torch.Tensor) -> torch.Tensor:
        """Logical [n, block_size, n_kv, hd] contents of the blocks, in the
        cache's dtype."""
        n = block_ids.numel()
        out = torch.empty((n, self.block_size, self.n_kv_heads,
                           self.head_dim), dtype=self.dtype,
                          device=self.device)
        check(self._L.rvkv_read_blocks(self._pool, layer, which,
                                       _ptr(block_ids), n, _ptr(out)))
        return out

    def block_checksums(self, layer: int, which: int,
                        block_ids: torch.Tensor) -> torch.Tensor:
        """FNV-1a 64 of each block's logical little-endian bytes (int64
        bits)."""
        n = block_ids.numel()
        out = torch.empty(n, dtype=torch.int64, device=self.device)
        check(self._L.rvkv_block_checksums(self._pool, layer, which,
                                           _ptr(block_ids), n, _ptr(out)))
        return out
