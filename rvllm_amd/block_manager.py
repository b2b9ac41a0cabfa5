"""Python handle on the native block manager (rvkv_bm_* in include/rvkv.h).

The block manager is host C++ (csrc/block_manager.cpp); this wrapper only
marshals arguments. It restates the parts of the external kv-cache-scheduler
crate that rvllm's engine relies on (src/engine.rs:351-539): pool
availability, per-sequence block tables, logical_to_physical slot mapping,
prefix sharing with refcounts, and the copy-on-write decision on append.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Tuple

from . import _lib
from ._lib import RvkvError

_U32_MAX = 0xFFFFFFFF


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        self._L = _lib.load()
        self._h = self._L.rvkv_bm_create(num_blocks, block_size)
        if not self._h:
            raise RvkvError("block_manager: num_blocks/block_size must be "
                            "positive")
        self.num_blocks, self.block_size = num_blocks, block_size

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.rvkv_bm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def available(self) -> int:
        """Free blocks (kv-cache-scheduler's pool.available())."""
        return self._L.rvkv_bm_available(self._h)

    def shuffle_free(self, seed: int) -> None:
        self._L.rvkv_bm_shuffle_free(self._h, seed & (2**64 - 1))

    def add_seq(self, n_tokens: int) -> int:
        sid = self._L.rvkv_bm_add_seq(self._h, n_tokens)
        if sid < 0:
            raise RvkvError("block_manager: pool full", int(sid))
        return sid

    def fork_seq(self, parent: int, n_shared: int, n_tokens: int) -> int:
        sid = self._L.rvkv_bm_fork_seq(self._h, parent, n_shared, n_tokens)
        if sid < 0:
            raise RvkvError("block_manager: cannot fork "
                            f"(parent {parent}, shared {n_shared}, "
                            f"tokens {n_tokens})", int(sid))
        return sid

    def free_seq(self, seq: int) -> None:
        if self._L.rvkv_bm_free_seq(self._h, seq) != 0:
            raise RvkvError(f"block_manager: unknown sequence {seq}")

    def append_slot(self, seq: int) -> Tuple[int, int, Optional[Tuple[int, int]]]:
        """Reserves the next token's slot: (block, offset, cow) where cow is
        (src, dst) when a shared block had to be copied first."""
        blk, off, cs, cd = (ctypes.c_uint32() for _ in range(4))
        rc = self._L.rvkv_bm_append_slot(self._h, seq, ctypes.byref(blk),
                                         ctypes.byref(off), ctypes.byref(cs),
                                         ctypes.byref(cd))
        if rc != 0:
            raise RvkvError(f"block_manager: append to {seq} failed", rc)
        cow = None if cs.value == _U32_MAX else (cs.value, cd.value)
        return blk.value, off.value, cow

    def free_seqs(self, seqs) -> None:
        import numpy as np
        seqs = np.ascontiguousarray(np.asarray(seqs, dtype=np.int64))
        rc = self._L.rvkv_bm_free_seqs(
            self._h, seqs.ctypes.data_as(ctypes.c_void_p), seqs.size)
        if rc != 0:
            raise RvkvError("block_manager: free_seqs: unknown sequence", rc)

    def add_seqs(self, n_tokens):
        """New sequences holding n_tokens[i] tokens each (all or none)."""
        import numpy as np
        n_tokens = np.ascontiguousarray(np.asarray(n_tokens, dtype=np.uint32))
        ids = np.empty(n_tokens.size, np.int64)
        rc = self._L.rvkv_bm_add_seqs(
            self._h, n_tokens.ctypes.data_as(ctypes.c_void_p), n_tokens.size,
            ids.ctypes.data_as(ctypes.c_void_p))
        if rc != 0:
            raise RvkvError("block_manager: pool full", rc)
        return ids

    def append_slots(self, seqs):
        """Slots of one decode step for every sequence in `seqs` (in order):
        (blocks u32[n], offsets u32[n], cow_src u32[k], cow_dst u32[k])."""
        import numpy as np
        seqs = np.ascontiguousarray(np.asarray(seqs, dtype=np.int64))
        n = seqs.size
        blocks = np.empty(n, np.uint32)
        offs = np.empty(n, np.uint32)
        cs = np.empty(max(n, 1), np.uint32)
        cd = np.empty(max(n, 1), np.uint32)
        k = ctypes.c_uint32()
        P = ctypes.c_void_p
        rc = self._L.rvkv_bm_append_slots(
            self._h, seqs.ctypes.data_as(P), n, blocks.ctypes.data_as(P),
            offs.ctypes.data_as(P), cs.ctypes.data_as(P),
            cd.ctypes.data_as(P), ctypes.byref(k))
        if rc != 0:
            raise RvkvError("block_manager: append_slots failed "
                            f"after {k.value} copies", rc)
        return blocks, offs, cs[:k.value].copy(), cd[:k.value].copy()

    def fill_tables(self, seqs, max_blocks: int, out=None, lens_out=None):
        """Padded block tables [n, max_blocks] and token counts of `seqs`."""
        import numpy as np
        seqs = np.ascontiguousarray(np.asarray(seqs, dtype=np.int64))
        n = seqs.size
        tables = out if out is not None else np.empty((n, max_blocks),
                                                      np.uint32)
        lens = lens_out if lens_out is not None else np.empty(n, np.uint32)
        assert tables.shape == (n, max_blocks) and tables.dtype == np.uint32
        P = ctypes.c_void_p
        rc = self._L.rvkv_bm_fill_tables(
            self._h, seqs.ctypes.data_as(P), n, max_blocks,
            tables.ctypes.data_as(P), lens.ctypes.data_as(P))
        if rc != 0:
            raise RvkvError("block_manager: fill_tables failed (unknown "
                            "sequence or table longer than max_blocks)", rc)
        return tables, lens

    def slot(self, seq: int, pos: int) -> Tuple[int, int]:
        """logical_to_physical(pos)."""
        blk, off = ctypes.c_uint32(), ctypes.c_uint32()
        rc = self._L.rvkv_bm_slot(self._h, seq, pos, ctypes.byref(blk),
                                  ctypes.byref(off))
        if rc != 0:
            raise RvkvError(f"block_manager: no slot {pos} in {seq}", rc)
        return blk.value, off.value

    def num_tokens(self, seq: int) -> int:
        return self._L.rvkv_bm_num_tokens(self._h, seq)

    def num_blocks_of(self, seq: int) -> int:
        return self._L.rvkv_bm_num_blocks(self._h, seq)

    def refcount(self, block: int) -> int:
        return self._L.rvkv_bm_refcount(self._h, block)

    def table(self, seq: int) -> List[int]:
        n = self._L.rvkv_bm_table(self._h, seq, None, 0)
        if n < 0:
            raise RvkvError(f"block_manager: unknown sequence {seq}")
        buf = (ctypes.c_uint32 * max(n, 1))()
        self._L.rvkv_bm_table(self._h, seq, buf, n)
        return list(buf[:n])
