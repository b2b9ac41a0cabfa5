"""Python handle on the native continuous-batching scheduler (rvkv_sched_*
in include/rvkv.h, csrc/scheduler.cpp).

It restates what rvllm's engine uses from the kv-cache-scheduler crate
(src/engine.rs:351-539): FIFO waiting / running lists, per-sequence
token_ids and block tables, pool.available() / total_allocs,
prefix_cache.match_prefix, prefill, step (with preemption), finish_sequence
and the prefix-cache metrics. This wrapper only marshals arguments.
"""
from __future__ import annotations

import ctypes
from typing import List, Sequence, Tuple

import numpy as np

from . import _lib
from ._lib import RvkvError


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64).astype(np.int32))


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class Scheduler:
    def __init__(self, num_blocks: int, block_size: int):
        self._L = _lib.load()
        self._h = self._L.rvkv_sched_create(num_blocks, block_size)
        if not self._h:
            raise RvkvError(self._err())
        self.num_blocks, self.block_size = num_blocks, block_size

    def _err(self) -> str:
        return (self._L.rvkv_sched_last_error() or b"sched: failed").decode()

    def _check(self, rc: int) -> int:
        if rc < 0:
            raise RvkvError(self._err(), int(rc))
        return rc

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.rvkv_sched_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- queues ---------------------------------------------------------------
    def add_request(self, tokens: Sequence[int]) -> int:
        t = _i32(tokens)
        return self._check(self._L.rvkv_sched_add_request(self._h, _p(t),
                                                          len(t)))

    def _ids(self, fn, n: int) -> List[int]:
        out = np.zeros(max(n, 1), np.int64)
        m = fn(self._h, _p(out), n)
        return out[:m].tolist()

    @property
    def waiting(self) -> List[int]:
        return self._ids(self._L.rvkv_sched_waiting,
                         self._L.rvkv_sched_num_waiting(self._h))

    @property
    def running(self) -> List[int]:
        return self._ids(self._L.rvkv_sched_running,
                         self._L.rvkv_sched_num_running(self._h))

    def num_waiting(self) -> int:
        return self._L.rvkv_sched_num_waiting(self._h)

    def num_running(self) -> int:
        return self._L.rvkv_sched_num_running(self._h)

    def has(self, seq: int) -> bool:
        return bool(self._L.rvkv_sched_has_seq(self._h, seq))

    # -- pool and metrics -----------------------------------------------------
    def available(self) -> int:
        return self._L.rvkv_sched_available(self._h)

    @property
    def total_allocs(self) -> int:
        return self._L.rvkv_sched_total_allocs(self._h)

    def metrics(self) -> Tuple[int, int, int]:
        """(prefix_hits, prefix_total, preemptions)."""
        v = [ctypes.c_uint64() for _ in range(3)]
        self._L.rvkv_sched_metrics(self._h, *[ctypes.byref(x) for x in v])
        return tuple(int(x.value) for x in v)

    def refcount(self, block: int) -> int:
        return self._L.rvkv_sched_refcount(self._h, block)

    # -- scheduling -----------------------------------------------------------
    def match_prefix(self, tokens: Sequence[int]) -> Tuple[int, List[int]]:
        """(matched_tokens, matched_blocks) of prefix_cache.match_prefix."""
        t = _i32(tokens)
        cap = len(t) // self.block_size + 1
        out = np.zeros(cap, np.uint32)
        n = self._L.rvkv_sched_match_prefix(self._h, _p(t), len(t), _p(out),
                                            cap)
        return n * self.block_size, out[:n].tolist()

    def prefill(self, seq: int) -> int:
        m = ctypes.c_uint32()
        self._check(self._L.rvkv_sched_prefill(self._h, seq, ctypes.byref(m)))
        return m.value

    def step(self) -> int:
        n = ctypes.c_uint32()
        self._check(self._L.rvkv_sched_step(self._h, ctypes.byref(n)))
        return n.value

    def take_cow(self) -> Tuple[np.ndarray, np.ndarray]:
        cap = 64
        while True:
            src = np.zeros(cap, np.uint32)
            dst = np.zeros(cap, np.uint32)
            n = self._L.rvkv_sched_take_cow(self._h, _p(src), _p(dst), cap)
            if n <= cap:
                return src[:n], dst[:n]
            cap = n

    def finish_sequence(self, seq: int) -> None:
        self._check(self._L.rvkv_sched_finish(self._h, seq))

    def remove(self, seq: int) -> None:
        self._check(self._L.rvkv_sched_remove(self._h, seq))

    def fork(self, seq: int) -> int:
        return self._check(self._L.rvkv_sched_fork(self._h, seq))

    # -- one sequence ---------------------------------------------------------
    def num_tokens(self, seq: int) -> int:
        return self._L.rvkv_sched_num_tokens(self._h, seq)

    def blocks(self, seq: int) -> List[int]:
        n = self._L.rvkv_sched_num_blocks(self._h, seq)
        out = np.zeros(max(n, 1), np.uint32)
        m = self._L.rvkv_sched_table(self._h, seq, _p(out), n)
        return out[:m].tolist()

    def logical_to_physical(self, seq: int, pos: int) -> Tuple[int, int]:
        b, o = ctypes.c_uint32(), ctypes.c_uint32()
        self._check(self._L.rvkv_sched_slot(self._h, seq, pos,
                                            ctypes.byref(b), ctypes.byref(o)))
        return b.value, o.value

    def tokens(self, seq: int) -> List[int]:
        n = self._L.rvkv_sched_tokens(self._h, seq, None, 0)
        out = np.zeros(max(n, 1), np.int32)
        self._L.rvkv_sched_tokens(self._h, seq, _p(out), n)
        return out[:n].tolist()

    def set_tokens(self, seq: int, tokens: Sequence[int]) -> None:
        t = _i32(tokens)
        self._check(self._L.rvkv_sched_set_tokens(self._h, seq, _p(t),
                                                  len(t)))
