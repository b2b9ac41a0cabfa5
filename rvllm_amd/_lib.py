"""ctypes binding of librvkv.so (the C ABI declared in include/rvkv.h).

There is no fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librvkv.so")

RVKV_F16, RVKV_F32 = 1, 2
RVKV_OK, RVKV_EINVAL, RVKV_EHIP, RVKV_ENOMEM, RVKV_EUNSUPPORTED = 0, -1, -2, -3, -4

# Every symbol include/rvkv.h declares, with (restype, argtypes).
_P = ctypes.c_void_p
_u32, _i32, _u64, _i64 = (ctypes.c_uint32, ctypes.c_int32, ctypes.c_uint64,
                          ctypes.c_int64)
_sz, _f32, _int = ctypes.c_size_t, ctypes.c_float, ctypes.c_int
_pu32 = ctypes.POINTER(ctypes.c_uint32)

SIGNATURES = {
    "rvkv_last_error": (ctypes.c_char_p, []),
    "rvkv_pool_create": (_int, [_u32, _u32, _u32, _u32, _u32, _int, _P,
                                ctypes.POINTER(_P)]),
    "rvkv_pool_destroy": (None, [_P]),
    "rvkv_pool_bytes": (_sz, [_P]),
    "rvkv_pool_set_stream": (_int, [_P, _P]),
    "rvkv_append": (_int, [_P, _u32, _P, _P, _int, _P, _P, _u32]),
    "rvkv_append_layers": (_int, [_P, _u32, _u32, _P, _P, _int, _u64, _P, _P,
                                  _u32]),
    "rvkv_gather": (_int, [_P, _u32, _P, _u32, _u32, _u32, _P, _P, _int]),
    "rvkv_paged_decode": (_int, [_P, _u32, _P, _P, _P, _u32, _u32, _u32, _u32,
                                 _f32, _i32, _P, _P, _sz]),
    "rvkv_paged_decode_noalloc": (_int, [_P, _u32, _P, _P, _P, _u32, _u32,
                                         _u32, _u32, _f32, _i32, _P]),
    "rvkv_decode_workspace_bytes": (_sz, [_P, _u32, _u32, _u32]),
    "rvkv_decode_partition_tokens": (_u32, [_P, _u32, _u32, _u32]),
    "rvkv_decode_plan_create": (_int, [_P, _P, _u32, _u32, _i32,
                                       ctypes.POINTER(_P)]),
    "rvkv_decode_plan_update": (_int, [_P, _P, _u32]),
    "rvkv_decode_plan_update_tables": (_int, [_P, _P, _P, _u32, _u32]),
    "rvkv_decode_plan_destroy": (None, [_P]),
    "rvkv_decode_plan_workspace_bytes": (_sz, [_P]),
    "rvkv_decode_plan_items": (_u32, [_P]),
    "rvkv_paged_decode_planned": (_int, [_P, _P, _u32, _P, _P, _P, _u32, _f32,
                                         _P, _P, _sz]),
    "rvkv_decode_step": (_int, [_P, _P, _u32, _P, _P, _int, _P, _P, _P, _P,
                                _P, _u32, _u32, _u32, _u32, _f32, _i32, _P,
                                _P, _sz]),
    "rvkv_paged_prefill": (_int, [_P, _u32, _P, _P, _P, _P, _u32, _u32, _u32,
                                  _u32, _f32, _i32, _P]),
    "rvkv_attn_prep": (_int, [_P, _u32, _P, _P, _P, _u32, _u32, _P, _P, _P,
                              _P, _P, _f32, _P, _P, _P, _P, _P]),
    "rvkv_attn_prep_qkv": (_int, [_P, _u32, _P, _u32, _u32, _P, _P, _P, _f32,
                                  _P, _P, _P, _P, _P]),
    "rvkv_copy_blocks": (_int, [_P, _P, _P, _u32]),
    "rvkv_read_blocks": (_int, [_P, _u32, _u32, _P, _u32, _P]),
    "rvkv_block_checksums": (_int, [_P, _u32, _u32, _P, _u32, _P]),
    "rvkv_bm_create": (_P, [_u32, _u32]),
    "rvkv_bm_destroy": (None, [_P]),
    "rvkv_bm_available": (_u32, [_P]),
    "rvkv_bm_shuffle_free": (None, [_P, _u64]),
    "rvkv_bm_add_seq": (_i64, [_P, _u32]),
    "rvkv_bm_fork_seq": (_i64, [_P, _i64, _u32, _u32]),
    "rvkv_bm_free_seq": (_int, [_P, _i64]),
    "rvkv_bm_append_slot": (_int, [_P, _i64, _pu32, _pu32, _pu32, _pu32]),
    "rvkv_bm_free_seqs": (_int, [_P, _P, _u32]),
    "rvkv_bm_add_seqs": (_int, [_P, _P, _u32, _P]),
    "rvkv_bm_append_slots": (_int, [_P, _P, _u32, _P, _P, _P, _P, _pu32]),
    "rvkv_bm_fill_tables": (_int, [_P, _P, _u32, _u32, _P, _P]),
    "rvkv_bm_slot": (_int, [_P, _i64, _u32, _pu32, _pu32]),
    "rvkv_bm_num_tokens": (_u32, [_P, _i64]),
    "rvkv_bm_num_blocks": (_u32, [_P, _i64]),
    "rvkv_bm_refcount": (_u32, [_P, _u32]),
    "rvkv_bm_table": (_int, [_P, _i64, _pu32, _u32]),
    "rvkv_argmax": (_int, [_P, _u32, _u32, _P, _P]),
    "rvkv_sched_last_error": (ctypes.c_char_p, []),
    "rvkv_sched_create": (_P, [_u32, _u32]),
    "rvkv_sched_destroy": (None, [_P]),
    "rvkv_sched_add_request": (_i64, [_P, _P, _u32]),
    "rvkv_sched_available": (_u32, [_P]),
    "rvkv_sched_total_allocs": (_u64, [_P]),
    "rvkv_sched_metrics": (None, [_P, _P, _P, _P]),
    "rvkv_sched_num_waiting": (_u32, [_P]),
    "rvkv_sched_num_running": (_u32, [_P]),
    "rvkv_sched_waiting": (_u32, [_P, _P, _u32]),
    "rvkv_sched_running": (_u32, [_P, _P, _u32]),
    "rvkv_sched_has_seq": (_int, [_P, _i64]),
    "rvkv_sched_match_prefix": (_u32, [_P, _P, _u32, _P, _u32]),
    "rvkv_sched_prefill": (_int, [_P, _i64, _pu32]),
    "rvkv_sched_step": (_int, [_P, _pu32]),
    "rvkv_sched_take_cow": (_u32, [_P, _P, _P, _u32]),
    "rvkv_sched_finish": (_int, [_P, _i64]),
    "rvkv_sched_remove": (_int, [_P, _i64]),
    "rvkv_sched_fork": (_i64, [_P, _i64]),
    "rvkv_sched_num_tokens": (_u32, [_P, _i64]),
    "rvkv_sched_num_blocks": (_u32, [_P, _i64]),
    "rvkv_sched_table": (_u32, [_P, _i64, _P, _u32]),
    "rvkv_sched_slot": (_int, [_P, _i64, _u32, _pu32, _pu32]),
    "rvkv_sched_tokens": (_u32, [_P, _i64, _P, _u32]),
    "rvkv_sched_set_tokens": (_int, [_P, _i64, _P, _u32]),
    "rvkv_sched_refcount": (_u32, [_P, _u32]),
}


class RvkvError(RuntimeError):
    """A failed rvkv call; ``code`` is the negative RVKV_E* value and the
    message is the library's "<op>: <reason>" string."""

    def __init__(self, message: str, code: int = RVKV_EINVAL):
        super().__init__(message)
        self.code = code


_lib = None


def load() -> ctypes.CDLL:
    """Loads librvkv.so once; raises RvkvError if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RvkvError(
                f"{LIB_PATH} is not built (run: python -m rvllm_amd.build)",
                RVKV_EUNSUPPORTED)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


_calib = None


def load_calib() -> ctypes.CDLL:
    """Loads librvkv_calib.so, the benchmark's streaming-read probe (not part
    of the product ABI): rvkv_calib_read_probe(buf, bytes, workgroups, sink,
    stream) -> 0 or -1, reason in rvkv_calib_last_error()."""
    global _calib
    if _calib is None:
        path = os.path.join(HERE, "librvkv_calib.so")
        if not os.path.exists(path):
            raise RvkvError(f"{path} is not built (run: python -m "
                            "rvllm_amd.build)", RVKV_EUNSUPPORTED)
        L = ctypes.CDLL(path)
        L.rvkv_calib_read_probe.restype = _int
        L.rvkv_calib_read_probe.argtypes = [_P, _sz, _u32, _P, _P]
        L.rvkv_calib_paged_probe.restype = _int
        L.rvkv_calib_paged_probe.argtypes = [_P, _u32, _P, _u32, _u32, _P]
        L.rvkv_calib_copy_probe.restype = _int
        L.rvkv_calib_copy_probe.argtypes = [_P, _P, _sz, _sz, _u32, _P]
        L.rvkv_calib_last_error.restype = ctypes.c_char_p
        L.rvkv_calib_last_error.argtypes = []
        _calib = L
    return _calib


def check_calib(rc: int) -> None:
    if rc != 0:
        raise RvkvError(load_calib().rvkv_calib_last_error().decode(), rc)


def check(rc: int) -> None:
    """Raises RvkvError carrying the library's message when rc != 0."""
    if rc != RVKV_OK:
        msg = load().rvkv_last_error().decode()
        raise RvkvError(msg or f"rvkv call failed with code {rc}", rc)
