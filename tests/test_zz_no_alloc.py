"""rvkv_paged_decode_noalloc: the decode entry point that allocates nothing
(its split-sequence partials live in a static per-GPU device array). Called
through the C ABI and checked against rvkv_paged_decode on the same inputs,
two calls in a row, the second smaller; plus the size limit."""
from __future__ import annotations

import ctypes
import math
import sys

import numpy as np
import pytest
import torch

from rvllm_amd import workloads as W
from rvllm_amd._lib import RVKV_EUNSUPPORTED, RvkvError, check, load
from rvllm_amd.kv_storage import HipKvStorage
from tests.gpu_util import dev_u32, fill_layer

pytestmark = pytest.mark.gpu


def _noalloc(st, q, tables, ctx, max_ctx, window=0):
    L = load()
    out = torch.empty_like(q)
    batch, n_heads, hd = q.shape
    rc = L.rvkv_paged_decode_noalloc(
        st._pool, 0, ctypes.c_void_p(q.data_ptr()),
        ctypes.c_void_p(tables.data_ptr()), ctypes.c_void_p(ctx.data_ptr()),
        batch, tables.shape[1], n_heads, max_ctx, 1.0 / math.sqrt(hd),
        window, ctypes.c_void_p(out.data_ptr()))
    check(rc)
    return out


def test_noalloc_decode_matches_workspace_decode():
    print("\n[gpu] noalloc decode vs paged_decode", flush=True)
    sys.stdout.flush()
    bs, nkv, hd, H = 16, 4, 128, 16
    st = HipKvStorage(1, 2200, bs, nkv, hd)
    fill_layer(st, 0, seed=11)
    cases = [(np.array([9000, 17, 4000, 12000, 1], np.uint32), 0),
             (np.array([3000, 700, 5], np.uint32), 300)]
    for i, (lens, window) in enumerate(cases):
        cfg = W.Config("na", 9, 1, H, nkv, hd, bs, len(lens))
        db = W.ragged_batch(cfg, lens, seed=i)
        assert db.num_blocks <= 2200
        max_ctx = int(lens.max())
        # the split path (partials in the scratch array) is what is tested
        assert st.decode_workspace_bytes(len(lens), H, max_ctx) > 0
        tables, ctx = dev_u32(db.padded_tables()), dev_u32(lens)
        q = torch.randn(len(lens), H, hd, device="cuda",
                        generator=torch.Generator("cuda").manual_seed(i))
        want = st.paged_decode(0, q, tables, ctx, max_ctx, window=window)
        got = _noalloc(st, q, tables, ctx, max_ctx, window)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        # same kernels and partitioning: bit-identical
        assert torch.equal(got, want), (i, (got - want).abs().max().item())


@pytest.mark.parametrize("hd,bs,dtype,split", [(128, 16, torch.float32, True),
                                                (96, 16, torch.float16, True),
                                                (96, 12, torch.float16, False)])
def test_noalloc_decode_other_pools(hd, bs, dtype, split):
    """An f32 pool (the f32 decode kernel, its partials in the scratch
    array), head_dim 96 on an f16 pool with power-of-two blocks (the tuned
    kernel at a rounded-up head_dim, whose partial rows have the rounded
    width, in the scratch array) and a shape on the generic kernel (no
    partials): bit-identical to rvkv_paged_decode, two calls in a row, the
    second smaller."""
    print(f"\n[gpu] noalloc other pools hd={hd} bs={bs} {dtype}", flush=True)
    nkv, H = 2, 6
    st = HipKvStorage(1, 1200, bs, nkv, hd, dtype=dtype)
    g = torch.Generator(device="cuda").manual_seed(hd)
    n = 1200 * bs
    slots = torch.arange(n, device="cuda")
    k = torch.randn((n, nkv, hd), generator=g, device="cuda")
    st.write_tokens(0, (slots // bs).int(), (slots % bs).int(), k, k * 0.5)
    for i, lens in enumerate([np.array([5000, 17, 900, 3], np.uint32),
                              np.array([700, 40], np.uint32)]):
        cfg = W.Config("na2", 9, 1, H, nkv, hd, bs, len(lens))
        db = W.ragged_batch(cfg, lens, seed=i)
        assert db.num_blocks <= 1200
        max_ctx = int(lens.max())
        tables, ctx = dev_u32(db.padded_tables()), dev_u32(lens)
        q = torch.randn(len(lens), H, hd, device="cuda", generator=g)
        if split and i == 0:
            assert st.decode_workspace_bytes(len(lens), H, max_ctx) > 0
        want = st.paged_decode(0, q, tables, ctx, max_ctx)
        got = _noalloc(st, q, tables, ctx, max_ctx)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), (i, (got - want).abs().max().item())


def test_noalloc_decode_rejects_oversized_partials():
    """A shape whose partials need more than the 8 MiB array (head_dim 256,
    8 query heads per KV head, 511 sequences split in two) is refused
    before anything is launched."""
    bs, nkv, hd, H = 16, 1, 256, 8
    st = HipKvStorage(1, 64, bs, nkv, hd)
    batch, max_ctx = 511, 512
    need = st.decode_workspace_bytes(batch, H, max_ctx)
    assert need > (8 << 20)
    q = torch.zeros(batch, H, hd, device="cuda")
    tables = torch.zeros(batch, 32, dtype=torch.int32, device="cuda")
    ctx = torch.ones(batch, dtype=torch.int32, device="cuda")
    with pytest.raises(RvkvError, match="paged_decode_noalloc: decode "
                       "partials exceed the 8 MiB scratch") as e:
        _noalloc(st, q, tables, ctx, max_ctx)
    assert e.value.code == RVKV_EUNSUPPORTED


def test_noalloc_decode_two_streams():
    """Two calls that both keep partials in the scratch array, queued on two
    different streams with no host synchronisation between them: the second
    waits for the first on the device, so both match rvkv_paged_decode."""
    print("\n[gpu] noalloc decode on two streams", flush=True)
    bs, nkv, hd, H = 16, 4, 128, 16
    st = HipKvStorage(1, 2200, bs, nkv, hd)
    fill_layer(st, 0, seed=5)
    lens = [np.array([9000, 12000, 4000], np.uint32),
            np.array([15000, 300, 8000, 7000], np.uint32)]
    dbs = [W.ragged_batch(W.Config("na3", 9, 1, H, nkv, hd, bs, len(x)), x,
                          seed=20 + i) for i, x in enumerate(lens)]
    args = []
    for i, (x, db) in enumerate(zip(lens, dbs)):
        assert db.num_blocks <= 2200
        q = torch.randn(len(x), H, hd, device="cuda",
                        generator=torch.Generator("cuda").manual_seed(30 + i))
        args.append((q, dev_u32(db.padded_tables()), dev_u32(x),
                     int(x.max())))
        assert st.decode_workspace_bytes(len(x), H, int(x.max())) > 0
    want = [st.paged_decode(0, q, t, c, m) for q, t, c, m in args]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    got = []
    for s, (q, t, c, m) in zip((s1, s2), args):
        with torch.cuda.stream(s):
            st.set_stream(s)
            got.append(_noalloc(st, q, t, c, m))
    torch.cuda.synchronize()
    st.set_stream(torch.cuda.current_stream())
    for i in range(2):
        assert torch.equal(got[i], want[i]), (
            i, (got[i] - want[i]).abs().max().item())
