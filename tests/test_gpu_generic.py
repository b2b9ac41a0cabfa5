"""GPU parity of the shapes the tuned attention kernels do not take, which
run the generic kernel: head_dim above 256 (up to 1024), block sizes that
are not a power of two (or too small for the decode kernel's loads), and
paged prefill over an f32 cache or at any head_dim. rvllm's CPU path takes
every such shape (src/model.rs:346-415, 628-644; the Metal test runs head_dim
6 and 200, src/metal/ops.rs:684-691). All through the C ABI, against the
oracle's float64 attention over the same cells and, for the Metal cases,
against the reference test's own f32-cache expectations."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rvllm_amd import workloads as W
from rvllm_amd._lib import RvkvError
from rvllm_amd.kv_storage import HipDecodePlan, HipKvStorage
from tests.golden.make_golden import METAL_CASES, metal_case_inputs
from tests.gpu_util import dev_u32

pytestmark = pytest.mark.gpu

# The generic kernel widens cells exactly and computes in f32.
ATOL = 1e-4
# The Metal golden values are float64 over the same f32 cells.
ATOL_GOLDEN = 2e-5


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu] {request.node.name}", flush=True)
    sys.stdout.flush()
    yield
    torch.cuda.synchronize()


def _pool(bs, nkv, hd, lens, seed, dtype=torch.float16, extra=3):
    """A pool filled with N(0,1) rows at every slot and the oracle cache
    holding the same cells."""
    cfg = W.Config("gen", 9, 1, nkv, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, np.maximum(lens, 1), seed=seed,
                        extra_blocks=extra)
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd, dtype=dtype)
    ref = orc.KvCache(db.num_blocks, bs, nkv, hd,
                      orc.F32 if dtype == torch.float32 else orc.F16)
    rng = np.random.default_rng(seed)
    n = db.num_blocks * bs
    k = rng.standard_normal((n, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((n, nkv, hd)).astype(np.float32)
    slots = np.arange(n)
    st.write_tokens(0, dev_u32(slots // bs), dev_u32(slots % bs),
                    torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    ref.write_tokens(slots // bs, slots % bs, k, v)
    return db, st, ref


@pytest.mark.parametrize("hd,bs,G,dtype", [
    (264, 16, 2, torch.float16), (512, 16, 3, torch.float16),
    (1024, 8, 1, torch.float16), (320, 16, 4, torch.float32),
    (64, 12, 4, torch.float16), (128, 3, 2, torch.float16),
    (64, 4, 7, torch.float16), (256, 1, 2, torch.float16),
    (96, 24, 3, torch.float32), (128, 48, 2, torch.float32)])
def test_generic_decode(hd, bs, G, dtype):
    """Uniform, windowed and planned decode and both decode steps (append
    then attend) on shapes outside the tuned kernels: an empty sequence
    gets zeros, the step's rows land bit-exactly at their slots."""
    nkv = 2
    lens = np.array([1, 17, 300, 700, 5, 40], np.uint32)
    db, st, ref = _pool(bs, nkv, hd, lens, seed=hd + bs + G, dtype=dtype)
    H = G * nkv
    rng = np.random.default_rng(G)
    qn = rng.standard_normal((len(lens), H, hd)).astype(np.float32)
    q = torch.from_numpy(qn).cuda()
    padded = db.padded_tables()
    tab = dev_u32(padded)
    flat = padded.reshape(-1)
    assert st.decode_workspace_bytes(len(lens), H, int(lens.max())) == 0
    ctx = lens.copy()
    ctx[4] = 0
    for window in (0, 100):
        out = st.paged_decode(0, q, tab, dev_u32(ctx), int(ctx.max()),
                              window=window)
        want = orc.paged_decode_f64(ref, qn, flat, db.max_blocks, ctx,
                                    window=window)
        assert np.abs(out.cpu().numpy() - want).max() < ATOL, window
        assert out[4].eq(0).all()
    plan = HipDecodePlan(st, ctx, H)
    out = st.paged_decode_planned(0, plan, q, tab, dev_u32(ctx))
    want = orc.paged_decode_f64(ref, qn, flat, db.max_blocks, ctx)
    assert np.abs(out.cpu().numpy() - want).max() < ATOL
    plan.update(lens)
    nk = rng.standard_normal((len(lens), nkv, hd)).astype(np.float32)
    nv = rng.standard_normal((len(lens), nkv, hd)).astype(np.float32)
    for use_plan in (False, True):
        got = st.decode_step(0, torch.from_numpy(nk).cuda(),
                             torch.from_numpy(nv).cuda(),
                             dev_u32(db.slot_block), dev_u32(db.slot_off), q,
                             tab, dev_u32(lens), int(lens.max()),
                             plan=plan if use_plan else None)
        want = orc.decode_step(ref, db.slot_block, db.slot_off, nk, nv, flat,
                               db.max_blocks, lens, qn)
        assert np.abs(got.cpu().numpy() - want).max() < ATOL, use_plan
        ids = dev_u32(np.arange(db.num_blocks))
        raw = st.read_blocks(0, 0, ids).cpu().numpy()
        if dtype == torch.float32:
            assert np.array_equal(raw.view(np.uint32), ref.k.view(np.uint32))
        else:
            assert np.array_equal(raw.view(np.uint16), ref.k)
        nk, nv = nv, nk


def test_generic_decode_skips_unreadable_blocks():
    """A table entry past the pool on the generic path: no fault, the keys
    behind it are left out. Expected values: float64 attention over the
    remaining keys (numpy; the oracle is only given valid tables)."""
    hd, bs, nkv, G = 96, 12, 1, 2
    lens = np.array([50, 30], np.uint32)
    db, st, ref = _pool(bs, nkv, hd, lens, seed=3)
    padded = db.padded_tables()
    good = padded.copy()
    padded[0, 1] = 1_000_000
    qn = np.random.default_rng(1).standard_normal(
        (2, G * nkv, hd)).astype(np.float32)
    out = st.paged_decode(0, torch.from_numpy(qn).cuda(), dev_u32(padded),
                          dev_u32(lens), 50).cpu().numpy()
    assert np.isfinite(out).all()
    kf = ref.as_f32(0).astype(np.float64)
    vf = ref.as_f32(1).astype(np.float64)
    keys = [j for j in range(50) if j // bs != 1]
    blk = good[0][np.array(keys) // bs]
    K = kf[blk, np.array(keys) % bs, 0]
    V = vf[blk, np.array(keys) % bs, 0]
    s = qn[0].astype(np.float64) @ K.T / np.sqrt(hd)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    want0 = (p / p.sum(axis=1, keepdims=True)) @ V
    assert np.abs(out[0] - want0).max() < ATOL
    want1 = orc.paged_decode_f64(ref, qn[1:], good[1:].reshape(-1),
                                 db.max_blocks, lens[1:])
    assert np.abs(out[1:] - want1).max() < ATOL


@pytest.mark.parametrize("hd,bs,G,dtype", [
    (6, 16, 2, torch.float16), (40, 3, 3, torch.float16),
    (96, 16, 1, torch.float32), (200, 12, 2, torch.float16),
    (64, 16, 4, torch.float32), (512, 8, 2, torch.float16),
    (128, 4, 2, torch.float16)])
@pytest.mark.parametrize("window", [0, 7])
def test_generic_prefill(hd, bs, G, dtype, window):
    """Chunked prefill (rows at pos_offset + i, read counts below and above
    the chunk's end) on the generic path against the oracle's batch_mask
    attention."""
    nkv, Q = 2, 5
    rng = np.random.default_rng(hd * 3 + bs)
    prior = np.array([0, 3, 20, 41], np.int64)
    read = np.minimum(prior + Q + np.array([0, -2, 1, 0]), prior + Q + 4)
    read = np.maximum(read, 0).astype(np.uint32)
    lens = np.maximum(read, prior + Q).astype(np.uint32)
    db, st, ref = _pool(bs, nkv, hd, lens, seed=hd + G, dtype=dtype)
    H = G * nkv
    qn = rng.standard_normal((len(lens), Q, H, hd)).astype(np.float32)
    out = st.paged_prefill(0, torch.from_numpy(qn).cuda(),
                           dev_u32(db.padded_tables()),
                           dev_u32(prior.astype(np.uint32)), dev_u32(read),
                           window=window).cpu().numpy()
    want = orc.paged_prefill_f64(ref, qn, db.padded_tables().reshape(-1),
                                 db.max_blocks, prior.astype(np.uint32),
                                 read, window=window)
    assert np.abs(out - want).max() < ATOL


@pytest.mark.parametrize("case", range(len(METAL_CASES)))
def test_metal_cases_f32_pool(golden, case):
    """All six attn_decode cases of src/metal/ops.rs:676-766 over an f32
    pool (the reference's own cells): paged prefill with each case's q_len,
    and decode for the q_len 1 cases, against the golden expectations at
    2e-5."""
    c = metal_case_inputs(case)
    B, Q, H, D, bs = c["batch"], c["q_len"], c["n_heads"], c["hd"], c["bs"]
    st = HipKvStorage(1, c["num_blocks"], bs, c["n_kv"], D,
                      dtype=torch.float32)
    nslot = c["num_blocks"] * bs
    slots = np.arange(nslot)
    st.write_tokens(0, dev_u32(slots // bs), dev_u32(slots % bs),
                    torch.from_numpy(c["cache_k"].reshape(nslot, c["n_kv"],
                                                          D)).cuda(),
                    torch.from_numpy(c["cache_v"].reshape(nslot, c["n_kv"],
                                                          D)).cuda())
    valid = np.array([c["ctx"] - 2 * b for b in range(B)], np.uint32)
    tables = dev_u32(c["block_idx"].reshape(B, c["max_blocks"]))
    exp = np.array(golden["metal_attn_decode"][case]["expected"],
                   np.float32).reshape(B, Q, H, D)
    q = c["q"].reshape(B, Q, H, D)
    out = st.paged_prefill(0, torch.from_numpy(q).cuda(), tables,
                           dev_u32(valid - Q), dev_u32(valid)).cpu().numpy()
    assert np.abs(out - exp).max() < ATOL_GOLDEN
    if Q == 1:
        out = st.paged_decode(0, torch.from_numpy(q[:, 0]).cuda(), tables,
                              dev_u32(valid), c["ctx"]).cpu().numpy()
        assert np.abs(out - exp[:, 0]).max() < ATOL_GOLDEN


def test_head_dim_above_1024_raises():
    st = HipKvStorage(1, 4, 16, 1, 1040)
    q = torch.zeros(1, 2, 1040, device="cuda")
    with pytest.raises(RvkvError, match="paged_decode: head_dim"):
        st.paged_decode(0, q, dev_u32([[0]]), dev_u32([4]), 4)
    with pytest.raises(RvkvError, match="paged_prefill: head_dim"):
        st.paged_prefill(0, q.reshape(1, 1, 2, 1040), dev_u32([[0]]),
                         dev_u32([0]), dev_u32([1]))


@pytest.mark.parametrize("hd,dtype,bias,norm", [
    (48, torch.float16, True, True), (96, torch.float16, False, False),
    (200, torch.float16, True, False), (6, torch.float16, False, True),
    (64, torch.float32, True, True), (128, torch.float32, False, False),
    (320, torch.float16, True, True), (512, torch.float32, False, True)])
def test_generic_attn_prep(hd, dtype, bias, norm):
    """rvkv_attn_prep on the generic kernel (head_dim other than
    32/64/128/256, or an f32 pool) against the oracle's restatement of
    src/model.rs:600-626 over the same cell type: without the RMS norm q and
    the cache are bit-identical; with it the sum of squares is reduced in
    another order (q to 2e-6 * (1 + |q|), f16 cells to one ulp, f32 cells to
    2e-6 * (1 + |x|)). The fused-QKV entry point gives the same bits."""
    rng = np.random.default_rng(hd + 2 * bias + norm)
    rows, nb, bs, H, KV = 29, 20, 16, 6, 2
    q = rng.standard_normal((rows, H, hd)).astype(np.float32)
    k = rng.standard_normal((rows, KV, hd)).astype(np.float32)
    v = rng.standard_normal((rows, KV, hd)).astype(np.float32)
    opt = {}
    if bias:
        opt.update(q_bias=rng.standard_normal(H * hd).astype(np.float32),
                   k_bias=rng.standard_normal(KV * hd).astype(np.float32),
                   v_bias=rng.standard_normal(KV * hd).astype(np.float32))
    if norm:
        opt.update(q_norm=rng.standard_normal(hd).astype(np.float32),
                   k_norm=rng.standard_normal(hd).astype(np.float32))
    c, s = orc.rope_cos_sin(1e6, hd, rng.integers(0, 8192, rows))
    slots = rng.permutation(nb * bs)[:rows]
    sb, so = slots // bs, slots % bs
    f32 = dtype == torch.float32
    cache = orc.KvCache(nb, bs, KV, hd, orc.F32 if f32 else orc.F16)
    want_q = orc.attn_prep(cache, q, k, v, c, s, sb, so, eps=1e-6, **opt)
    st = HipKvStorage(1, nb, bs, KV, hd, dtype=dtype)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    got_q = st.attn_prep(0, T(q), T(k), T(v), T(c), T(s), dev_u32(sb),
                         dev_u32(so), eps=1e-6,
                         **{n: T(a) for n, a in opt.items()}).cpu().numpy()
    ids = dev_u32(np.arange(nb))
    gk = st.read_blocks(0, 0, ids).cpu().numpy()
    gv = st.read_blocks(0, 1, ids).cpu().numpy()
    view = np.uint32 if f32 else np.uint16
    ck, cv = cache.k.view(view), cache.v.view(view)
    assert np.array_equal(gv.view(view), cv)  # v: bias + store only
    if not norm:
        assert np.array_equal(got_q, want_q)
        assert np.array_equal(gk.view(view), ck)
    else:
        assert np.max(np.abs(got_q - want_q) / (1 + np.abs(want_q))) < 2e-6
        if f32:
            assert np.max(np.abs(gk - cache.k) / (1 + np.abs(cache.k))) < 2e-6
        else:
            ulp = np.abs(gk.view(np.uint16).astype(np.int32) -
                         cache.k.astype(np.int32))
            assert ulp.max() <= 1
    # the fused [rows, (H + 2 KV) * hd] entry point: same bits
    st2 = HipKvStorage(1, nb, bs, KV, hd, dtype=dtype)
    qkv = np.concatenate([q.reshape(rows, -1), k.reshape(rows, -1),
                          v.reshape(rows, -1)], axis=1)
    fb = None
    if bias:
        fb = T(np.concatenate([opt["q_bias"], opt["k_bias"], opt["v_bias"]]))
    q2 = st2.attn_prep_qkv(0, T(qkv), H, T(c), T(s), dev_u32(sb), dev_u32(so),
                           bias=fb, q_norm=T(opt["q_norm"]) if norm else None,
                           k_norm=T(opt["k_norm"]) if norm else None,
                           eps=1e-6).cpu().numpy()
    assert np.array_equal(q2, got_q)
    assert torch.equal(st2.read_blocks(0, 0, ids), st.read_blocks(0, 0, ids))
    assert torch.equal(st2.read_blocks(0, 1, ids), st.read_blocks(0, 1, ids))
