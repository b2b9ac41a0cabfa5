"""GPU parity: librvkv's HIP kernels (through the C ABI) against the oracle.

Append, gather and copy are bit-exact on cache contents; decode attention
agrees with the oracle's float64 paged attention over the SAME f16 cache
within 2e-3 max-abs (f16 storage, f32 accumulation). Full-size configs are
checked on sampled sequences plus size-independent properties.
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rvllm_amd import workloads as W
from rvllm_amd._lib import RvkvError
from rvllm_amd.kv_storage import HipDecodePlan, HipGatherPlan, HipKvStorage
from tests.golden.make_golden import METAL_CASES, metal_case_inputs
from tests.gpu_util import dev_u32, fill_layer, oracle_subset

pytestmark = pytest.mark.gpu

ATOL = 2e-3  # decode/prefill tolerance: f16 KV with f32 accumulation


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu] {request.node.name}", flush=True)
    sys.stdout.flush()
    yield
    torch.cuda.synchronize()


def f16_from(x_f32: np.ndarray) -> torch.Tensor:
    bits = orc.f32_to_f16_bits(x_f32)
    return torch.from_numpy(bits.view(np.int16).copy()).view(
        torch.float16).cuda()


def bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


# ---- the reference's KATs through the C ABI -------------------------------
def test_kat_round_trip_across_blocks(golden):
    g = golden["reference_kats"]["round_trip_across_blocks"]
    st = HipKvStorage(1, 3, 2, 1, 2)
    k = torch.tensor(g["k"], dtype=torch.float32).reshape(4, 1, 2).cuda()
    st.write_tokens(0, dev_u32(g["block_ids"]), dev_u32(g["offsets"]), k, k)
    raw = st.read_blocks(0, 0, dev_u32([0, 1, 2])).float().cpu().reshape(-1)
    assert raw.tolist() == g["raw_cache"]
    plan = HipGatherPlan([(g["tables"][0], 3), (g["tables"][1], 1)])
    assert plan.ctx_len == 3
    assert plan.block_idx.cpu().tolist() == g["plan_block_idx"]
    ok = torch.zeros(2 * 1 * 3 * 2, device="cuda")
    ov = torch.zeros_like(ok)
    st.gather(0, plan, ok, ov)
    got = ok.cpu().tolist()
    assert got == ov.cpu().tolist()
    assert got[:6] == g["gather_prefix_a"]
    assert got[6:8] == g["gather_prefix_b"]


def test_kat_untouched_slots(golden):
    g = golden["reference_kats"]["untouched_slots"]
    st = HipKvStorage(1, 1, 4, 1, 2)
    t = torch.tensor(g["k"], dtype=torch.float32).reshape(1, 1, 2).cuda()
    st.write_tokens(0, dev_u32([0]), dev_u32([2]), t, t)
    plan = HipGatherPlan([([0], 4)])
    ok = torch.zeros(8, device="cuda")
    ov = torch.zeros(8, device="cuda")
    st.gather(0, plan, ok, ov)
    assert ok.cpu().tolist() == g["gather"]


def test_kat_copy_is_independent_of_original(golden):
    """KvStorage::clone independence (src/kv_storage.rs:239-255) at block
    granularity: copy block 0 -> 1, then write block 0; the copy keeps the
    old contents."""
    st = HipKvStorage(1, 2, 2, 1, 2)
    st.copy_blocks(dev_u32([0]), dev_u32([1]))
    t = torch.tensor([1.0, 1.5]).reshape(1, 1, 2).cuda()
    st.write_tokens(0, dev_u32([0]), dev_u32([0]), t, t)
    raw = st.read_blocks(0, 0, dev_u32([0, 1])).float().cpu().reshape(-1)
    assert raw[:2].tolist() == [1.0, 1.5]
    assert raw[4:6].tolist() == [0.0, 0.0]


def test_rejections_mirror_the_reference():
    st = HipKvStorage(1, 4, 4, 1, 2)
    k = torch.zeros(2, device="cuda")
    v = torch.zeros(4, device="cuda")
    ids = dev_u32([0])
    with pytest.raises(RvkvError, match="kv_write: k and v have different"):
        st.write_tokens(0, ids, ids, k, v)
    k4 = torch.zeros(4, device="cuda")
    with pytest.raises(RvkvError, match="kv_write: block_ids/offsets length"):
        st.write_tokens(0, ids, ids, k4, k4)  # 2 tokens, 1 position
    plan = HipGatherPlan([([0, 1], 2), ([0, 1], 2)])
    with pytest.raises(RvkvError, match="kv_gather: output length"):
        st.gather(0, plan, torch.zeros(3, device="cuda"),
                  torch.zeros(3, device="cuda"))
    plan.ctx_len = 9
    with pytest.raises(RvkvError, match="kv_gather: ctx_len must not exceed"):
        n = 2 * 1 * 9 * 2
        st.gather(0, plan, torch.zeros(n, device="cuda"),
                  torch.zeros(n, device="cuda"))
    with pytest.raises(RvkvError, match="kv_write: layer out of range"):
        st.write_tokens(1, ids, ids, k, k)


# ---- append: bit-exact f32 -> f16 and f16 copies --------------------------
SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0,
                     -1e6, np.inf, -np.inf, 6.1e-5, 6.0e-5, 5.96e-8, 2.98e-8,
                     2.9802326e-08, 1 + 2**-11, 1 + 3 * 2**-11, 1e-9, -3e-6,
                     0.333333], np.float32)


@pytest.mark.parametrize("nkv,hd,bs", [(8, 64, 16), (8, 128, 16), (1, 256, 16),
                                       (2, 64, 32), (3, 2, 2), (5, 12, 3)])
def test_append_bit_exact_f32_source(nkv, hd, bs):
    rng = np.random.default_rng(hd * 7 + nkv)
    nb = 37
    st = HipKvStorage(2, nb, bs, nkv, hd)
    ref = orc.KvCache(nb, bs, nkv, hd, orc.F16)
    slots = rng.permutation(nb * bs)[: nb * bs // 2]
    n = len(slots)
    k = (rng.standard_normal((n, nkv, hd)) * 4).astype(np.float32)
    v = (rng.standard_normal((n, nkv, hd)) * 1e-4).astype(np.float32)
    flat = k.reshape(-1)
    flat[: len(SPECIALS)] = SPECIALS[: min(len(SPECIALS), flat.size)]
    blk, off = slots // bs, slots % bs
    st.write_tokens(1, dev_u32(blk), dev_u32(off), torch.from_numpy(k).cuda(),
                    torch.from_numpy(v).cuda())
    ref.write_tokens(blk, off, k, v)
    ids = dev_u32(np.arange(nb))
    assert np.array_equal(bits(st.read_blocks(1, 0, ids)), ref.k)
    assert np.array_equal(bits(st.read_blocks(1, 1, ids)), ref.v)
    # layer 0 untouched
    assert not bits(st.read_blocks(0, 0, ids)).any()


def test_append_f16_source_copies_bits():
    rng = np.random.default_rng(11)
    nb, bs, nkv, hd = 20, 16, 4, 64
    st = HipKvStorage(1, nb, bs, nkv, hd)
    ref = orc.KvCache(nb, bs, nkv, hd, orc.F16)
    slots = rng.permutation(nb * bs)[:150]
    kb = rng.integers(0, 65536, (150, nkv, hd), dtype=np.uint16)
    kb[(kb & 0x7C00) == 0x7C00] = 0x3C00  # keep values finite
    vb = kb[::-1].copy()
    kt = torch.from_numpy(kb.view(np.int16)).view(torch.float16).cuda()
    vt = torch.from_numpy(vb.view(np.int16)).view(torch.float16).cuda()
    st.write_tokens(0, dev_u32(slots // bs), dev_u32(slots % bs), kt, vt)
    ref.write_tokens_f16(slots // bs, slots % bs, kb, vb)
    ids = dev_u32(np.arange(nb))
    assert np.array_equal(bits(st.read_blocks(0, 0, ids)), ref.k)
    assert np.array_equal(bits(st.read_blocks(0, 1, ids)), ref.v)


@pytest.mark.parametrize("src", ["f32", "f16"])
@pytest.mark.parametrize("nkv,hd,bs,pool_dt", [(1, 256, 16, torch.float16),
                                               (8, 128, 16, torch.float16),
                                               (3, 12, 3, torch.float16),
                                               (2, 64, 16, torch.float32)])
def test_append_layers_equals_per_layer_appends(src, nkv, hd, bs, pool_dt):
    """rvkv_append_layers over layers 1..3 of a 5-layer pool (one launch on
    f16 pools with head_dim % 8 == 0, per-layer appends otherwise) leaves
    exactly the cache bits of three rvkv_append calls, and the oracle's;
    layers 0 and 4 stay untouched. Out-of-range slots are skipped."""
    rng = np.random.default_rng(hd + nkv + bs)
    nb, L = 29, 5
    a = HipKvStorage(L, nb, bs, nkv, hd, dtype=pool_dt)
    b = HipKvStorage(L, nb, bs, nkv, hd, dtype=pool_dt)
    slots = rng.permutation(nb * bs)[: nb * bs // 3]
    n = len(slots)
    blk, off = (slots // bs).astype(np.int64), slots % bs
    blk[3] = nb + 5  # skipped
    rows = (rng.standard_normal((2, 3, n, nkv, hd)) * 3).astype(np.float32)
    rows.reshape(-1)[: len(SPECIALS)] = SPECIALS
    if src == "f16":
        rows = rows.astype(np.float16)
    k, v = torch.from_numpy(rows[0]).cuda(), torch.from_numpy(rows[1]).cuda()
    sb, so = dev_u32(blk), dev_u32(off)
    a.write_tokens_layers(1, sb, so, k, v)
    for l in range(3):
        b.write_tokens(1 + l, sb, so, k[l].contiguous(), v[l].contiguous())
    ids = dev_u32(np.arange(nb))
    for layer in range(L):
        for which in (0, 1):
            ga = bits(a.read_blocks(layer, which, ids))
            gb = bits(b.read_blocks(layer, which, ids))
            assert np.array_equal(ga, gb), (layer, which)
            if layer in (0, 4):
                assert not ga.any()
    if pool_dt == torch.float16:
        for l in range(3):
            ref = orc.KvCache(nb, bs, nkv, hd, orc.F16)
            keep = blk < nb
            if src == "f32":
                ref.write_tokens(blk[keep], off[keep], rows[0, l][keep],
                                 rows[1, l][keep])
            else:
                ref.write_tokens_f16(blk[keep], off[keep],
                                     rows[0, l][keep].view(np.uint16),
                                     rows[1, l][keep].view(np.uint16))
            assert np.array_equal(bits(a.read_blocks(1 + l, 0, ids)), ref.k)
            assert np.array_equal(bits(a.read_blocks(1 + l, 1, ids)), ref.v)
    with pytest.raises(RvkvError, match="kv_write: layer range out of range"):
        a.write_tokens_layers(3, sb, so, k, v)


def test_append_skips_out_of_range_slots():
    st = HipKvStorage(1, 4, 16, 1, 64)
    k = torch.ones(3, 1, 64, device="cuda")
    st.write_tokens(0, dev_u32([0, 99, 1]), dev_u32([0, 0, 40]), k, k)
    raw = st.read_blocks(0, 0, dev_u32([0, 1, 2, 3])).float().cpu()
    assert raw[0, 0].eq(1).all() and raw.sum().item() == 64


# ---- gather: bit-exact, padded plan ---------------------------------------
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("nkv,hd,bs", [(8, 64, 16), (2, 6, 4), (1, 256, 16)])
def test_gather_bit_exact(out_dtype, nkv, hd, bs):
    rng = np.random.default_rng(hd + nkv)
    nb = 50
    st = HipKvStorage(1, nb, bs, nkv, hd)
    fill_layer(st, 0, seed=hd)
    ids = dev_u32(np.arange(nb))
    ref = orc.KvCache(nb, bs, nkv, hd, orc.F16)
    ref.k[:] = bits(st.read_blocks(0, 0, ids))
    ref.v[:] = bits(st.read_blocks(0, 1, ids))
    perm = rng.permutation(nb)
    lens = [3 * bs + 1, bs, 1, 5 * bs]
    tables, at = [], 0
    for n in lens:
        p = -(-n // bs)
        tables.append(perm[at:at + p].tolist())
        at += p
    plan = HipGatherPlan(list(zip(tables, lens)))
    idx, mb, cl = orc.gather_plan(tables, lens)
    assert plan.block_idx.cpu().numpy().view(np.uint32).tolist() == idx.tolist()
    n = len(lens) * nkv * cl * hd
    ok = torch.empty(n, dtype=out_dtype, device="cuda")
    ov = torch.empty(n, dtype=out_dtype, device="cuda")
    st.gather(0, plan, ok, ov)
    wk, wv = ref.gather(idx, len(lens), mb, cl)
    if out_dtype == torch.float32:
        assert np.array_equal(ok.cpu().numpy().reshape(wk.shape), wk)
        assert np.array_equal(ov.cpu().numpy().reshape(wv.shape), wv)
    else:
        assert np.array_equal(bits(ok).reshape(wk.shape),
                              orc.f32_to_f16_bits(wk))
        assert np.array_equal(bits(ov).reshape(wv.shape),
                              orc.f32_to_f16_bits(wv))


# ---- copy-on-write --------------------------------------------------------
def test_copy_blocks_all_layers_bit_exact():
    nl, nb, bs, nkv, hd = 3, 24, 16, 2, 64
    st = HipKvStorage(nl, nb, bs, nkv, hd)
    for layer in range(nl):
        fill_layer(st, layer, seed=100 + layer)
    ids = dev_u32(np.arange(nb))
    before = [[bits(st.read_blocks(l, w, ids)) for w in (0, 1)]
              for l in range(nl)]
    src, dst = [3, 10, 17], [20, 0, 5]
    st.copy_blocks(dev_u32(src), dev_u32(dst))
    for l in range(nl):
        for w in (0, 1):
            ref = orc.KvCache(nb, bs, nkv, hd, orc.F16)
            ref.k[:] = before[l][w]
            ref.v[:] = before[l][w]
            ref.copy_blocks(src, dst)
            after = bits(st.read_blocks(l, w, ids))
            assert np.array_equal(after, ref.k)
    # checksums agree with the oracle's FNV-1a
    csum = st.block_checksums(2, 1, ids).cpu().numpy().view(np.uint64)
    ref = orc.KvCache(nb, bs, nkv, hd, orc.F16)
    ref.v[:] = bits(st.read_blocks(2, 1, ids))
    assert np.array_equal(csum, ref.checksums(1, np.arange(nb)))


def test_cow_then_append_touches_only_the_copy():
    """The sharer's append after a CoW changes its private block only; the
    other sharer's view (its gather) is unchanged (parity unpinned:
    invariant)."""
    nb, bs, nkv, hd = 8, 16, 2, 64
    st = HipKvStorage(1, nb, bs, nkv, hd)
    fill_layer(st, 0, seed=5)
    plan_a = HipGatherPlan([([0, 1], 24)])
    n = 1 * nkv * 24 * hd
    before = torch.empty(n, device="cuda")
    st.gather(0, plan_a, before, torch.empty_like(before))
    st.copy_blocks(dev_u32([1]), dev_u32([6]))
    k = torch.full((1, nkv, hd), 7.0, device="cuda")
    st.write_tokens(0, dev_u32([6]), dev_u32([8]), k, k)
    after = torch.empty_like(before)
    st.gather(0, plan_a, after, torch.empty_like(after))
    assert torch.equal(before, after)
    plan_b = HipGatherPlan([([0, 6], 25)])
    nb_ = 1 * nkv * 25 * hd
    gb = torch.empty(nb_, device="cuda")
    st.gather(0, plan_b, gb, torch.empty_like(gb))
    gb = gb.reshape(nkv, 25, hd)
    assert gb[:, 24].eq(7.0).all()
    assert torch.equal(gb[:, :24].reshape(-1),
                       before.reshape(nkv, 24, hd).reshape(-1))


# ---- paged decode attention ----------------------------------------------
def _decode_vs_oracle(st, layer, db, q, window=0, sample=None):
    tables_pad = dev_u32(db.padded_tables())
    ctx = dev_u32(db.ctx_lens)
    max_ctx = int(db.ctx_lens.max())
    out = st.paged_decode(layer, q, tables_pad, ctx, max_ctx, window=window)
    out = out.cpu().numpy()
    idx = range(db.batch) if sample is None else sample
    tables = [db.tables[b] for b in idx]
    lens = db.ctx_lens[list(idx)]
    cache, padded, mb = oracle_subset(st, layer, tables, lens)
    qn = q.cpu().numpy()[list(idx)]
    want = orc.paged_decode_f64(cache, qn, padded.reshape(-1), mb, lens,
                                window=window)
    err = np.abs(out[list(idx)] - want).max()
    assert np.isfinite(out).all()
    return err


@pytest.mark.parametrize("case", [0, 1, 2, 3, 4, 5])
def test_decode_metal_cases(golden, case):
    """attn_decode cases of src/metal/ops.rs:684-691 at q_len 1 (the decode
    kernel), xorshift data stored as f16, ragged ctx - 2b, reversed block
    tables."""
    c = metal_case_inputs(case)
    B, H, D, bs = c["batch"], c["n_heads"], c["hd"], c["bs"]
    st = HipKvStorage(1, c["num_blocks"], bs, c["n_kv"], D)
    nslot = c["num_blocks"] * bs
    slots = np.arange(nslot)
    st.write_tokens(0, dev_u32(slots // bs), dev_u32(slots % bs),
                    torch.from_numpy(c["cache_k"].reshape(nslot, c["n_kv"],
                                                          D)).cuda(),
                    torch.from_numpy(c["cache_v"].reshape(nslot, c["n_kv"],
                                                          D)).cuda())
    q = torch.from_numpy(c["q"][: B * H * D].reshape(B, H, D)).cuda()
    ctx = np.array([c["ctx"] - 2 * b for b in range(B)], np.uint32)
    tables = dev_u32(c["block_idx"].reshape(B, c["max_blocks"]))
    out = st.paged_decode(0, q, tables, dev_u32(ctx), c["ctx"]).cpu().numpy()
    ref = orc.KvCache(c["num_blocks"], bs, c["n_kv"], D, orc.F16)
    ref.write_tokens(slots // bs, slots % bs,
                     c["cache_k"].reshape(nslot, c["n_kv"], D),
                     c["cache_v"].reshape(nslot, c["n_kv"], D))
    want = orc.paged_decode_f64(ref, q.cpu().numpy(), c["block_idx"],
                                c["max_blocks"], ctx)
    assert np.abs(out - want).max() < ATOL
    if case in (0, 1, 5):  # q_len 1 in the reference too: the golden applies
        exp = np.array(golden["metal_attn_decode"][case]["expected"],
                       np.float32).reshape(B, H, D)
        # golden is over the f32 cache; f16 storage adds <= ~1e-3
        assert np.abs(out - exp).max() < ATOL


@pytest.mark.parametrize("hd,G", [(6, 2), (40, 3), (80, 4), (96, 1),
                                  (200, 2), (136, 8)])
def test_decode_any_head_dim(hd, G):
    """head_dim that is not 32/64/128/256 (rows read element by element,
    the missing lanes as zeros): uniform, planned (split sequences) and the
    fused step against the oracle, the fused step's cache bits equal to
    rvkv_append's."""
    from rvllm_amd.kv_storage import HipDecodePlan
    bs, nkv = 16, 2
    lens = np.array([1, 37, 700, 3000, 16], np.uint32)
    cfg = W.Config("anyhd", 9, 1, G * nkv, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, lens, seed=hd, extra_blocks=3)
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=hd)
    q = torch.randn(len(lens), G * nkv, hd, device="cuda")
    assert _decode_vs_oracle(st, 0, db, q) < ATOL
    assert _decode_vs_oracle(st, 0, db, q, window=100) < ATOL
    err, plan, _ = _planned_vs_oracle(st, 0, db, q)
    assert err < ATOL
    # fused step == append + decode
    nk = torch.randn(len(lens), nkv, hd, device="cuda")
    nv = torch.randn(len(lens), nkv, hd, device="cuda")
    sb, so = dev_u32(db.slot_block), dev_u32(db.slot_off)
    tab, ctx = dev_u32(db.padded_tables()), dev_u32(lens)
    st2 = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st2, 0, seed=hd)
    got = st.decode_step(0, nk, nv, sb, so, q, tab, ctx, int(lens.max()),
                         plan=plan)
    st2.write_tokens(0, sb, so, nk, nv)
    want = st2.paged_decode(0, q, tab, ctx, int(lens.max()))
    ids = dev_u32(np.arange(db.num_blocks))
    for w in (0, 1):
        assert torch.equal(st.read_blocks(0, w, ids), st2.read_blocks(0, w, ids))
    assert (got - want).abs().max().item() < 5e-4


def test_decode_edge_cases():
    """ctx 0 -> zero row; ctx 1; lengths off every boundary; an
    out-of-range block id in a table is read as masked (no fault)."""
    nb, bs, nkv, hd, H = 64, 16, 2, 64, 8
    st = HipKvStorage(1, nb, bs, nkv, hd)
    fill_layer(st, 0, seed=9)
    rng = np.random.default_rng(1)
    perm = rng.permutation(nb).astype(np.uint32)
    lens = np.array([0, 1, 15, 16, 17, 255, 256, 257], np.uint32)
    tables, at = [], 0
    for n in lens:
        p = max(1, -(-int(n) // bs))
        tables.append(perm[at:at + p])
        at += p
    cfg = W.Config("edge", 9, 1, H, nkv, hd, bs, len(lens))
    db = W.DecodeBatch(cfg, nb, lens, tables, np.zeros(len(lens), np.uint32),
                       np.zeros(len(lens), np.uint32))
    q = torch.randn(len(lens), H, hd, device="cuda")
    out = st.paged_decode(0, q, dev_u32(db.padded_tables()),
                          dev_u32(lens), int(lens.max()))
    assert out[0].eq(0).all()
    err = _decode_vs_oracle(st, 0, db, q, sample=list(range(1, len(lens))))
    assert err < ATOL
    # A table entry past the pool: no fault, finite output.
    bad = db.padded_tables()
    bad[7, 3] = 10_000
    out2 = st.paged_decode(0, q, dev_u32(bad), dev_u32(lens), 257)
    assert torch.isfinite(out2).all()
    assert torch.equal(out2[:7], out[:7])


@pytest.mark.parametrize("hd,G", [(64, 4), (128, 2), (256, 4)])
def test_decode_all_blocks_unreadable_gives_zeros(hd, G):
    """Every table entry of one sequence past the pool: nothing readable to
    attend to, so its output rows are zeros (not 0/0), through the uniform
    and the planned path; the other sequences are unaffected."""
    from rvllm_amd.kv_storage import HipDecodePlan
    bs, nkv = 16, 2
    lens = np.array([40, 700, 2100], np.uint32)
    cfg = W.Config("unr", 9, 1, G * nkv, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, lens, seed=hd)
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=hd + 1)
    q = torch.randn(len(lens), G * nkv, hd, device="cuda")
    good = st.paged_decode(0, q, dev_u32(db.padded_tables()), dev_u32(lens),
                           int(lens.max()))
    for victim in (0, 2):
        bad = db.padded_tables()
        bad[victim, :] = 3_000_000_000
        out = st.paged_decode(0, q, dev_u32(bad), dev_u32(lens),
                              int(lens.max()))
        plan = HipDecodePlan(st, lens, G * nkv)
        outp = st.paged_decode_planned(0, plan, q, dev_u32(bad),
                                       dev_u32(lens))
        for o in (out, outp):
            assert o[victim].eq(0).all()
            others = [i for i in range(len(lens)) if i != victim]
            assert torch.allclose(o[others], good[others], atol=ATOL, rtol=0)


@pytest.mark.parametrize("max_ctx", [300, 5000])
def test_decode_multi_partition_and_window(max_ctx):
    """Partition split + reduction pass (several partitions) and the
    sliding window (keys j >= ctx - window)."""
    bs, nkv, hd, H = 16, 4, 128, 8
    rng = np.random.default_rng(2)
    lens = rng.integers(1, max_ctx + 1, 6).astype(np.uint32)
    lens[0] = max_ctx
    cfg = W.Config("mp", 9, 1, H, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, lens, seed=3, extra_blocks=7)
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=max_ctx)
    q = torch.randn(len(lens), H, hd, device="cuda")
    assert st.decode_partition_tokens(len(lens), H, max_ctx) >= 256
    for window in (0, 100, 4096):
        err = _decode_vs_oracle(st, 0, db, q, window=window)
        assert err < ATOL, (window, err)


@pytest.mark.parametrize("G", [1, 2, 3, 5, 7, 8, 9, 16])
def test_decode_group_sizes(G):
    nb, bs, nkv, hd = 96, 16, 2, 64
    st = HipKvStorage(1, nb, bs, nkv, hd)
    fill_layer(st, 0, seed=G)
    cfg = W.Config("g", 9, 1, nkv * G, nkv, hd, bs, 4)
    db = W.ragged_batch(cfg, [300, 17, 700, 64], seed=G)
    q = torch.randn(4, nkv * G, hd, device="cuda")
    assert _decode_vs_oracle(st, 0, db, q) < ATOL


# ---- benchmark workloads (one layer each, full batch and context) ------------
def test_config_smollm2():
    db = W.smollm2_batch()
    c = db.cfg
    st = HipKvStorage(1, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim)
    fill_layer(st, 0, seed=c.seed)
    rng = W.Rng(c.seed + 1)
    # append this step's token (f32 source, reference dtype), then decode
    nk = rng.normal((db.batch, c.n_kv_heads, c.head_dim))
    nv = rng.normal((db.batch, c.n_kv_heads, c.head_dim))
    st.write_tokens(0, dev_u32(db.slot_block), dev_u32(db.slot_off),
                    torch.from_numpy(nk).cuda(), torch.from_numpy(nv).cuda())
    q = torch.from_numpy(rng.normal((db.batch, c.n_heads, c.head_dim))).cuda()
    assert _decode_vs_oracle(st, 0, db, q) < ATOL
    # the oracle's reference pipeline (f32 gqa over the padded gather)
    # agrees too, and its append is bit-identical to the HIP append
    ids = dev_u32(np.arange(db.num_blocks))
    cache = orc.KvCache(db.num_blocks, c.block_size, c.n_kv_heads,
                        c.head_dim, orc.F16)
    cache.k[:] = bits(st.read_blocks(0, 0, ids))
    cache.v[:] = bits(st.read_blocks(0, 1, ids))
    before_k = cache.k.copy()
    idx, mb, _ = orc.gather_plan(db.tables, db.ctx_lens)
    out_ref = orc.decode_step(cache, db.slot_block, db.slot_off, nk, nv, idx,
                              mb, db.ctx_lens, q.cpu().numpy(), n_threads=4)
    assert np.array_equal(cache.k, before_k)  # re-append: same bits
    out = st.paged_decode(0, q, dev_u32(db.padded_tables()),
                          dev_u32(db.ctx_lens), int(db.ctx_lens.max()))
    assert np.abs(out.cpu().numpy() - out_ref).max() < ATOL


@pytest.mark.parametrize("name", ["llama-3.2-1b", "qwen3-0.6b",
                                  "gemma-3-270m"])
def test_config_uniform_full_size(name):
    c = W.CONFIGS[name]
    ctx = {"llama-3.2-1b": 2048, "qwen3-0.6b": 4096, "gemma-3-270m": 1024}[name]
    db = W.uniform_batch(c, ctx)
    st = HipKvStorage(1, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim)
    fill_layer(st, 0, seed=c.seed, scale=c.value_scale)
    q = torch.randn(db.batch, c.n_heads, c.head_dim, device="cuda",
                    generator=torch.Generator("cuda").manual_seed(c.seed))
    rng = np.random.default_rng(c.seed)
    sample = sorted(rng.choice(db.batch, 8, replace=False).tolist())
    assert _decode_vs_oracle(st, 0, db, q, sample=sample) < ATOL
    # size-independent property: a duplicate of every sequence through the
    # same table gives bit-identical rows (deterministic kernel, no races).
    tp = db.padded_tables()
    tables2 = dev_u32(np.concatenate([tp, tp]))
    ctx2 = dev_u32(np.concatenate([db.ctx_lens, db.ctx_lens]))
    out = st.paged_decode(0, torch.cat([q, q]), tables2, ctx2, ctx)
    assert torch.equal(out[: db.batch], out[db.batch:])
    if name == "gemma-3-270m":  # gemma's local layers: 512-token window
        assert _decode_vs_oracle(st, 0, db, q, window=512,
                                 sample=sample) < ATOL


def test_config_qwen25_ragged_prefix_cow():
    db = W.qwen25_batch()
    c = db.cfg
    st = HipKvStorage(2, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim)
    for layer in range(2):
        fill_layer(st, layer, seed=c.seed + layer)
    assert len(db.cow_src) > 0
    # CoW first (all layers), then the append, then decode.
    st.copy_blocks(dev_u32(db.cow_src), dev_u32(db.cow_dst))
    ids = dev_u32(db.cow_dst)
    src_ids = dev_u32(db.cow_src)
    for layer in range(2):
        assert torch.equal(st.read_blocks(layer, 1, ids),
                           st.read_blocks(layer, 1, src_ids))
    g = torch.Generator("cuda").manual_seed(1)
    nk = torch.randn(db.batch, c.n_kv_heads, c.head_dim, device="cuda",
                     generator=g)
    st.write_tokens(1, dev_u32(db.slot_block), dev_u32(db.slot_off), nk, nk)
    q = torch.randn(db.batch, c.n_heads, c.head_dim, device="cuda",
                    generator=g)
    sharers = db.shared_prefix["sharers"]
    rng = np.random.default_rng(0)
    sample = sorted(set(sharers[:6]) | set(rng.choice(db.batch, 6).tolist()))
    assert _decode_vs_oracle(st, 1, db, q, sample=sample) < ATOL
    # The benchmark's path: the plan built with the host tables (shared
    # prefix blocks read by group items on the matrix cores).
    from rvllm_amd.kv_storage import HipDecodePlan
    plan = HipDecodePlan(st, db.ctx_lens, c.n_heads)
    plan.update(db.ctx_lens, db.padded_tables())
    out = st.paged_decode_planned(1, plan, q, dev_u32(db.padded_tables()),
                                  dev_u32(db.ctx_lens)).cpu().numpy()
    cache, padded, mb = oracle_subset(st, 1, [db.tables[b] for b in sample],
                                      db.ctx_lens[sample])
    want = orc.paged_decode_f64(cache, q.cpu().numpy()[sample],
                                padded.reshape(-1), mb, db.ctx_lens[sample])
    assert np.abs(out[sample] - want).max() < ATOL


# ---- planned decode (ragged batches) --------------------------------------
def _planned_vs_oracle(st, layer, db, q, window=0, sample=None):
    from rvllm_amd.kv_storage import HipDecodePlan
    plan = HipDecodePlan(st, db.ctx_lens, q.shape[1], window=window)
    out = st.paged_decode_planned(layer, plan, q, dev_u32(db.padded_tables()),
                                  dev_u32(db.ctx_lens)).cpu().numpy()
    idx = list(range(db.batch)) if sample is None else list(sample)
    cache, padded, mb = oracle_subset(st, layer, [db.tables[b] for b in idx],
                                      db.ctx_lens[idx])
    want = orc.paged_decode_f64(cache, q.cpu().numpy()[idx],
                                padded.reshape(-1), mb, db.ctx_lens[idx],
                                window=window)
    assert np.isfinite(out).all()
    return np.abs(out[idx] - want).max(), plan, out


@pytest.mark.parametrize("bs", [32, 128])
@pytest.mark.parametrize("window", [0, 300])
def test_planned_decode_ragged_splits(window, bs):
    """One long sequence among short ones forces split work items (and the
    reduction rows); an empty sequence gets a zero row. (Block size 128:
    the matrix-core decode's 32-key tiles start inside blocks.)"""
    nkv, hd, H = 2, 64, 14
    lens = np.array([9000, 0, 1, 31, 33, 700, 2048, 5], np.uint32)
    cfg = W.Config("pl", 9, 1, H, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, np.maximum(lens, 1), seed=4)
    db.ctx_lens = lens
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=21)
    q = torch.randn(len(lens), H, hd, device="cuda")
    err, plan, out = _planned_vs_oracle(st, 0, db, q, window=window,
                                        sample=[0, 2, 3, 4, 5, 6, 7])
    assert err < ATOL
    assert plan.items > len(lens)  # the long sequence was split
    assert (out[1] == 0).all()
    # same numbers as the unplanned path within the tolerance
    ref = st.paged_decode(0, q, dev_u32(db.padded_tables()), dev_u32(lens),
                          int(lens.max()), window=window).cpu().numpy()
    assert np.abs(ref - out).max() < ATOL


@pytest.mark.parametrize("case", range(16))
def test_decode_random_shapes(case):
    """Seeded random decode batches: head_dim 32-256 (and 80, the ragged
    path), groups 1-12, block sizes 8-128, 1-40 sequences of log-uniform
    lengths (some empty), windows. The unplanned and the planned decode
    are checked against the float64 oracle on a sample; then the fused
    decode step (append + attend) on the sequences that hold a token, with
    the oracle reading the cache after the append."""
    rng = np.random.default_rng(9300 + case)
    hd = int(rng.choice([32, 64, 80, 128, 256]))
    G = int(rng.integers(1, 13))
    nkv = int(rng.integers(1, 3))
    bs = int(rng.choice([8, 16, 32, 64, 128]))
    n = int(rng.integers(1, 41))
    lens = np.exp(rng.uniform(0, np.log(3000), n)).astype(np.uint32)
    lens[rng.random(n) < 0.1] = 0
    window = int(rng.choice([0, 0, 0, 50]))
    H = G * nkv
    cfg = W.Config("rnd", 9, 1, H, nkv, hd, bs, n)
    db = W.ragged_batch(cfg, np.maximum(lens, 1), seed=case)
    db.ctx_lens = lens
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=case)
    q = torch.randn(n, H, hd, device="cuda",
                    generator=torch.Generator("cuda").manual_seed(case))
    sample = sorted(rng.choice(n, min(n, 10), replace=False).tolist())
    shape = (case, hd, G, nkv, bs, n, window)
    assert _decode_vs_oracle(st, 0, db, q, window, sample) < ATOL, shape
    err, _, out = _planned_vs_oracle(st, 0, db, q, window, sample)
    assert err < ATOL, shape
    assert (out[lens == 0] == 0).all(), shape
    live = [b for b in sample if lens[b] > 0]
    if not live:
        return
    k = torch.randn(n, nkv, hd, device="cuda")
    v = torch.randn(n, nkv, hd, device="cuda")
    keep = lens > 0  # empty sequences append nothing: an out-of-range slot
    sb = np.where(keep, db.slot_block, 0xFFFFFFFF).astype(np.uint32)
    got = st.decode_step(0, k, v, dev_u32(sb), dev_u32(db.slot_off), q,
                         dev_u32(db.padded_tables()), dev_u32(lens),
                         int(lens.max()), window=window).cpu().numpy()
    cache, padded, mb = oracle_subset(st, 0, [db.tables[b] for b in live],
                                      lens[live])
    want = orc.paged_decode_f64(cache, q.cpu().numpy()[live],
                                padded.reshape(-1), mb, lens[live],
                                window=window)
    assert np.abs(got[live] - want).max() < ATOL, shape
    # the appended rows are in the cache, rounded to f16
    for b in live:
        blk, off = int(db.slot_block[b]), int(db.slot_off[b])
        row = st.read_blocks(0, 0, dev_u32([blk])).cpu()[0, off]
        assert torch.equal(row, k[b].cpu().to(torch.float16)), shape


@pytest.mark.parametrize("G", [4, 7])
def test_decode_reduction_over_more_than_64_partitions(G):
    """A 40000-token sequence beside a short one, one KV head: the uniform
    path splits it into ~157 partitions of 256 tokens and the planned path
    into ~79 items of 512, so the reduction merges more than one
    64-partition chunk (G 7 planned: the matrix-core decode's partials)."""
    bs, nkv, hd = 16, 1, 64
    lens = np.array([40000, 300], np.uint32)
    cfg = W.Config("long", 9, 1, G * nkv, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, lens, seed=G)
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=5)
    q = torch.randn(len(lens), G * nkv, hd, device="cuda",
                    generator=torch.Generator("cuda").manual_seed(G))
    assert st.decode_partition_tokens(len(lens), G, 40000) * 64 < 40000
    assert _decode_vs_oracle(st, 0, db, q) < ATOL
    err, plan, _ = _planned_vs_oracle(st, 0, db, q)
    assert err < ATOL
    assert plan.items > 64


@pytest.mark.parametrize("G,hd", [(4, 64), (7, 64), (4, 256)])
def test_decode_large_scores(G, hd):
    """Scores with a standard deviation of ~23 in log2 units (q scaled by
    16): a near one-hot softmax. Probabilities are formed in f16 against a
    running max, so a max taken from a stale accumulator would overflow
    them; the result must stay finite and match the oracle to ATOL (q keeps
    its f32 precision as an f16 hi + lo pair; with q rounded to f16 alone
    the outputs moved by up to 0.007-0.011 here). G 7: the matrix-core
    decode."""
    bs, nkv = 16, 2
    lens = np.array([3000, 77, 1200, 5], np.uint32)
    cfg = W.Config("sharp", 9, 1, G * nkv, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, lens, seed=G + hd)
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=6)
    q = 16.0 * torch.randn(len(lens), G * nkv, hd, device="cuda",
                           generator=torch.Generator("cuda").manual_seed(G))
    assert _decode_vs_oracle(st, 0, db, q) < ATOL
    err, _, _ = _planned_vs_oracle(st, 0, db, q)
    assert err < ATOL


@pytest.mark.parametrize("G,hd", [(4, 64), (2, 128), (4, 256), (7, 64)])
def test_decode_masked_slots_hold_inf(G, hd):
    """Keys the decode must not see are dropped, not weighted by 0: +inf
    (an overflowing f32 -> f16 append) in the unused slots of every
    sequence's last block, in the slot the fused step appends to, and in
    block 0, which the kernels read in place of an out-of-range table id.
    Outputs stay finite and match the oracle, the bad block's keys counted
    as absent. G 7 at hd 64: the matrix-core decode (planned)."""
    from rvllm_amd.kv_storage import HipDecodePlan
    bs, nkv = 16, 2
    lens = np.array([37, 250, 1000, 5, 2001], np.uint32)
    per = [-(-int(n) // bs) for n in lens]
    nb = 1 + sum(per)
    perm = np.random.default_rng(hd + G).permutation(np.arange(1, nb))
    tables, at = [], 0
    for p_ in per:
        tables.append(perm[at:at + p_].astype(np.uint32))
        at += p_
    st = HipKvStorage(1, nb, bs, nkv, hd)
    fill_layer(st, 0, seed=G)

    def put_inf(blocks, offs):
        n = len(blocks)
        big = torch.full((n, nkv, hd), 1e6, device="cuda")  # -> +inf in f16
        st.write_tokens(0, dev_u32(blocks), dev_u32(offs), big, big)
    ub, uo = [0] * bs, list(range(bs))  # all of block 0
    for t, n in zip(tables, lens):
        for pos in range(int(n), len(t) * bs):
            ub.append(int(t[pos // bs]))
            uo.append(pos % bs)
    put_inf(ub, uo)
    bad = [np.array(t) for t in tables]
    bad[2][3] = 10_000  # read as block 0 (all inf), masked
    cfg = W.Config("inf", 9, 1, G * nkv, nkv, hd, bs, len(lens))
    db = W.DecodeBatch(cfg, nb, lens, bad, np.zeros(len(lens), np.uint32),
                       np.zeros(len(lens), np.uint32))
    tab = dev_u32(db.padded_tables())
    ctx = dev_u32(lens)
    q = torch.randn(len(lens), G * nkv, hd, device="cuda",
                    generator=torch.Generator("cuda").manual_seed(hd))
    out_u = st.paged_decode(0, q, tab, ctx, int(lens.max())).cpu().numpy()
    plan = HipDecodePlan(st, lens, G * nkv)
    out_p = st.paged_decode_planned(0, plan, q, tab, ctx).cpu().numpy()
    # Oracle: sequence 2 without its bad block (keys absent).
    exp_tabs = [np.array(t) for t in tables]
    exp_tabs[2] = np.delete(exp_tabs[2], 3)
    exp_lens = lens.copy()
    exp_lens[2] -= bs
    cache, padded, mb = oracle_subset(st, 0, exp_tabs, exp_lens)
    want = orc.paged_decode_f64(cache, q.cpu().numpy(), padded.reshape(-1),
                                mb, exp_lens)
    for out in (out_u, out_p):
        assert np.isfinite(out).all()
        assert np.abs(out - want).max() < ATOL
    # Fused step over slots holding inf: the appended rows replace them.
    last_b = np.array([t[(int(n) - 1) // bs] for t, n in zip(bad, lens)],
                      np.uint32)
    last_o = (lens - 1) % bs
    keep = last_b < nb  # (sequence 2's last block is a good one)
    put_inf(last_b[keep], last_o[keep])
    nk = torch.randn(len(lens), nkv, hd, device="cuda")
    nv = torch.randn(len(lens), nkv, hd, device="cuda")
    for pl in (None, plan):
        got = st.decode_step(0, nk, nv, dev_u32(last_b), dev_u32(last_o), q,
                             tab, ctx, int(lens.max()), plan=pl)
        assert torch.isfinite(got).all()
        after = st.paged_decode(0, q, tab, ctx, int(lens.max()))
        assert (got - after).abs().max().item() < 5e-4
        put_inf(last_b[keep], last_o[keep])


@pytest.mark.parametrize("G", [2, 7])
def test_planned_decode_shared_prefix_order(G):
    """A plan updated with the host block tables orders the items of
    prefix sharers back to back and match the oracle. G 2 (VALU decode):
    bitwise the outputs of the plan built from the lengths alone. G 7
    (matrix-core decode): the sharers' common blocks become group items
    read once for up to four sharers, so the partition (and the summation
    order) differs: within 5e-4 of the lengths-only plan."""
    from rvllm_amd.kv_storage import HipDecodePlan
    bs, nkv, hd = 32, 2, 64
    rng = np.random.default_rng(G)
    n, n_pref = 40, 12
    lens = rng.integers(40, 3000, n).astype(np.uint32)
    prefix = rng.permutation(200)[:32].astype(np.uint32)  # 1024 tokens
    free = list(range(200, 200 + 4000))
    tables = []
    for b in range(n):
        nb = -(-int(lens[b]) // bs)
        t = []
        for i in range(nb):
            if b < n_pref and i < len(prefix) and (i + 1) * bs <= lens[b]:
                t.append(int(prefix[i]))
            else:
                t.append(free.pop(rng.integers(len(free))))
        tables.append(np.array(t, np.uint32))
    num_blocks = 200 + 4000
    cfg = W.Config("pfx", 9, 1, G * nkv, nkv, hd, bs, n)
    db = W.DecodeBatch(cfg, num_blocks, lens, tables,
                       np.zeros(n, np.uint32), np.zeros(n, np.uint32))
    st = HipKvStorage(1, num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=G)
    q = torch.randn(n, G * nkv, hd, device="cuda")
    tab = dev_u32(db.padded_tables())
    ctx = dev_u32(lens)
    plan = HipDecodePlan(st, lens, G * nkv)
    a = st.paged_decode_planned(0, plan, q, tab, ctx).clone()
    ws_plain = plan.workspace_bytes
    plan.update(lens, db.padded_tables())
    b = st.paged_decode_planned(0, plan, q, tab, ctx)
    if G < 5:
        assert torch.equal(a, b)
    else:
        # the group partials are extra partitions of their members
        assert plan.workspace_bytes > ws_plain
        assert (a - b).abs().max().item() < 5e-4
    cache, padded, mb = oracle_subset(st, 0, tables, lens)
    want = orc.paged_decode_f64(cache, q.cpu().numpy(), padded.reshape(-1),
                                mb, lens)
    assert np.abs(b.cpu().numpy() - want).max() < ATOL


@pytest.mark.parametrize("G", [5, 7, 8, 16])
def test_planned_decode_prefix_groups(G):
    """Matrix-core decode with shared-prefix group items (up to 32 // G
    sharers per item). Sharers of two prefixes, with members whose common
    part ends mid-prefix (a private block replaces a shared one), members
    shorter than the prefix, sequences sharing only their first block (no
    group), long members whose own range is split, and one empty sequence.
    The planned decode, the fused decode step (uniform plan rebuilt with
    tables) and a second update all match the oracle; the fused step's
    cache bits equal rvkv_append's."""
    from rvllm_amd.kv_storage import HipDecodePlan
    print(f"\n[gpu] prefix groups G={G}", flush=True)
    bs, nkv, hd = 32, 2, 64
    rng = np.random.default_rng(100 + G)
    n = 48
    lens = rng.integers(300, 5000, n).astype(np.uint32)
    lens[5] = 0
    lens[6:9] = [400, 700, 260]
    prefixes = [rng.permutation(300)[:48].astype(np.uint32),
                300 + rng.permutation(300)[:40].astype(np.uint32)]
    free = list(range(600, 600 + 9000))
    tables = []
    for b in range(n):
        nb = -(-int(lens[b]) // bs)
        pref = prefixes[0] if b < 20 else prefixes[1] if b < 34 else None
        cut = None
        if b in (3, 22):  # the common part ends at block 9 / 17
            cut = 9 if b == 3 else 17
        if b in (40, 41):  # only the first block in common
            pref, cut = prefixes[1], 1
        t = []
        for i in range(nb):
            last = (i + 1) * bs >= lens[b]  # the block the append writes
            if (pref is not None and i < len(pref) and not last and
                    (cut is None or i < cut)):
                t.append(int(pref[i]))
            else:
                t.append(free.pop(rng.integers(len(free))))
        tables.append(np.array(t, np.uint32))
    num_blocks = 600 + 9000
    H = G * nkv
    cfg = W.Config("pfg", 9, 1, H, nkv, hd, bs, n)
    db = W.DecodeBatch(cfg, num_blocks, lens, tables,
                       np.zeros(n, np.uint32), np.zeros(n, np.uint32))
    st = HipKvStorage(1, num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=G)
    q = torch.randn(n, H, hd, device="cuda")
    padded_host = db.padded_tables()
    tab = dev_u32(padded_host)
    ctx = dev_u32(lens)
    plan = HipDecodePlan(st, lens, H)
    plain = st.paged_decode_planned(0, plan, q, tab, ctx).clone()
    ws_plain = plan.workspace_bytes
    plan.update(lens, padded_host)
    assert plan.workspace_bytes > ws_plain  # groups were formed
    got = st.paged_decode_planned(0, plan, q, tab, ctx)
    live = [b for b in range(n) if lens[b]]
    cache, padded, mb = oracle_subset(st, 0, [tables[b] for b in live],
                                      lens[live])
    want = orc.paged_decode_f64(cache, q.cpu().numpy()[live],
                                padded.reshape(-1), mb, lens[live])
    assert np.abs(got.cpu().numpy()[live] - want).max() < ATOL
    assert np.abs(plain.cpu().numpy()[live] - want).max() < ATOL
    assert not got[5].any()
    assert (got - plain).abs().max().item() < 5e-4
    # Fused decode step under the grouped plan: append at position n - 1.
    last_b = np.array([t[(int(x) - 1) // bs] if x else 0
                       for t, x in zip(tables, lens)], np.uint32)
    last_o = np.array([(int(x) - 1) % bs if x else bs for x in lens],
                      np.uint32)
    nk = torch.randn(n, nkv, hd, device="cuda")
    nv = torch.randn(n, nkv, hd, device="cuda")
    ref = HipKvStorage(1, num_blocks, bs, nkv, hd)
    fill_layer(ref, 0, seed=G)
    ref.write_tokens(0, dev_u32(last_b), dev_u32(last_o), nk, nv)
    step = st.decode_step(0, nk, nv, dev_u32(last_b), dev_u32(last_o), q,
                          tab, ctx, int(lens.max()), plan=plan)
    ids = dev_u32(np.unique(last_b))
    for w in (0, 1):
        assert torch.equal(st.read_blocks(0, w, ids), ref.read_blocks(0, w, ids))
    after = ref.paged_decode_planned(0, HipDecodePlan(ref, lens, H), q, tab,
                                     ctx)
    assert (step - after).abs().max().item() < 5e-4
    # A later step: every sequence one token longer, plan updated in place.
    lens2 = np.where(lens > 0, lens + 1, 0).astype(np.uint32)
    ok2 = all(-(-int(x) // bs) <= len(t) for t, x in zip(tables, lens2))
    if ok2:
        plan.update(lens2, padded_host)
        got2 = st.paged_decode_planned(0, plan, q, tab, dev_u32(lens2))
        fresh = st.paged_decode_planned(0, HipDecodePlan(st, lens2, H), q,
                                        tab, dev_u32(lens2))
        assert (got2 - fresh).abs().max().item() < 5e-4
    ref.close()
    st.close()


@pytest.mark.parametrize("case", range(12))
def test_planned_decode_prefix_groups_random(case):
    """Random prefix forests for the group items: a few shared prefixes of
    random lengths, sharers that keep a random number of their prefix's
    blocks, random context lengths (some shorter than their prefix), group
    sizes 5-16, block sizes 16/32/64. The plan built with the host tables
    must give every row within 5e-4 of the lengths-only plan, and sampled
    rows within 2e-3 of the oracle."""
    from rvllm_amd.kv_storage import HipDecodePlan
    rng = np.random.default_rng(7000 + case)
    G = int(rng.choice([5, 6, 7, 8, 11, 16]))
    bs = int(rng.choice([16, 32, 64]))
    nkv, hd = int(rng.choice([1, 2])), 64
    H = G * nkv
    n = int(rng.integers(20, 90))
    n_pref = int(rng.integers(1, 4))
    pref_blocks = [int(rng.integers(4, 48)) for _ in range(n_pref)]
    pool_blocks = 0
    prefixes = []
    for pb in pref_blocks:
        prefixes.append(np.arange(pool_blocks, pool_blocks + pb, dtype=np.uint32))
        pool_blocks += pb
    lens = rng.integers(2, 3500, n).astype(np.uint32)
    tables = []
    for b in range(n):
        nb = -(-int(lens[b]) // bs)
        owner = int(rng.integers(-1, n_pref))  # -1: no prefix
        keep = int(rng.integers(0, pref_blocks[owner] + 1)) if owner >= 0 else 0
        t = []
        for i in range(nb):
            last = (i + 1) * bs >= lens[b]  # the appended key's block: private
            if owner >= 0 and i < keep and not last:
                t.append(int(prefixes[owner][i]))
            else:
                t.append(pool_blocks)
                pool_blocks += 1
        tables.append(np.array(t, np.uint32))
    perm = rng.permutation(pool_blocks).astype(np.uint32)
    tables = [perm[t] for t in tables]
    cfg = W.Config("pgr", 9, 1, H, nkv, hd, bs, n)
    db = W.DecodeBatch(cfg, pool_blocks, lens, tables,
                       np.zeros(n, np.uint32), np.zeros(n, np.uint32))
    st = HipKvStorage(1, pool_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=case)
    q = torch.randn(n, H, hd, device="cuda",
                    generator=torch.Generator("cuda").manual_seed(case))
    tab, ctx = dev_u32(db.padded_tables()), dev_u32(lens)
    plan = HipDecodePlan(st, lens, H)
    plain = st.paged_decode_planned(0, plan, q, tab, ctx).clone()
    plan.update(lens, db.padded_tables())
    got = st.paged_decode_planned(0, plan, q, tab, ctx)
    assert torch.isfinite(got).all()
    assert (got - plain).abs().max().item() < 5e-4, case
    sample = sorted(rng.choice(n, min(n, 10), replace=False).tolist())
    cache, padded, mb = oracle_subset(st, 0, [tables[b] for b in sample],
                                      lens[sample])
    want = orc.paged_decode_f64(cache, q.cpu().numpy()[sample],
                                padded.reshape(-1), mb, lens[sample])
    assert np.abs(got.cpu().numpy()[sample] - want).max() < ATOL, case
    st.close()


def test_planned_decode_update_reuses_plan():
    """update() with new lengths (a decode step later, batch change) gives
    the same results as a freshly built plan."""
    from rvllm_amd.kv_storage import HipDecodePlan
    bs, nkv, hd, H = 16, 4, 128, 8
    cfg = W.Config("pu", 9, 1, H, nkv, hd, bs, 6)
    db = W.ragged_batch(cfg, [4000, 17, 900, 2500, 64, 3000], seed=5)
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=22)
    q = torch.randn(6, H, hd, device="cuda")
    tables = dev_u32(db.padded_tables())
    plan = HipDecodePlan(st, [10, 10, 10], H)
    for lens in ([4000, 17, 900, 2500, 64, 3000], [3999, 16, 899, 2499, 63,
                                                   2999]):
        lens = np.array(lens, np.uint32)
        plan.update(lens)
        out = st.paged_decode_planned(0, plan, q, tables, dev_u32(lens))
        fresh = HipDecodePlan(st, lens, H)
        out2 = st.paged_decode_planned(0, fresh, q, tables, dev_u32(lens))
        assert torch.equal(out, out2)
        db.ctx_lens = lens
        assert _decode_vs_oracle(st, 0, db, q) < ATOL


def test_config_qwen25_planned():
    db = W.qwen25_batch()
    c = db.cfg
    st = HipKvStorage(1, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim)
    fill_layer(st, 0, seed=c.seed)
    q = torch.randn(db.batch, c.n_heads, c.head_dim, device="cuda",
                    generator=torch.Generator("cuda").manual_seed(3))
    rng = np.random.default_rng(1)
    longest = int(np.argmax(db.ctx_lens))
    sample = sorted(set(rng.choice(db.batch, 10).tolist()) | {longest})
    err, plan, _ = _planned_vs_oracle(st, 0, db, q, sample=sample)
    assert err < ATOL


# ---- fused decode step (append + decode in one launch) --------------------
@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("src", [torch.float32, torch.float16])
@pytest.mark.parametrize("G,hd,bs,window", [(4, 64, 16, 0), (2, 128, 16, 0),
                                            (9, 64, 32, 0), (4, 256, 16, 300),
                                            (7, 64, 16, 500), (7, 64, 128, 0)])
def test_decode_step_equals_append_then_decode(planned, src, G, hd, bs,
                                               window):
    """rvkv_decode_step leaves the same cache bits as rvkv_append followed by
    the decode (uniform or planned) and the same output up to summation
    order. Planned with G >= 5 at hd 64 is the matrix-core decode, whose
    fused append puts the new rows into its tile from registers."""
    from rvllm_amd.kv_storage import HipDecodePlan
    nkv = 2
    lens = np.array([5000, 1, 16, 17, 700, 2049, 64, 333], np.uint32)
    cfg = W.Config("fs", 9, 1, nkv * G, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, lens, seed=G + hd)
    stores = [HipKvStorage(1, db.num_blocks, bs, nkv, hd) for _ in range(2)]
    for st in stores:
        fill_layer(st, 0, seed=31)
    g = torch.Generator("cuda").manual_seed(7)
    nk = torch.randn(len(lens), nkv, hd, device="cuda", generator=g).to(src)
    nv = torch.randn(len(lens), nkv, hd, device="cuda", generator=g).to(src)
    q = torch.randn(len(lens), nkv * G, hd, device="cuda", generator=g)
    sb, so = dev_u32(db.slot_block), dev_u32(db.slot_off)
    tables, ctx = dev_u32(db.padded_tables()), dev_u32(lens)
    max_ctx = int(lens.max())
    a, b = stores
    if planned:
        pa = HipDecodePlan(a, lens, nkv * G, window=window)
        pb = HipDecodePlan(b, lens, nkv * G, window=window)
        out_a = a.decode_step(0, nk, nv, sb, so, q, tables, ctx, plan=pa)
        b.write_tokens(0, sb, so, nk, nv)
        out_b = b.paged_decode_planned(0, pb, q, tables, ctx)
    else:
        out_a = a.decode_step(0, nk, nv, sb, so, q, tables, ctx, max_ctx,
                              window=window)
        b.write_tokens(0, sb, so, nk, nv)
        out_b = b.paged_decode(0, q, tables, ctx, max_ctx, window=window)
    ids = dev_u32(np.arange(db.num_blocks))
    for which in (0, 1):
        assert torch.equal(a.read_blocks(0, which, ids),
                           b.read_blocks(0, which, ids))
    # The fused launch folds the new key in after its chunk loop, so only the
    # summation order (and the f16 rounding of that key's probability under
    # a different running max) differs from append-then-decode.
    assert (out_a - out_b).abs().max().item() < 5e-4
    db.ctx_lens = lens
    assert _decode_vs_oracle(a, 0, db, q, window=window) < ATOL


@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("G,hd", [(1, 32), (4, 64), (2, 128), (4, 256),
                                  (3, 64), (6, 64)])
def test_decode_step_short_items(planned, G, hd):
    """Contexts all under 192 tokens: the launch shape for short items (four
    waves of two loads per chunk for groups of up to four
    heads, two waves of four otherwise). The fused step leaves the cache bits of
    append-then-decode and matches it and the oracle."""
    from rvllm_amd.kv_storage import HipDecodePlan
    nkv, bs = 2, 16
    rng = np.random.default_rng(hd * 10 + G)
    lens = rng.integers(1, 192, 40).astype(np.uint32)
    lens[:3] = [1, 191, 64]
    cfg = W.Config("short", 9, 1, nkv * G, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, lens, seed=G + hd)
    stores = [HipKvStorage(1, db.num_blocks, bs, nkv, hd) for _ in range(2)]
    for st in stores:
        fill_layer(st, 0, seed=5)
    g = torch.Generator("cuda").manual_seed(11)
    nk = torch.randn(len(lens), nkv, hd, device="cuda", generator=g)
    nv = torch.randn(len(lens), nkv, hd, device="cuda", generator=g)
    q = torch.randn(len(lens), nkv * G, hd, device="cuda", generator=g)
    sb, so = dev_u32(db.slot_block), dev_u32(db.slot_off)
    tables, ctx = dev_u32(db.padded_tables()), dev_u32(lens)
    a, b = stores
    if planned:
        plan = HipDecodePlan(a, lens, nkv * G)
        out_a = a.decode_step(0, nk, nv, sb, so, q, tables, ctx, plan=plan)
    else:
        out_a = a.decode_step(0, nk, nv, sb, so, q, tables, ctx,
                              int(lens.max()))
    b.write_tokens(0, sb, so, nk, nv)
    out_b = b.paged_decode(0, q, tables, ctx, int(lens.max()))
    ids = dev_u32(np.arange(db.num_blocks))
    for which in (0, 1):
        assert torch.equal(a.read_blocks(0, which, ids),
                           b.read_blocks(0, which, ids))
    assert (out_a - out_b).abs().max().item() < 5e-4
    db.ctx_lens = lens
    assert _decode_vs_oracle(a, 0, db, q) < ATOL


@pytest.mark.parametrize("ksplit", [1, 2, 4])
@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("G,bs,window", [(4, 16, 0), (7, 128, 0),
                                         (8, 16, 300), (7, 32, 5000)])
def test_decode_step_key_split_widths(monkeypatch, ksplit, planned, G, bs,
                                      window):
    """The matrix-core decode (head_dim 64, G >= 4) splits an item's keys
    over 1, 2 or 4 waves of its workgroup and merges them in LDS; the
    launch picks 4 or 1 by grid size, so each width is forced here
    (RVKV_DECODE_KSPLIT / RVKV_DECODE_PLAN_KSPLIT, read at every launch).
    Contexts from 1 key (three waves with nothing to read) to 9000 (several
    partitions and the reduction without a plan, split items with one): the
    fused step leaves append-then-decode's cache bits, its output agrees with
    every other width to summation order and with the oracle."""
    from rvllm_amd.kv_storage import HipDecodePlan
    nkv, hd = 2, 64
    lens = np.array([9000, 1, 2, 33, 64, 65, 700, 2049, 4097, 129],
                    np.uint32)
    cfg = W.Config("ks", 9, 1, nkv * G, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, lens, seed=G * bs)
    g = torch.Generator("cuda").manual_seed(3)
    nk = torch.randn(len(lens), nkv, hd, device="cuda", generator=g)
    nv = torch.randn(len(lens), nkv, hd, device="cuda", generator=g)
    q = torch.randn(len(lens), nkv * G, hd, device="cuda", generator=g)
    sb, so = dev_u32(db.slot_block), dev_u32(db.slot_off)
    tables, ctx = dev_u32(db.padded_tables()), dev_u32(lens)
    max_ctx = int(lens.max())

    def run(width):
        monkeypatch.setenv("RVKV_DECODE_KSPLIT", str(width))
        monkeypatch.setenv("RVKV_DECODE_PLAN_KSPLIT", str(width))
        st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
        fill_layer(st, 0, seed=17)
        if planned:
            plan = HipDecodePlan(st, lens, nkv * G, window=window)
            out = st.decode_step(0, nk, nv, sb, so, q, tables, ctx, plan=plan)
        else:
            out = st.decode_step(0, nk, nv, sb, so, q, tables, ctx, max_ctx,
                                 window=window)
        torch.cuda.synchronize()
        return st, out

    st, out = run(ksplit)
    ref_st, ref = run(1 if ksplit != 1 else 4)
    ids = dev_u32(np.arange(db.num_blocks))
    for which in (0, 1):
        assert torch.equal(st.read_blocks(0, which, ids),
                           ref_st.read_blocks(0, which, ids))
    assert torch.isfinite(out).all()
    assert (out - ref).abs().max().item() < 5e-4
    db.ctx_lens = lens
    assert _decode_vs_oracle(st, 0, db, q, window=window) < ATOL


@pytest.mark.parametrize("window", [0, 100])
@pytest.mark.parametrize("batch", [16, 24, 12])
@pytest.mark.parametrize("G,hd", [(2, 128), (4, 64)])
def test_decode_xcd_sequence_order(batch, G, hd, window):
    """One partition per sequence (contexts <= 256) and a batch of whole
    eights: the uniform decode (VALU at G 2, matrix cores at G 4, hd 64)
    renumbers its workgroups so a sequence's KV heads run back to back on
    one XCD; batch 12 keeps the head rotation. Every (sequence, head) is
    computed once and lands in its own output row: all rows against the
    oracle, fused step and append-then-decode alike, with and without a
    sliding window."""
    nkv, bs = 4, 16
    rng = np.random.default_rng(batch * 10 + G)
    lens = rng.integers(1, 257, batch).astype(np.uint32)
    lens[0] = 256
    cfg = W.Config("xcd", 9, 1, nkv * G, nkv, hd, bs, batch)
    db = W.ragged_batch(cfg, lens, seed=batch + G)
    stores = [HipKvStorage(1, db.num_blocks, bs, nkv, hd) for _ in range(2)]
    for st in stores:
        fill_layer(st, 0, seed=9)
    assert stores[0].decode_workspace_bytes(batch, nkv * G, 256) == 0
    g = torch.Generator("cuda").manual_seed(batch)
    nk = torch.randn(batch, nkv, hd, device="cuda", generator=g)
    nv = torch.randn(batch, nkv, hd, device="cuda", generator=g)
    q = torch.randn(batch, nkv * G, hd, device="cuda", generator=g)
    sb, so = dev_u32(db.slot_block), dev_u32(db.slot_off)
    tables, ctx = dev_u32(db.padded_tables()), dev_u32(lens)
    a, b = stores
    out_a = a.decode_step(0, nk, nv, sb, so, q, tables, ctx, int(lens.max()),
                          window=window)
    b.write_tokens(0, sb, so, nk, nv)
    out_b = b.paged_decode(0, q, tables, ctx, int(lens.max()), window=window)
    ids = dev_u32(np.arange(db.num_blocks))
    for which in (0, 1):
        assert torch.equal(a.read_blocks(0, which, ids),
                           b.read_blocks(0, which, ids))
    assert (out_a - out_b).abs().max().item() < 5e-4
    db.ctx_lens = lens
    assert _decode_vs_oracle(b, 0, db, q, window=window) < ATOL


# ---- continuous-batching churn through the block manager -------------------
def test_churn_driver_parity():
    """A few churn steps (finish 10%, admit 64-token prompts, decode all)
    over a shuffled pool: the last step's appended rows are in the cache bit
    for bit at the block manager's slots, and its decode output matches the
    oracle over the cache the tables point to."""
    from rvllm_amd.engine_sim import ChurnDriver
    cfg = W.Config("churn", 9, 2, 4, 1, 256, 16, 48)
    drv = ChurnDriver(cfg, 48, 200, prompt_len=64, churn=0.1, steps=8,
                      seed=77)
    for _ in range(6):
        drv.step()
    torch.cuda.synchronize()
    tables, lens, blocks, offs = drv.last
    st = drv.st
    for layer in range(cfg.n_layers):
        rows = st.read_blocks(layer, 0, dev_u32(blocks)).cpu().numpy()
        got = rows.view(np.uint16)[np.arange(len(blocks)), offs]
        want = orc.f32_to_f16_bits(drv.nk[layer].cpu().numpy())
        assert np.array_equal(got, want)
    db = W.DecodeBatch(cfg, drv.num_blocks, lens,
                       [tables[i, :-(-int(n) // 16)] for i, n in
                        enumerate(lens)], blocks, offs)
    sample = list(range(0, 48, 5))
    layer = 1
    cache, padded, mb = oracle_subset(st, layer, [db.tables[b] for b in sample],
                                      lens[sample])
    want = orc.paged_decode_f64(cache, drv.q[layer].cpu().numpy()[sample],
                                padded.reshape(-1), mb, lens[sample])
    got = drv.out[layer].cpu().numpy()[sample]
    assert np.abs(got - want).max() < ATOL
    assert drv.bm.available() + sum(
        drv.bm.num_blocks_of(int(s)) for s in drv.running) == drv.num_blocks


def test_churn_full_scale_gemma():
    """configs[4] at its real scale: gemma-3-270m shape (18 layers, 4 q / 1
    KV head, head_dim 256, block_size 16), 1024 sequences at 1024 tokens
    over the 81 920-block pool with a seeded-shuffled free list, 10 % churn
    with 64-token prompts, a few engine steps. Checks, on the last step:
    block accounting (every block free or owned by exactly one running
    sequence); in two layers, every block's checksum unchanged except the
    blocks this step wrote, and in those the written rows (prompt rows and
    decode appends) bit-exact and every other row unchanged; 16 sampled
    sequences' decode output against the oracle (2e-3)."""
    from rvllm_amd.engine_sim import ChurnDriver
    cfg = W.CONFIGS["gemma-3-270m"]
    drv = ChurnDriver(cfg, 1024, 1024, prompt_len=64, churn=0.1, steps=200)
    assert drv.num_blocks == 81920
    all_ids = dev_u32(np.arange(drv.num_blocks))
    check_layers = (0, cfg.n_layers - 1)
    for _ in range(3):
        drv.step()
    torch.cuda.synchronize()
    before = {(l, w): drv.st.block_checksums(l, w, all_ids).cpu().numpy()
              for l in check_layers for w in (0, 1)}
    drv.step()  # the checked step
    torch.cuda.synchronize()
    tables, lens, blocks, offs = drv.last
    pb, po = drv.last_prompt
    assert len(pb) == drv.n_churn * 64
    # accounting
    owned = np.concatenate([drv.bm.table(int(s)) for s in drv.running])
    assert len(np.unique(owned)) == len(owned)
    assert drv.bm.available() + len(owned) == drv.num_blocks
    written = np.unique(np.concatenate([blocks, pb]))
    others = np.setdiff1d(np.arange(drv.num_blocks), written)
    for layer in check_layers:
        for which, src_new, src_prompt in ((0, drv.nk, drv.pk),
                                           (1, drv.nv, drv.pv)):
            after = drv.st.block_checksums(layer, which,
                                           all_ids).cpu().numpy()
            assert np.array_equal(after[others],
                                  before[(layer, which)][others])
            rows = drv.st.read_blocks(layer, which, dev_u32(written)) \
                .cpu().numpy().view(np.uint16)
            at = {int(b): i for i, b in enumerate(written)}
            want_dec = orc.f32_to_f16_bits(src_new[layer].cpu().numpy())
            got_dec = rows[[at[int(b)] for b in blocks], offs]
            assert np.array_equal(got_dec, want_dec)
            want_pr = orc.f32_to_f16_bits(
                src_prompt[layer].cpu().numpy()[:len(pb)])
            got_pr = rows[[at[int(b)] for b in pb], po]
            assert np.array_equal(got_pr, want_pr)
    sample = list(range(0, 1024, 64))
    layer = cfg.n_layers - 1
    bs = cfg.block_size
    cache, padded, mb = oracle_subset(
        drv.st, layer, [tables[b, :-(-int(lens[b]) // bs)] for b in sample],
        lens[sample])
    want = orc.paged_decode_f64(cache, drv.q[layer].cpu().numpy()[sample],
                                padded.reshape(-1), mb, lens[sample])
    got = drv.out[layer].cpu().numpy()[sample]
    assert np.abs(got - want).max() < ATOL
    drv.st.close()


# ---- full-size append / gather (size-independent checks) -------------------
def test_full_size_gather_llama_layer():
    """One full Llama-3.2-1B layer (8192 blocks, 64 x 2048): the padded
    gather equals the oracle's gather of the same cache bit for bit."""
    c = W.CONFIGS["llama-3.2-1b"]
    db = W.uniform_batch(c, 2048)
    st = HipKvStorage(1, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim)
    fill_layer(st, 0, seed=41)
    ids = dev_u32(np.arange(db.num_blocks))
    ref = orc.KvCache(db.num_blocks, c.block_size, c.n_kv_heads, c.head_dim,
                      orc.F16)
    ref.k[:] = bits(st.read_blocks(0, 0, ids))
    ref.v[:] = bits(st.read_blocks(0, 1, ids))
    plan = HipGatherPlan([(t, 2048) for t in db.tables])
    n = db.batch * c.n_kv_heads * 2048 * c.head_dim
    ok = torch.empty(n, dtype=torch.float16, device="cuda")
    ov = torch.empty(n, dtype=torch.float16, device="cuda")
    st.gather(0, plan, ok, ov)
    idx, mb, cl = orc.gather_plan(db.tables, db.ctx_lens)
    wk, wv = ref.gather(idx, db.batch, mb, cl)
    assert np.array_equal(bits(ok).reshape(wk.shape), orc.f32_to_f16_bits(wk))
    assert np.array_equal(bits(ov).reshape(wv.shape), orc.f32_to_f16_bits(wv))


def test_full_size_prefill_append_checksums():
    """Qwen3-0.6B prefill at full size for one layer (256 x 4096 tokens
    scattered through permuted tables, f32 source): per-block FNV-1a
    checksums computed on the GPU equal the oracle's for a seeded 2 %
    sample of blocks, plus every block of one sequence."""
    c = W.CONFIGS["qwen3-0.6b"]
    db = W.uniform_batch(c, 4096)
    bs = c.block_size
    st = HipKvStorage(1, db.num_blocks, bs, c.n_kv_heads, c.head_dim)
    sb = np.concatenate([np.repeat(t, bs) for t in db.tables])
    so = np.tile(np.arange(bs, dtype=np.uint32), db.num_blocks)
    g = torch.Generator("cuda").manual_seed(5)
    n_tok = sb.size
    k = torch.randn((n_tok, c.n_kv_heads, c.head_dim), generator=g,
                    device="cuda") * 0.5
    st.write_tokens(0, dev_u32(sb), dev_u32(so), k, k)
    rng = np.random.default_rng(6)
    blocks = np.unique(np.concatenate([
        rng.choice(db.num_blocks, db.num_blocks // 50, replace=False),
        db.tables[17]])).astype(np.uint32)
    got = st.block_checksums(0, 0, dev_u32(blocks)).cpu().numpy().view(
        np.uint64)
    # token rows that landed in each sampled block, in slot order
    tok_of = np.empty(db.num_blocks * bs, np.int64)
    tok_of[sb.astype(np.int64) * bs + so] = np.arange(n_tok)
    rows = tok_of[(blocks.astype(np.int64)[:, None] * bs +
                   np.arange(bs)).reshape(-1)]
    src = k[torch.from_numpy(rows).cuda()].cpu().numpy()
    ref = orc.KvCache(len(blocks), bs, c.n_kv_heads, c.head_dim, orc.F16)
    ref.k[:] = orc.f32_to_f16_bits(src).reshape(ref.k.shape)
    want = ref.checksums(0, np.arange(len(blocks)))
    assert np.array_equal(got, want)
    v_sum = st.block_checksums(0, 1, dev_u32(blocks)).cpu().numpy()
    assert np.array_equal(v_sum.view(np.uint64), want)  # k was used for v


# ---- HIP graph capture (serving loops) -------------------------------------
def test_graph_capture_replays_match_eager():
    """rvkv_decode_step (uniform) and rvkv_paged_decode_planned captured in a
    HIP graph: every replay, with eager work and new q values between
    replays, equals the eager result (the kernels record no memset)."""
    from rvllm_amd.kv_storage import HipDecodePlan
    bs, nkv, hd, H = 16, 4, 128, 8
    cfg = W.Config("gr", 9, 1, H, nkv, hd, bs, 6)
    lens = np.array([3000, 17, 900, 2048, 64, 700], np.uint32)
    db = W.ragged_batch(cfg, lens, seed=8)
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd)
    fill_layer(st, 0, seed=12)
    g = torch.Generator("cuda").manual_seed(9)
    nk = torch.randn(6, nkv, hd, device="cuda", generator=g)
    nv = torch.randn(6, nkv, hd, device="cuda", generator=g)
    q = torch.randn(6, H, hd, device="cuda", generator=g)
    sb, so = dev_u32(db.slot_block), dev_u32(db.slot_off)
    tables, ctx = dev_u32(db.padded_tables()), dev_u32(lens)
    max_ctx = int(lens.max())
    ws = st.alloc_workspace(6, H, max_ctx)
    plan = HipDecodePlan(st, lens, H)
    out_g1 = torch.empty_like(q)
    out_g2 = torch.empty_like(q)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        st.set_stream(side)
        st.decode_step(0, nk, nv, sb, so, q, tables, ctx, max_ctx,
                       out=out_g1, ws=ws)  # warm-up outside the graph
        st.paged_decode_planned(0, plan, q, tables, ctx, out=out_g2)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        st.set_stream(torch.cuda.current_stream())
        st.decode_step(0, nk, nv, sb, so, q, tables, ctx, max_ctx,
                       out=out_g1, ws=ws)
        st.paged_decode_planned(0, plan, q, tables, ctx, out=out_g2)
    st.set_stream(torch.cuda.current_stream())
    for rep in range(3):
        q.copy_(torch.randn(6, H, hd, device="cuda", generator=g))
        out_g1.zero_()
        out_g2.zero_()
        graph.replay()
        torch.cuda.synchronize()
        e1 = st.decode_step(0, nk, nv, sb, so, q, tables, ctx, max_ctx,
                            ws=st.alloc_workspace(6, H, max_ctx))
        e2 = st.paged_decode_planned(0, plan, q, tables, ctx)
        torch.cuda.synchronize()
        assert torch.equal(out_g1, e1), rep
        assert torch.equal(out_g2, e2), rep


# ---- attention prep + append -------------------------------------------
@pytest.mark.parametrize("hd,H,KV", [(64, 32, 8), (128, 16, 8), (256, 4, 1),
                                     (64, 14, 2), (32, 9, 1)])
@pytest.mark.parametrize("bias,norm", [(False, False), (True, False),
                                       (False, True), (True, True)])
def test_attn_prep_matches_oracle(hd, H, KV, bias, norm):
    """rvkv_attn_prep vs the oracle's restatement of src/model.rs:600-639.
    Without the RMS norm every f32 q and every f16 cache bit is identical
    (same unfused operations); with it the per-head sum of squares is
    reduced in a different order, so q agrees to 2e-6 * (1 + |q|) and cache
    values to one f16 ulp."""
    rng = np.random.default_rng(hd + H + 2 * bias + norm)
    rows, nb, bs = 37, 40, 16
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
    pos = rng.integers(0, 8192, rows)
    factors = (rng.uniform(1, 8, hd // 2).astype(np.float32)
               if hd == 64 else None)
    c, s = orc.rope_cos_sin(500000.0, hd, pos, factors=factors)
    slots = rng.permutation(nb * bs)[:rows]
    sb, so = slots // bs, slots % bs
    cache = orc.KvCache(nb, bs, KV, hd, orc.F16)
    want_q = orc.attn_prep(cache, q, k, v, c, s, sb, so, eps=1e-6, **opt)
    st = HipKvStorage(1, nb, bs, KV, hd)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    got_q = st.attn_prep(0, T(q), T(k), T(v), T(c), T(s), dev_u32(sb),
                         dev_u32(so), eps=1e-6,
                         **{n: T(a) for n, a in opt.items()}).cpu().numpy()
    ids = dev_u32(np.arange(nb))
    gk, gv = bits(st.read_blocks(0, 0, ids)), bits(st.read_blocks(0, 1, ids))
    assert np.array_equal(gv, cache.v)  # v: bias + RNE only
    if not norm:
        assert np.array_equal(got_q, want_q)
        assert np.array_equal(gk, cache.k)
    else:
        # RoPE's x0*c - x1*s cancels, so the bound is absolute, scaled by
        # the output's magnitude rather than relative to it.
        assert np.max(np.abs(got_q - want_q) / (1 + np.abs(want_q))) < 2e-6
        ulp = np.abs(gk.astype(np.int32) - cache.k.astype(np.int32))
        assert ulp.max() <= 1 and (ulp == 0).mean() > 0.99


def _prep_then_decode(st, q, k, v, c, s, sb, so, tables, lens, opt):
    """attn_prep over every prompt token, then one decode over the cache
    with each sequence's last q row (the prefill -> decode hand-off)."""
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    qo = st.attn_prep(0, T(q), T(k), T(v), T(c), T(s), dev_u32(sb),
                      dev_u32(so), eps=1e-6,
                      **{n: T(a) for n, a in opt.items()})
    last = torch.from_numpy(np.cumsum(lens.astype(np.int64)) - 1).cuda()
    out = st.paged_decode(0, qo[last].contiguous(), dev_u32(tables),
                          dev_u32(lens), int(lens.max()))
    return qo.cpu().numpy(), out.cpu().numpy()


@pytest.mark.parametrize("hd,H,KV", [(128, 16, 8), (64, 14, 2)])
def test_attn_prep_then_decode_end_to_end(hd, H, KV):
    """Prompt rows through rvkv_attn_prep, then rvkv_paged_decode, against
    the oracle's attn_prep + float64 paged decode (2e-3 max-abs), and the
    reference's qk_norm_cancels_the_scale_of_the_qk_projections
    (src/model.rs:1132-1162): with QK norm, scaling the q and k rows by 7
    leaves the attention output unchanged (1e-4 in the reference; here
    the f16 cache may round the renormalised k differently, so 2e-3)."""
    rng = np.random.default_rng(hd + H)
    bs, lens = 16, np.array([1, 17, 64, 200, 33], np.uint32)
    nseq, rows = len(lens), int(lens.sum())
    max_blocks = -(-int(lens.max()) // bs)
    nb = nseq * max_blocks + 3
    perm = rng.permutation(nb).astype(np.uint32)
    tables = perm[:nseq * max_blocks].reshape(nseq, max_blocks)
    pos = np.concatenate([np.arange(n) for n in lens])
    seq = np.repeat(np.arange(nseq), lens)
    sb, so = tables[seq, pos // bs], (pos % bs).astype(np.uint32)
    from rvllm_amd.rope import rope_cos_sin
    c, s = rope_cos_sin(1e6, hd, pos)
    q = rng.standard_normal((rows, H, hd)).astype(np.float32)
    k = rng.standard_normal((rows, KV, hd)).astype(np.float32)
    v = rng.standard_normal((rows, KV, hd)).astype(np.float32)
    opt = dict(q_norm=rng.uniform(0.5, 2, hd).astype(np.float32),
               k_norm=rng.uniform(0.5, 2, hd).astype(np.float32))
    st = HipKvStorage(1, nb, bs, KV, hd)
    qo, out = _prep_then_decode(st, q, k, v, c, s, sb, so, tables, lens, opt)
    cache = orc.KvCache(nb, bs, KV, hd, orc.F16)
    want_q = orc.attn_prep(cache, q, k, v, c, s, sb, so, eps=1e-6, **opt)
    want = orc.paged_decode_f64(cache, want_q[np.cumsum(lens) - 1], tables,
                                max_blocks, lens)
    assert np.max(np.abs(out - want)) < 2e-3
    st2 = HipKvStorage(1, nb, bs, KV, hd)
    _, out7 = _prep_then_decode(st2, q * 7, k * 7, v, c, s, sb, so, tables,
                                lens, opt)
    assert np.max(np.abs(out7 - out)) < 2e-3
    # Without the norms the same scaling sharpens attention.
    st3 = HipKvStorage(1, nb, bs, KV, hd)
    _, a = _prep_then_decode(st3, q, k, v, c, s, sb, so, tables, lens, {})
    _, b = _prep_then_decode(st3, q * 7, k * 7, v, c, s, sb, so, tables,
                             lens, {})
    assert np.max(np.abs(a - b)) > 1e-2


# ---- paged prefill / chunked-prefill attention -------------------------
@pytest.mark.parametrize("case", range(len(METAL_CASES)))
def test_prefill_metal_cases(golden, case):
    """The attn_decode cases of src/metal/ops.rs:676-766 with their own
    q_len (1, 1, 2, 2, 3, 1) through rvkv_paged_prefill (head_dim 6 and 200
    on the generic kernel): the Metal mask is
    batch_mask with pos_offset = valid - q_len, read_num = valid. Against
    the oracle over the same f16 cache and against the f32-cache golden."""
    c = metal_case_inputs(case)
    B, Q, H, D, bs = c["batch"], c["q_len"], c["n_heads"], c["hd"], c["bs"]
    st = HipKvStorage(1, c["num_blocks"], bs, c["n_kv"], D)
    nslot = c["num_blocks"] * bs
    slots = np.arange(nslot)
    kk = c["cache_k"].reshape(nslot, c["n_kv"], D)
    vv = c["cache_v"].reshape(nslot, c["n_kv"], D)
    st.write_tokens(0, dev_u32(slots // bs), dev_u32(slots % bs),
                    torch.from_numpy(kk).cuda(), torch.from_numpy(vv).cuda())
    valid = np.array([c["ctx"] - 2 * b for b in range(B)], np.uint32)
    q = c["q"].reshape(B, Q, H, D)
    tables = c["block_idx"].reshape(B, c["max_blocks"])
    out = st.paged_prefill(0, torch.from_numpy(q).cuda(), dev_u32(tables),
                           dev_u32(valid - Q), dev_u32(valid)).cpu().numpy()
    ref = orc.KvCache(c["num_blocks"], bs, c["n_kv"], D, orc.F16)
    ref.write_tokens(slots // bs, slots % bs, kk, vv)
    want = orc.paged_prefill_f64(ref, q, c["block_idx"], c["max_blocks"],
                                 valid - Q, valid)
    assert np.abs(out - want).max() < ATOL
    exp = np.array(golden["metal_attn_decode"][case]["expected"],
                   np.float32).reshape(B, Q, H, D)
    assert np.abs(out - exp).max() < ATOL


def _prefill_case(seed, B, Q, nkv, G, hd, bs, window, ragged=True,
                  prior=None, qscale=1.0):
    """A chunked-prefill batch over a random pool: sequence b already holds
    prior[b] tokens and appends a chunk of Q (pos_offset = prior[b]);
    read_num is prior + Q, or a little less/more when ragged (padding past
    read_num, rows that see fewer keys). Returns the GPU result and the
    oracle's."""
    rng = np.random.default_rng(seed)
    if prior is None:
        prior = rng.integers(0, 3 * Q + 1, B)
    prior = np.asarray(prior, np.int64)
    read = prior + Q
    if ragged:
        read = np.maximum(read + rng.integers(-3, 2, B), 0)
    mb = max(1, -(-int(max(read.max(), (prior + Q).max())) // bs))
    nb = B * mb + 5
    st = HipKvStorage(1, nb, bs, nkv, hd)
    fill_layer(st, 0, seed=seed)
    perm = rng.permutation(nb).astype(np.uint32)
    tables = perm[:B * mb].reshape(B, mb)
    q = (rng.standard_normal((B, Q, nkv * G, hd)) * qscale).astype(np.float32)
    out = st.paged_prefill(0, torch.from_numpy(q).cuda(), dev_u32(tables),
                           dev_u32(prior), dev_u32(read),
                           window=window).cpu().numpy()
    cache, padded, mbo = oracle_subset(st, 0, list(tables), read)
    want = orc.paged_prefill_f64(cache, q, padded, mbo, prior, read,
                                 window=window)
    return out, want


@pytest.mark.parametrize("G,hd,bs", [(1, 64, 16), (2, 128, 16), (4, 64, 32),
                                     (7, 64, 32), (8, 128, 8), (3, 32, 16),
                                     (16, 64, 16), (4, 256, 16), (1, 256, 8),
                                     (2, 256, 64), (4, 64, 128), (3, 32, 128),
                                     (2, 128, 128)])
def test_prefill_chunked_vs_oracle(G, hd, bs):
    """Several query-row tiles per (sequence, KV head) (G * Q > 128),
    chunk offsets that are not tile or block aligned, ragged read counts."""
    out, want = _prefill_case(G * 100 + hd, 3, 97, 2, G, hd, bs, 0)
    err = np.abs(out - want).max()
    assert np.isfinite(out).all() and err < ATOL, err


@pytest.mark.parametrize("case", range(16))
def test_prefill_random_shapes(case):
    """Seeded random prefill shapes on the tuned kernels: head_dim 32-256,
    block sizes 8-256, groups 1-8, chunk lengths 1-300 (one to several
    query tiles, partial last tiles), earlier context up to three chunks,
    ragged read counts, windows, and a sharper q on some cases; each
    against the float64 oracle."""
    rng = np.random.default_rng(9100 + case)
    hd = int(rng.choice([32, 64, 128, 256]))
    bs = int(rng.choice([8, 16, 32, 64, 128, 256]))
    G = int(rng.integers(1, 9))
    nkv = int(rng.integers(1, 3))
    B = int(rng.integers(1, 4))
    Q = int(rng.choice([1, 7, 64, 65, 129, 300]))
    window = int(rng.choice([0, 0, 5, 100]))
    qscale = float(rng.choice([1.0, 1.0, 6.0]))
    out, want = _prefill_case(9100 + case, B, Q, nkv, G, hd, bs, window,
                              qscale=qscale)
    assert np.isfinite(out).all()
    err = np.abs(out - want).max()
    assert err < ATOL, (case, hd, bs, G, nkv, B, Q, window, qscale, err)


@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("window", [1, 37, 300])
def test_prefill_window(window, hd):
    out, want = _prefill_case(window, 2, 200, 2, 4, hd, 16, window,
                              prior=[0, 333])
    assert np.abs(out - want).max() < ATOL


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_prefill_deterministic(hd):
    """Repeated launches on the same inputs are bitwise equal (the kernels
    use no atomics; a difference would mean a read of LDS or registers
    before their data is in place). 1000-token prompts: many tiles per
    workgroup, a partial last tile."""
    nb, bs, nkv, H = 200, 16, 2, 8
    st = HipKvStorage(1, nb, bs, nkv, hd)
    fill_layer(st, 0, seed=hd)
    rng = np.random.default_rng(hd)
    tables = dev_u32(rng.permutation(nb).astype(np.uint32)[:192].reshape(3, 64))
    q = torch.randn(3, 1000, H, hd, device="cuda")
    z, full = dev_u32([0, 0, 0]), dev_u32([1000, 1000, 1000])
    ref = st.paged_prefill(0, q, tables, z, full)
    for _ in range(6):
        assert torch.equal(st.paged_prefill(0, q, tables, z, full), ref)


@pytest.mark.parametrize("G,hd", [(4, 64), (7, 64), (2, 128), (4, 256)])
def test_decode_deterministic(G, hd):
    """The same for planned decode (split sequences, the reduction pass;
    the matrix-core kernel at G 7)."""
    nb, bs, nkv = 600, 16, 2
    H = G * nkv
    st = HipKvStorage(1, nb, bs, nkv, hd)
    fill_layer(st, 0, seed=G + hd)
    rng = np.random.default_rng(G + hd)
    lens = np.array([1, 37, 900, 4000, 2500], np.uint32)
    mb = 256
    tables = np.zeros((lens.size, mb), np.uint32)
    perm = rng.permutation(nb).astype(np.uint32)
    for i in range(lens.size):
        tables[i] = perm[(np.arange(mb) + 97 * i) % nb]
    q = torch.randn(lens.size, H, hd, device="cuda")
    plan = HipDecodePlan(st, lens, H)
    t, ln = dev_u32(tables), dev_u32(lens)
    ref = st.paged_decode_planned(0, plan, q, t, ln).clone()
    for _ in range(6):
        assert torch.equal(st.paged_decode_planned(0, plan, q, t, ln), ref)


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_prefill_large_scores(hd):
    """The same for prefill: q scaled by 16, several tiles per row."""
    out, want = _prefill_case(hd + 1, 2, 150, 2, 4, hd, 16, 0, qscale=16.0)
    assert np.isfinite(out).all() and np.abs(out - want).max() < ATOL


def test_prefill_full_prompt_from_empty():
    """Whole-prompt prefill (pos_offset 0, read_num = q_len), the
    reference's first forward of a sequence, at 1000 tokens."""
    out, want = _prefill_case(5, 2, 1000, 2, 2, 128, 16, 0, ragged=False,
                              prior=[0, 0])
    assert np.abs(out - want).max() < ATOL


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_prefill_edges(hd):
    """Rows that see no key (read_num <= pos_offset) are zero; q_len 1
    agrees with the decode kernel; an out-of-range table entry is read as
    masked, never faults, and leaves rows that do not reach it unchanged.
    (At head_dim 256 the wave pairs split the head dimension.)"""
    nb, bs, nkv, H = 40, 16, 2, 8
    st = HipKvStorage(1, nb, bs, nkv, hd)
    fill_layer(st, 0, seed=4)
    rng = np.random.default_rng(4)
    tables = rng.permutation(nb).astype(np.uint32)[:36].reshape(3, 12)
    q = torch.randn(3, 5, H, hd, device="cuda")
    off = dev_u32([10, 50, 0])
    read = dev_u32([0, 53, 0])  # seq 0 and 2 see nothing
    out = st.paged_prefill(0, q, dev_u32(tables), off, read)
    assert out[0].eq(0).all() and out[2].eq(0).all()
    assert (out[1].abs().sum(-1) > 0).all()  # rows past read_num see < 53
    # window 1: a row sees only its own position, absent past read_num
    w1 = st.paged_prefill(0, q, dev_u32(tables), off, read, window=1)
    assert (w1[1, :3].abs().sum(-1) > 0).all() and w1[1, 3:].eq(0).all()
    # q_len 1 == decode
    lens = np.array([1, 150, 192], np.uint32)
    q1 = torch.randn(3, 1, H, hd, device="cuda")
    a = st.paged_prefill(0, q1, dev_u32(tables), dev_u32(lens - 1),
                         dev_u32(lens))
    b = st.paged_decode(0, q1[:, 0].contiguous(), dev_u32(tables),
                        dev_u32(lens), 192)
    assert (a[:, 0] - b).abs().max().item() < 1e-3
    # a bad block id in the last block of sequence 2
    bad = tables.copy()
    bad[2, 11] = 10_000
    qq = torch.randn(3, 192, H, hd, device="cuda")
    z = dev_u32([0, 0, 0])
    full = dev_u32([192, 192, 192])
    good = st.paged_prefill(0, qq, dev_u32(tables), z, full)
    got = st.paged_prefill(0, qq, dev_u32(bad), z, full)
    assert torch.isfinite(got).all()
    assert torch.equal(got[:2], good[:2])
    assert torch.equal(got[2, :176], good[2, :176])
    # rows past the bad block see exactly keys 0..175: as if read_num = 176
    cut = st.paged_prefill(0, qq, dev_u32(tables), z, dev_u32([192, 192, 176]))
    assert (got[2, 176:] - cut[2, 176:]).abs().max().item() < 1e-6


def test_prefill_rejections():
    st = HipKvStorage(1, 4, 16, 2, 64)
    with pytest.raises(RvkvError, match="paged_prefill: n_heads"):
        st.paged_prefill(0, torch.zeros(1, 2, 3, 64, device="cuda"),
                         dev_u32([[0]]), dev_u32([0]), dev_u32([2]))


# ---- argmax and the engine over the paged KV path -------------------------
def test_argmax_kat_and_random():
    """rvkv_argmax: the reference KAT (src/cuda/ops.rs:1447-1477) and random
    rows with ties/NaN at vocab sizes that are and are not multiples of 4."""
    from rvllm_amd import _lib
    import ctypes
    from tests.test_oracle import argmax_kat_rows
    L = _lib.load()

    def gpu_argmax(x):
        t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
        out = torch.empty(x.shape[0], dtype=torch.int32, device="cuda")
        _lib.check(L.rvkv_argmax(ctypes.c_void_p(t.data_ptr()), x.shape[0],
                                 x.shape[1], ctypes.c_void_p(out.data_ptr()),
                                 ctypes.c_void_p(
                                     torch.cuda.current_stream().cuda_stream)))
        torch.cuda.synchronize()
        return out.cpu().numpy().view(np.uint32).tolist()

    assert gpu_argmax(argmax_kat_rows()) == [1, 1, 0, 599]
    rng = np.random.default_rng(31)
    for V in (1, 7, 1000, 32000, 151936):
        x = rng.integers(-5, 6, (33, V)).astype(np.float32)
        x[rng.random(x.shape) < 0.05] = np.nan
        x[3] = -np.inf
        assert gpu_argmax(x) == orc.argmax_rows(x).tolist(), V


def test_read_probe_runs_and_writes_nothing():
    """The bench's streaming-read probe (librvkv_calib.so) reads the
    buffer, leaves the sink alone, and rejects unaligned sizes."""
    from rvllm_amd import _lib
    import ctypes
    L = _lib.load_calib()
    buf = torch.arange(1 << 20, dtype=torch.int32, device="cuda")
    sink = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for wg in (0, 1, 3, 4096):
        _lib.check_calib(L.rvkv_calib_read_probe(
            ctypes.c_void_p(buf.data_ptr()), buf.numel() * 4, wg,
            ctypes.c_void_p(sink.data_ptr()), stream))
    torch.cuda.synchronize()
    assert sink.item() == 7
    with pytest.raises(RvkvError, match="read_probe: buf and bytes"):
        _lib.check_calib(L.rvkv_calib_read_probe(
            ctypes.c_void_p(buf.data_ptr()), 20, 0, None, stream))


def _engine_pair(cfg, num_blocks, bs):
    from rvllm_amd.attn_model import HipBackend, init_weights
    from tests.engine_backends import LockstepBackend, OracleBackend
    w = init_weights(cfg)
    return LockstepBackend(HipBackend(cfg, w, num_blocks, bs),
                           OracleBackend(cfg, w, num_blocks, bs))


@pytest.mark.parametrize("variant", ["plain", "qwen3", "qwen25", "window"])
def test_engine_lockstep_with_oracle(variant):
    """The engine over the native scheduler with the GPU backend: every
    prefill and decode forward (attn_prep + append, paged prefill, paged
    decode, argmax) agrees with the oracle's computation of the same model;
    requests share prefixes (prefix-cache hits skip their tokens) and the
    pool is small enough to force preemption and re-prefill."""
    from rvllm_amd.attn_model import AttnModelConfig
    from rvllm_amd.engine import Engine, EngineConfig, Request
    cfg = AttnModelConfig(
        vocab=512, hidden=128, n_layers=2, n_heads=8, n_kv_heads=2,
        head_dim=64, qkv_bias=variant == "qwen25",
        qk_norm=variant == "qwen3", context_length=512,
        window=24 if variant == "window" else 0)
    be = _engine_pair(cfg, num_blocks=14, bs=16)  # tight: preempts twice
    eng = Engine(be, EngineConfig(block_size=16, num_blocks=14,
                                  max_running=6))
    rng = np.random.default_rng(5)
    shared = rng.integers(0, 512, 40).tolist()
    ids = []
    for i in range(7):
        prompt = (shared if i % 2 == 0 else []) + rng.integers(
            0, 512, int(rng.integers(3, 30))).tolist()
        ids.append(eng.add_request(Request(prompt, int(rng.integers(8, 40)))))
    while eng.has_work():
        eng.step()
    hits, total, pre = eng.scheduler.metrics()
    print(f"forwards {be.calls} worst/tol {be.worst:.3f} hits {hits}/{total} "
          f"preemptions {pre} close {be.close_calls}")
    assert hits > 0 and pre > 0 and be.calls > 20
    assert eng.scheduler.available() == 14


def test_engine_fork_copy_on_write_on_gpu():
    """A forked sequence shares its parent's half-full tail block; the
    first step copies it (rvkv_copy_blocks) before either writes, and both
    continue to agree with the oracle."""
    from rvllm_amd.attn_model import AttnModelConfig
    from rvllm_amd.engine import Engine, EngineConfig, Request
    cfg = AttnModelConfig(vocab=256, hidden=128, n_layers=2, n_heads=4,
                          n_kv_heads=2, head_dim=64, context_length=256)
    be = _engine_pair(cfg, num_blocks=16, bs=8)
    eng = Engine(be, EngineConfig(block_size=8, num_blocks=16))
    a = eng.add_request(Request(list(range(20, 33)), 6))
    eng.step()  # prefill + one decode
    b = eng.scheduler.fork(a)
    eng.seqs[b] = type(eng.seqs[a])(**vars(eng.seqs[a]))
    while eng.has_work():
        eng.step()
    assert be.calls > 5


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("hd,bias_on,qn_on,kn_on", [(64, True, True, True),
                                                    (128, False, False, False),
                                                    (6, True, False, True),
                                                    (2, False, True, False)])
def test_attn_prep_qkv_metal_cases(hd, bias_on, qn_on, kn_on, dtype):
    """attn_prep_matches_reference (src/metal/ops.rs:771-858) through the
    fused-QKV entry point: 6 q / 2 kv heads, 5 rows, xorshift values (seeds
    40-45), row r to (block r % 3 + 1, offset r % 4), eps 1e-5. The expected
    values are computed as that test computes them (rms in float64, the
    rotate-half in f32); q within its 1e-5, the f16 cache equal to the
    expected f32 rounded to f16 (one ulp where the norm's sum order shows);
    on an f32 pool (the reference's cells) v exactly and k within 1e-5.
    Head widths 6 and 2 run the generic kernel."""
    from tests.golden.make_golden import values
    H, KV, rows, bs = 6, 2, 5, 4
    width = (H + 2 * KV) * hd
    half, eps = hd // 2, np.float32(1e-5)
    qkv = values(rows * width, 40).reshape(rows, width)
    bias, qn, kn = values(width, 41), values(hd, 42), values(hd, 43)
    cos = values(rows * half, 44).reshape(rows, half)
    sin = values(rows * half, 45).reshape(rows, half)
    blk = np.arange(rows, dtype=np.uint32) % 3 + 1
    off = np.arange(rows, dtype=np.uint32) % bs

    def head(r, slot):
        x = qkv[r, slot * hd:(slot + 1) * hd]
        return (x + bias[slot * hd:(slot + 1) * hd]) if bias_on else x.copy()

    def rotate(r, x, w):
        if w is not None:
            ms = np.sum(x.astype(np.float64) ** 2) / hd
            rms = np.float32(np.sqrt(ms + np.float64(eps)))
            x = (x / rms) * w
        c, s = cos[r], sin[r]
        return np.concatenate([x[:half] * c - x[half:] * s,
                               x[:half] * s + x[half:] * c]).astype(np.float32)

    want_q = np.stack([[rotate(r, head(r, h), qn if qn_on else None)
                        for h in range(H)] for r in range(rows)])
    want_k = np.zeros((4, bs, KV, hd), np.float32)
    want_v = np.zeros_like(want_k)
    for r in range(rows):
        for h in range(KV):
            want_k[blk[r], off[r], h] = rotate(r, head(r, H + h),
                                               kn if kn_on else None)
            want_v[blk[r], off[r], h] = head(r, H + KV + h)
    st = HipKvStorage(1, 4, bs, KV, hd, dtype=dtype)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    q = st.attn_prep_qkv(0, T(qkv), H, T(cos), T(sin), dev_u32(blk),
                         dev_u32(off), bias=T(bias) if bias_on else None,
                         q_norm=T(qn) if qn_on else None,
                         k_norm=T(kn) if kn_on else None, eps=1e-5)
    assert np.abs(q.cpu().numpy() - want_q).max() < 1e-5
    ids = dev_u32(np.arange(4))
    if dtype == torch.float32:
        gk = st.read_blocks(0, 0, ids).cpu().numpy()
        gv = st.read_blocks(0, 1, ids).cpu().numpy()
        assert np.array_equal(gv, want_v)
        assert np.abs(gk - want_k).max() < 1e-5
        return
    gk, gv = bits(st.read_blocks(0, 0, ids)), bits(st.read_blocks(0, 1, ids))
    assert np.array_equal(gv, orc.f32_to_f16_bits(want_v))
    d = np.abs(gk.astype(np.int32) - orc.f32_to_f16_bits(want_k).astype(
        np.int32))
    assert d.max() <= (1 if kn_on else 0)


def test_attn_prep_qkv_equals_split_entry_point():
    """The fused-QKV entry point and the split one give identical bits."""
    rng = np.random.default_rng(44)
    H, KV, hd, rows, nb, bs = 16, 8, 128, 50, 20, 16
    width = (H + 2 * KV) * hd
    qkv = rng.standard_normal((rows, width)).astype(np.float32)
    bias = rng.standard_normal(width).astype(np.float32)
    qn, kn = (rng.standard_normal(hd).astype(np.float32) for _ in range(2))
    from rvllm_amd.rope import rope_cos_sin
    c, s = rope_cos_sin(1e6, hd, rng.integers(0, 4096, rows))
    slots = rng.permutation(nb * bs)[:rows]
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    a = HipKvStorage(1, nb, bs, KV, hd)
    b = HipKvStorage(1, nb, bs, KV, hd)
    qa = a.attn_prep_qkv(0, T(qkv), H, T(c), T(s), dev_u32(slots // bs),
                         dev_u32(slots % bs), bias=T(bias), q_norm=T(qn),
                         k_norm=T(kn), eps=1e-6)
    qb = b.attn_prep(0, T(qkv[:, :H * hd].reshape(rows, H, hd)),
                     T(qkv[:, H * hd:(H + KV) * hd].reshape(rows, KV, hd)),
                     T(qkv[:, (H + KV) * hd:].reshape(rows, KV, hd)), T(c),
                     T(s), dev_u32(slots // bs), dev_u32(slots % bs),
                     q_bias=T(bias[:H * hd]),
                     k_bias=T(bias[H * hd:(H + KV) * hd]),
                     v_bias=T(bias[(H + KV) * hd:]), q_norm=T(qn),
                     k_norm=T(kn), eps=1e-6)
    assert torch.equal(qa, qb)
    ids = dev_u32(np.arange(nb))
    for w in (0, 1):
        assert torch.equal(a.read_blocks(0, w, ids), b.read_blocks(0, w, ids))


def test_graph_capture_prep_prefill_argmax():
    """rvkv_attn_prep_qkv (QK norm, bias) -> rvkv_paged_prefill ->
    rvkv_argmax captured in one HIP graph: on every replay, with new QKV
    input between replays, the graph's q, attention output, picked ids and
    cache bits equal an eager run of the same calls on a twin pool."""
    import ctypes
    from rvllm_amd import _lib
    from rvllm_amd.rope import rope_cos_sin
    L = _lib.load()
    H, KV, hd, bs, nb = 8, 2, 64, 16, 12
    rows, off = 40, 7  # a 40-token chunk after 7 cached tokens
    width = (H + 2 * KV) * hd
    g = torch.Generator("cuda").manual_seed(3)
    rnd = lambda *s: torch.randn(*s, device="cuda", generator=g)
    bias, qn, kn = rnd(width), rnd(hd), rnd(hd)
    c, s = (torch.from_numpy(a).cuda()
            for a in rope_cos_sin(1e4, hd, np.arange(off, off + rows)))
    table = np.random.default_rng(3).permutation(nb).astype(np.uint32)
    pos = np.arange(off, off + rows)
    sb, so = dev_u32(table[pos // bs]), dev_u32(pos % bs)
    tables = dev_u32(table[None, :])
    offs, reads = dev_u32([off]), dev_u32([off + rows])
    pools = [HipKvStorage(1, nb, bs, KV, hd) for _ in range(2)]
    for p in pools:  # the same cached prefix in both
        fill_layer(p, 0, seed=4)
    qkv = rnd(rows, width)
    outs = [dict(q=torch.empty(rows, H, hd, device="cuda"),
                 att=torch.empty(1, rows, H, hd, device="cuda"),
                 ids=torch.empty(rows, dtype=torch.int32, device="cuda"))
            for _ in range(2)]

    def forward(p, o):
        p.attn_prep_qkv(0, qkv, H, c, s, sb, so, bias=bias, q_norm=qn,
                        k_norm=kn, eps=1e-6, q_out=o["q"])
        p.paged_prefill(0, o["q"].view(1, rows, H, hd), tables, offs, reads,
                        out=o["att"])
        _lib.check(L.rvkv_argmax(
            ctypes.c_void_p(o["att"].data_ptr()), rows, H * hd,
            ctypes.c_void_p(o["ids"].data_ptr()),
            ctypes.c_void_p(p.stream.cuda_stream)))

    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pools[0].set_stream(side)
        forward(pools[0], outs[0])  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pools[0].set_stream(torch.cuda.current_stream())
        forward(pools[0], outs[0])
    pools[0].set_stream(torch.cuda.current_stream())
    ids = dev_u32(np.arange(nb))
    for rep in range(3):
        qkv.copy_(rnd(rows, width))
        for v in outs[0].values():
            v.zero_()
        graph.replay()
        torch.cuda.synchronize()
        forward(pools[1], outs[1])
        torch.cuda.synchronize()
        for k in ("q", "att", "ids"):
            assert torch.equal(outs[0][k], outs[1][k]), (rep, k)
        for w in (0, 1):
            assert torch.equal(pools[0].read_blocks(0, w, ids),
                               pools[1].read_blocks(0, w, ids)), (rep, w)
