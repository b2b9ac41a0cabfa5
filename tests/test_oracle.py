"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Each check is chosen so a plausible mistake (dropped term, wrong index,
transposed operand, wrong rounding) fails it: the reference's own known
answers (tests/golden/kats.json), numpy's float16 conversion, an
independent float64 brute force, torch's CPU scaled_dot_product_attention,
and invariants.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.golden.make_golden import metal_case_inputs


# ---- f32 -> f16 round to nearest even ------------------------------------
def test_f16_matches_numpy_on_random_and_edge_values():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * 3,
        (rng.standard_normal(50_000) * 1e-5).astype(np.float32),  # subnormals
        (rng.standard_normal(50_000) * 7e4).astype(np.float32),   # overflow
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, -65520.0, 6.1e-5,
                  5.96e-8, 2.98e-8, 2.9802322e-08, 2.9802326e-08,
                  np.inf, -np.inf, 1.0 + 2**-11, 1.0 + 3 * 2**-11,
                  2**-24 * 1.5, 2**-24 * 0.5, 2**-25 * 1.0000001],
                 dtype=np.float32),
    ])
    got = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):  # the overflow cases round to inf
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_ties_round_to_even():
    # 1 + 2^-11 is exactly half-way between 1 and 1 + 2^-10: even is 1.
    assert orc.f32_to_f16_bits(np.float32(1 + 2**-11)) == 0x3C00
    # 1 + 3*2^-11 is half-way between 1+2^-10 and 1+2^-9: even is 1+2^-9.
    assert orc.f32_to_f16_bits(np.float32(1 + 3 * 2**-11)) == 0x3C02
    # half of the smallest subnormal rounds to zero (even).
    assert orc.f32_to_f16_bits(np.float32(2**-25)) == 0x0000
    assert orc.f32_to_f16_bits(np.float32(-2**-25)) == 0x8000


def test_f16_nan_stays_nan_and_all_f16_values_round_trip():
    nan = orc.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert np.isnan(nan.view(np.float16)).all()
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = orc.f16_bits_to_f32(allbits)
    ref = allbits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(f[finite], ref[finite])
    assert np.array_equal(np.isnan(f), np.isnan(ref))
    back = orc.f32_to_f16_bits(f[finite])
    assert np.array_equal(back, allbits[finite])


# ---- append / gather: the reference KATs ---------------------------------
@pytest.mark.parametrize("dtype", [orc.F32, orc.F16])
def test_round_trip_across_blocks_kat(golden, dtype):
    g = golden["reference_kats"]["round_trip_across_blocks"]
    c = orc.KvCache(g["num_blocks"], g["block_size"], g["n_kv"], g["hd"],
                    dtype)
    k = np.array(g["k"], np.float32).reshape(-1, 1, 2)
    c.write_tokens(g["block_ids"], g["offsets"], k, k)
    assert np.array_equal(c.as_f32(0).reshape(-1), g["raw_cache"])
    idx, mb, cl = orc.gather_plan(g["tables"], g["n_tokens"])
    assert idx.tolist() == g["plan_block_idx"] and cl == g["ctx_len"]
    gk, gv = c.gather(idx, 2, mb, cl)
    assert gk.shape == (2, 1, 3, 2)
    assert np.array_equal(gk, gv)
    flat = gk.reshape(-1)
    assert flat[:6].tolist() == g["gather_prefix_a"]
    assert flat[6:8].tolist() == g["gather_prefix_b"]


def test_untouched_slots_kat(golden):
    g = golden["reference_kats"]["untouched_slots"]
    c = orc.KvCache(1, 4, 1, 2, orc.F32)
    t = np.array(g["k"], np.float32).reshape(1, 1, 2)
    c.write_tokens(g["block_ids"], g["offsets"], t, t)
    idx, mb, cl = orc.gather_plan(g["tables"], g["n_tokens"])
    gk, _ = c.gather(idx, 1, mb, cl)
    assert gk.reshape(-1).tolist() == g["gather"]


def test_clone_independence_kat(golden):
    g = golden["reference_kats"]["clone_independence"]
    orig = orc.KvCache(1, 2, 1, 2, orc.F32)
    snap_k = orig.k.copy()
    t = np.array(g["k"], np.float32).reshape(1, 1, 2)
    orig.write_tokens([0], [0], t, t)
    assert orig.k.reshape(-1)[:2].tolist() == g["after_write"]
    assert snap_k.reshape(-1)[:2].tolist() == g["snapshot"]


def test_write_tokens_runs_equal_per_token_scatter():
    """Run-coalesced write (src/kv_storage.rs:126-148) == the per-scalar
    index formula of kv_write.cu:17-31, on a random slot list mixing runs,
    breaks and out-of-order slots."""
    rng = np.random.default_rng(3)
    nb, bs, nkv, hd = 9, 4, 3, 5
    slots = rng.permutation(nb * bs)[:20]
    slots[5:9] = slots[4] + np.arange(1, 5)  # a run (may cross a block)
    slots = np.unique(slots)[:16]
    rng.shuffle(slots)
    blocks, offs = slots // bs, slots % bs
    ok = offs + 0 < bs
    blocks, offs = blocks[ok], offs[ok]
    k = rng.standard_normal((len(blocks), nkv, hd)).astype(np.float32)
    c = orc.KvCache(nb, bs, nkv, hd, orc.F32)
    c.write_tokens(blocks, offs, k, -k)
    want = np.zeros(nb * bs * nkv * hd, np.float32)
    for t in range(len(blocks)):
        for h in range(nkv):
            for d in range(hd):
                dest = ((blocks[t] * bs + offs[t]) * nkv + h) * hd + d
                want[dest] = k[t, h, d]
    assert np.array_equal(c.k.reshape(-1), want)
    assert np.array_equal(c.v.reshape(-1), -want)


def test_gather_matches_brute_force_formula():
    rng = np.random.default_rng(4)
    nb, bs, nkv, hd = 12, 4, 2, 3
    c = orc.KvCache(nb, bs, nkv, hd, orc.F16)
    c.k[:] = orc.f32_to_f16_bits(rng.standard_normal(c.k.shape))
    c.v[:] = orc.f32_to_f16_bits(rng.standard_normal(c.v.shape))
    tables = [[3, 7, 1], [0], [11, 2]]
    ntok = [10, 3, 6]
    idx, mb, cl = orc.gather_plan(tables, ntok)
    gk, gv = c.gather(idx, 3, mb, cl)
    kf, vf = c.as_f32(0), c.as_f32(1)
    for b in range(3):
        for h in range(nkv):
            for p in range(cl):
                blk = idx[b * mb + p // bs]
                assert np.array_equal(gk[b, h, p], kf[blk, p % bs, h])
                assert np.array_equal(gv[b, h, p], vf[blk, p % bs, h])


# ---- mask / attention ----------------------------------------------------
def test_mask_window_kat(golden):
    g = golden["reference_kats"]["mask_window"]
    m = orc.batch_mask(g["position_offset"], g["read_num_tokens"], g["q_len"],
                       g["ctx_len"], g["window"])
    want = np.array([[-np.inf if x == "-inf" else 0.0 for x in r]
                     for r in g["expected"]], np.float32)
    assert np.array_equal(m.reshape(4, 4), want)


def test_decode_mask_reduces_to_ctx_len_bound():
    """For q_len 1 at offset = read_num_tokens - 1 the causal term is
    redundant: mask == (j >= ctx_len) (what the HIP decode kernel uses)."""
    rn = [5, 1, 9, 3]
    m = orc.batch_mask([n - 1 for n in rn], rn, 1, 9)
    for b, n in enumerate(rn):
        row = m[b, 0, 0]
        assert np.all(row[:n] == 0) and np.all(np.isneginf(row[n:]))


def test_gqa_hand_computed_kat(golden):
    g = golden["reference_kats"]["gqa_hand_computed"]
    q = np.array(g["q"], np.float32).reshape(1, 2, 2, 2)
    k = np.array(g["k"], np.float32).reshape(1, 1, 2, 2)
    v = np.array(g["v"], np.float32).reshape(1, 1, 2, 2)
    m = orc.batch_mask(g["position_offset"], g["read_num_tokens"], 2, 2)
    out = orc.gqa_attention(q, k, v, m).reshape(-1)
    assert np.max(np.abs(out - np.array(g["expected"]))) < g["tol"]


def _torch_sdpa(q, k, v, mask):
    """torch CPU SDPA in float64 with GQA expanded by repeat_interleave."""
    q, k, v = (torch.from_numpy(np.asarray(x, np.float64)) for x in (q, k, v))
    group = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(group, dim=1)
    v = v.repeat_interleave(group, dim=1)
    m = torch.from_numpy(np.asarray(mask, np.float64))
    return torch.nn.functional.scaled_dot_product_attention(
        q, k, v, attn_mask=m).numpy()


def test_gqa_matches_naive_per_head_and_torch(golden):
    g = golden["reference_kats"]["naive_per_head_shape"]
    rng = np.random.default_rng(5)
    B, H, KV, Q, C, D = (g["batch"], g["n_heads"], g["n_kv"], g["q_len"],
                         g["ctx_len"], g["hd"])
    q = rng.standard_normal((B, H, Q, D)).astype(np.float32)
    k = rng.standard_normal((B, KV, C, D)).astype(np.float32)
    v = rng.standard_normal((B, KV, C, D)).astype(np.float32)
    m = orc.batch_mask(g["position_offset"], g["read_num_tokens"], Q, C)
    out = orc.gqa_attention(q, k, v, m)
    group = H // KV
    for b in range(B):  # naive per-head, as src/model.rs:929-949
        for h in range(H):
            s = q[b, h] @ k[b, h // group].T / math.sqrt(D) + m[b, 0]
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            assert np.max(np.abs(out[b, h] - p @ v[b, h // group])) < g["tol"]
    assert np.max(np.abs(out - _torch_sdpa(q, k, v, m))) < 1e-5


@pytest.mark.parametrize("case", range(6))
def test_metal_cases_f32_pipeline_matches_f64_golden(golden, case):
    """The reference pipeline (padded gather + batch mask + gqa_attention)
    on the six attn_decode cases of src/metal/ops.rs:676-766 reproduces the
    float64 expectations within that test's 1e-4."""
    c = metal_case_inputs(case)
    exp = np.array(golden["metal_attn_decode"][case]["expected"], np.float32)
    cache = orc.KvCache(c["num_blocks"], c["bs"], c["n_kv"], c["hd"], orc.F32)
    cache.k[:] = c["cache_k"]
    cache.v[:] = c["cache_v"]
    B, Q, H, D = c["batch"], c["q_len"], c["n_heads"], c["hd"]
    gk, gv = cache.gather(c["block_idx"], B, c["max_blocks"], c["ctx"])
    q = c["q"].reshape(B, Q, H, D).transpose(0, 2, 1, 3).copy()
    mask = c["mask"].reshape(B, 1, Q, c["ctx"])
    out = orc.gqa_attention(q, gk, gv, mask)  # [B, H, Q, D]
    got = out.transpose(0, 2, 1, 3).reshape(-1)
    assert np.max(np.abs(got - exp)) < golden["metal_attn_decode"][case]["tol"]
    # torch's SDPA (float64) agrees with the golden too.
    ref = _torch_sdpa(q, gk, gv, mask).transpose(0, 2, 1, 3).reshape(-1)
    assert np.max(np.abs(ref - exp)) < 1e-6


@pytest.mark.parametrize("case", [0, 1, 5])
def test_paged_decode_f64_matches_golden(golden, case):
    """The oracle's direct float64 paged attention reproduces the golden on
    the q_len == 1 cases (decode)."""
    c = metal_case_inputs(case)
    exp = np.array(golden["metal_attn_decode"][case]["expected"], np.float32)
    cache = orc.KvCache(c["num_blocks"], c["bs"], c["n_kv"], c["hd"], orc.F32)
    cache.k[:] = c["cache_k"]
    cache.v[:] = c["cache_v"]
    B, H, D = c["batch"], c["n_heads"], c["hd"]
    ctx = np.array([c["ctx"] - 2 * b for b in range(B)], np.uint32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = orc.paged_decode_f64(cache, c["q"].reshape(B, H, D),
                               c["block_idx"], c["max_blocks"], ctx,
                               scale=scale)
    assert np.max(np.abs(out.reshape(-1) - exp)) < 1e-6


def test_paged_decode_f64_window_matches_masked_sdpa():
    rng = np.random.default_rng(6)
    nb, bs, nkv, hd, H, B = 40, 16, 2, 32, 6, 3
    cache = orc.KvCache(nb, bs, nkv, hd, orc.F16)
    cache.k[:] = orc.f32_to_f16_bits(rng.standard_normal(cache.k.shape))
    cache.v[:] = orc.f32_to_f16_bits(rng.standard_normal(cache.v.shape))
    ctx = np.array([100, 37, 160], np.uint32)
    perm = rng.permutation(nb).astype(np.uint32)
    tables = np.stack([perm[0:10], perm[10:20], perm[20:30]])
    q = rng.standard_normal((B, H, hd)).astype(np.float32)
    for window in (0, 50):
        out = orc.paged_decode_f64(cache, q, tables.reshape(-1), 10, ctx,
                                   window=window)
        idx = tables.reshape(-1)
        gk, gv = cache.gather(idx, B, 10, 160)
        m = orc.batch_mask(ctx - 1, ctx, 1, 160, window)
        ref = _torch_sdpa(q[:, :, None], gk, gv, m)[:, :, 0]
        assert np.max(np.abs(out - ref)) < 1e-5


@pytest.mark.parametrize("dt", [orc.F16, orc.F32])
def test_decode_step_matches_f64(dt):
    """orc_decode_step (append + padded gather + mask + gqa in f32, the CPU
    baseline) against the float64 paged reference, multi-threaded, over f16
    cells and over the reference's f32 cells."""
    rng = np.random.default_rng(7)
    nb, bs, nkv, hd, H = 64, 16, 2, 64, 6
    cache = orc.KvCache(nb, bs, nkv, hd, dt)
    cache.write_tokens(np.repeat(np.arange(nb), bs), np.tile(np.arange(bs), nb),
                       rng.standard_normal((nb * bs, nkv, hd)),
                       rng.standard_normal((nb * bs, nkv, hd)))
    ctx = np.array([33, 200, 17, 128], np.uint32)
    perm = rng.permutation(nb).astype(np.uint32)
    tables = [perm[i * 16:(i + 1) * 16] for i in range(4)]
    idx, mb, _ = orc.gather_plan(tables, ctx)
    sb = np.array([t[(n - 1) // bs] for t, n in zip(tables, ctx)], np.uint32)
    so = (ctx - 1) % bs
    nk = rng.standard_normal((4, nkv, hd)).astype(np.float32)
    nv = rng.standard_normal((4, nkv, hd)).astype(np.float32)
    q = rng.standard_normal((4, H, hd)).astype(np.float32)
    ref_cache = orc.KvCache(nb, bs, nkv, hd, dt)
    ref_cache.k[:] = cache.k
    ref_cache.v[:] = cache.v
    ref_cache.write_tokens(sb, so, nk, nv)
    out = orc.decode_step(cache, sb, so, nk, nv, idx, mb, ctx, q, n_threads=3)
    assert np.array_equal(cache.k, ref_cache.k)
    want = orc.paged_decode_f64(ref_cache, q, idx, mb, ctx)
    assert np.max(np.abs(out - want)) < 2e-5


# ---- copy-on-write and checksums (parity unpinned: invariants) -----------
def test_copy_blocks_invariants():
    rng = np.random.default_rng(8)
    c = orc.KvCache(10, 4, 2, 8, orc.F16)
    c.k[:] = orc.f32_to_f16_bits(rng.standard_normal(c.k.shape))
    c.v[:] = orc.f32_to_f16_bits(rng.standard_normal(c.v.shape))
    before_k, before_v = c.k.copy(), c.v.copy()
    c.copy_blocks([1, 4, 7], [9, 0, 5])
    for s, d in ((1, 9), (4, 0), (7, 5)):
        assert np.array_equal(c.k[d], before_k[s])
        assert np.array_equal(c.v[d], before_v[s])
    for b in (1, 2, 3, 4, 6, 7, 8):
        assert np.array_equal(c.k[b], before_k[b])


def _fnv1a64(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for byte in data:
        h = ((h ^ byte) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_block_checksums_match_independent_fnv():
    rng = np.random.default_rng(9)
    c = orc.KvCache(6, 2, 2, 4, orc.F16)
    c.k[:] = rng.integers(0, 65536, c.k.shape, dtype=np.uint16)
    got = c.checksums(0, [5, 0, 3])
    for i, b in enumerate([5, 0, 3]):
        assert int(got[i]) == _fnv1a64(c.k[b].astype("<u2").tobytes())
    # f32 cells hash their little-endian bytes in logical order
    f = orc.KvCache(5, 2, 3, 4, orc.F32)
    f.v[:] = rng.standard_normal(f.v.shape).astype(np.float32)
    got = f.checksums(1, [4, 1])
    for i, b in enumerate([4, 1]):
        assert int(got[i]) == _fnv1a64(f.v[b].astype("<f4").tobytes())


# ---- RMS norm / RoPE / attention prep ---------------------------------
def test_rms_norm_kat():
    """src/model.rs:758-776: x = [1, 2, 3], w = 1, eps 1e-5."""
    out = orc.rms_norm([[1.0, 2.0, 3.0]], [1.0, 1.0, 1.0], 1e-5)
    assert np.max(np.abs(out - [0.46292, 0.92583, 1.38875])) < 1e-4


def test_rope_kats():
    """src/model.rs:778-823: position 0 is the identity; position 1 with
    theta [1, 0.01] rotates the rotate-half pairs (x0, x2), (x1, x3);
    Llama-3 factors divide each pair's frequency."""
    c, s = orc.rope_cos_sin(10000.0, 4, [0, 1])
    x = np.array([[1, 2, 3, 4], [1, 1, 0, 0]], np.float32)
    out = orc.rope_apply(x, c, s)
    assert np.max(np.abs(out[0] - [1, 2, 3, 4])) < 1e-4
    want = [np.cos(1.0), np.cos(0.01), np.sin(1.0), np.sin(0.01)]
    assert np.max(np.abs(out[1] - want)) < 1e-4
    c, s = orc.rope_cos_sin(10000.0, 4, [1], factors=[2.0, 4.0])
    assert np.max(np.abs(c[0] - np.cos([0.5, 0.0025]))) < 1e-6
    assert np.max(np.abs(s[0] - np.sin([0.5, 0.0025]))) < 1e-6


def test_rope_is_a_relative_position_rotation():
    """RoPE invariants: every rotate-half pair keeps its length, and
    <rope(q, m), rope(k, n)> depends only on m - n."""
    rng = np.random.default_rng(12)
    hd = 64
    q = rng.standard_normal((1, hd)).astype(np.float32)
    k = rng.standard_normal((1, hd)).astype(np.float32)
    c, s = orc.rope_cos_sin(10000.0, hd, [5, 2, 105, 102])
    rq = [orc.rope_apply(q, c[i:i + 1], s[i:i + 1]) for i in (0, 2)]
    rk = [orc.rope_apply(k, c[i:i + 1], s[i:i + 1]) for i in (1, 3)]
    half = hd // 2
    for r in rq:
        assert np.allclose(r[0, :half] ** 2 + r[0, half:] ** 2,
                           q[0, :half] ** 2 + q[0, half:] ** 2, rtol=1e-5)
    assert abs(float((rq[0] @ rk[0].T)[0, 0]) -
               float((rq[1] @ rk[1].T)[0, 0])) < 1e-4


def test_attn_prep_composes_the_pinned_parts():
    """orc_attn_prep = bias add, then rms_norm (q, k only), then rope_apply
    (q, k only), then the f16 write at each row's slot (v: bias only)."""
    rng = np.random.default_rng(13)
    rows, H, KV, hd, nb, bs = 5, 6, 2, 16, 8, 4
    q = rng.standard_normal((rows, H, hd)).astype(np.float32)
    k = rng.standard_normal((rows, KV, hd)).astype(np.float32)
    v = rng.standard_normal((rows, KV, hd)).astype(np.float32)
    qb = rng.standard_normal(H * hd).astype(np.float32)
    kb = rng.standard_normal(KV * hd).astype(np.float32)
    vb = rng.standard_normal(KV * hd).astype(np.float32)
    qn = rng.standard_normal(hd).astype(np.float32)
    kn = rng.standard_normal(hd).astype(np.float32)
    c, s = orc.rope_cos_sin(1e4, hd, [3, 9, 0, 40, 7])
    sb, so = [1, 4, 4, 7, 0], [2, 0, 3, 1, 3]
    cache = orc.KvCache(nb, bs, KV, hd, orc.F16)
    qo = orc.attn_prep(cache, q, k, v, c, s, sb, so, qb, kb, vb, qn, kn, 1e-6)
    for r in range(rows):
        for h in range(H):
            x = q[r, h] + qb[h * hd:(h + 1) * hd]
            x = orc.rope_apply(orc.rms_norm(x[None], qn, 1e-6), c[r:r + 1],
                               s[r:r + 1])[0]
            assert np.array_equal(qo[r, h], x)
        for h in range(KV):
            x = k[r, h] + kb[h * hd:(h + 1) * hd]
            x = orc.rope_apply(orc.rms_norm(x[None], kn, 1e-6), c[r:r + 1],
                               s[r:r + 1])[0]
            assert np.array_equal(cache.k[sb[r], so[r], h],
                                  orc.f32_to_f16_bits(x))
            y = v[r, h] + vb[h * hd:(h + 1) * hd]
            assert np.array_equal(cache.v[sb[r], so[r], h],
                                  orc.f32_to_f16_bits(y))
    # f32 cells (the reference's own): the same q, and cells whose f16
    # rounding is exactly the f16 cache's
    c32 = orc.KvCache(nb, bs, KV, hd, orc.F32)
    qo32 = orc.attn_prep(c32, q, k, v, c, s, sb, so, qb, kb, vb, qn, kn, 1e-6)
    assert np.array_equal(qo32, qo)
    assert np.array_equal(orc.f32_to_f16_bits(c32.k), cache.k)
    assert np.array_equal(orc.f32_to_f16_bits(c32.v), cache.v)


# ---- paged prefill / chunked attention ----------------------------------
@pytest.mark.parametrize("case", range(6))
def test_paged_prefill_f64_matches_metal_golden(golden, case):
    """orc_paged_prefill_f64 on all six attn_decode cases of
    src/metal/ops.rs:676-766, q_len 2 and 3 included: the Metal mask
    (j >= valid or j + q_len > valid + qi) is batch_mask with
    pos_offset = valid - q_len and read_num = valid."""
    c = metal_case_inputs(case)
    exp = np.array(golden["metal_attn_decode"][case]["expected"], np.float32)
    cache = orc.KvCache(c["num_blocks"], c["bs"], c["n_kv"], c["hd"], orc.F32)
    cache.k[:] = c["cache_k"]
    cache.v[:] = c["cache_v"]
    B, Q, H, D = c["batch"], c["q_len"], c["n_heads"], c["hd"]
    valid = np.array([c["ctx"] - 2 * b for b in range(B)], np.uint32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = orc.paged_prefill_f64(cache, c["q"].reshape(B, Q, H, D),
                                c["block_idx"], c["max_blocks"], valid - Q,
                                valid, scale=scale)
    assert np.max(np.abs(out.reshape(-1) - exp)) < 1e-6


def test_paged_prefill_f64_matches_reference_composition():
    """Against the reference's own prefill composition, gather +
    batch_mask + gqa_attention (src/model.rs:628-644, each pinned above),
    over chunked offsets, ragged read counts, padding past read_num,
    windows and GQA groups 1/3/4."""
    rng = np.random.default_rng(21)
    for (nkv, G, hd, B, Q, window) in [(2, 3, 16, 3, 5, 0), (1, 4, 8, 2, 9, 4),
                                       (2, 1, 32, 2, 1, 0), (3, 2, 16, 4, 7, 3)]:
        bs, mb = 4, 8
        nb = B * mb
        cache = orc.KvCache(nb, bs, nkv, hd, orc.F16)
        cache.k[:] = orc.f32_to_f16_bits(rng.standard_normal(cache.k.shape))
        cache.v[:] = orc.f32_to_f16_bits(rng.standard_normal(cache.v.shape))
        tables = rng.permutation(nb).astype(np.uint32)
        off = rng.integers(0, bs * mb - Q, B).astype(np.uint32)
        read = np.minimum(off + Q + rng.integers(-2, 3, B), bs * mb)
        read = read.astype(np.uint32)
        q = rng.standard_normal((B, Q, nkv * G, hd)).astype(np.float32)
        out = orc.paged_prefill_f64(cache, q, tables, mb, off, read,
                                    window=window)
        ctx = int(read.max())
        gk, gv = cache.gather(tables, B, mb, ctx)
        m = orc.batch_mask(off, read, Q, ctx, window)
        ref = orc.gqa_attention(q.transpose(0, 2, 1, 3).copy(), gk, gv, m)
        ref = ref.transpose(0, 2, 1, 3)
        seen = np.isfinite(m.reshape(B, Q, ctx)).any(-1)  # rows with keys
        assert np.max(np.abs(out - ref)[seen]) < 1e-5
        assert np.all(out[~seen] == 0)


def test_paged_prefill_f64_q_len_one_is_decode():
    rng = np.random.default_rng(22)
    cache = orc.KvCache(30, 16, 2, 32, orc.F16)
    cache.k[:] = orc.f32_to_f16_bits(rng.standard_normal(cache.k.shape))
    cache.v[:] = orc.f32_to_f16_bits(rng.standard_normal(cache.v.shape))
    tables = rng.permutation(30).astype(np.uint32)
    ctx = np.array([1, 77, 160], np.uint32)
    q = rng.standard_normal((3, 1, 6, 32)).astype(np.float32)
    for w in (0, 20):
        a = orc.paged_prefill_f64(cache, q, tables, 10, ctx - 1, ctx,
                                  window=w)
        b = orc.paged_decode_f64(cache, q[:, 0], tables, 10, ctx, window=w)
        assert np.array_equal(a[:, 0], b)


# ---- greedy argmax -------------------------------------------------------
def argmax_kat_rows():
    """The rows of argmax_matches_hand_computed (src/cuda/ops.rs:1447-1477):
    unique max; tie between 1 and 3 with a NaN; all -inf; max at 599."""
    n = 600
    d = np.zeros((4, n), np.float32)
    d[0, 0], d[0, 1], d[0, 2] = 1.0, 5.0, -2.0
    d[1, 0], d[1, 1], d[1, 3] = np.nan, 3.0, 3.0
    d[2, :] = -np.inf
    d[3, 599] = 9.0
    d[0, 4:] = -1.0
    d[1, 4:] = -1.0
    return d


def test_argmax_kat():
    assert orc.argmax_rows(argmax_kat_rows()).tolist() == [1, 1, 0, 599]


def test_argmax_matches_a_python_scan():
    rng = np.random.default_rng(30)
    x = rng.integers(-3, 4, (50, 37)).astype(np.float32)  # many ties
    x[rng.random(x.shape) < 0.1] = np.nan
    x[7] = np.nan
    for r, row in enumerate(x):
        best, bv = 0, -np.inf
        for i, v in enumerate(row):
            if v > bv:
                best, bv = i, v
        assert orc.argmax_rows(x)[r] == best
