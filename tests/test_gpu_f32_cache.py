"""GPU parity of the f32 cache (rvllm's own cache dtype, src/kv_storage.rs:
84-104 zeroes f32 K/V; src/cuda/kv_storage.rs:65-100 allocates the device
pool in f32): append, gather, copy and inspection bit-exact against the
oracle's f32 cache, paged decode against the oracle's float64 attention over
the same f32 cells, all through the C ABI."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rvllm_amd import workloads as W
from rvllm_amd._lib import RvkvError
from rvllm_amd.kv_storage import HipDecodePlan, HipGatherPlan, HipKvStorage
from tests.gpu_util import dev_u32

pytestmark = pytest.mark.gpu

F32 = torch.float32
# f32 cells and f32 arithmetic (scores, softmax, accumulation): the error
# against float64 stays far inside the f16 cache's 2e-3.
ATOL_F32 = 1e-4


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu] {request.node.name}", flush=True)
    sys.stdout.flush()
    yield
    torch.cuda.synchronize()


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_f32_kats(golden):
    """The reference's KATs at the reference's own cache dtype: the raw
    cache and the gather hold the written values exactly
    (src/kv_storage.rs:193-237)."""
    g = golden["reference_kats"]["round_trip_across_blocks"]
    st = HipKvStorage(1, 3, 2, 1, 2, dtype=F32)
    k = torch.tensor(g["k"], dtype=torch.float32).reshape(4, 1, 2).cuda()
    st.write_tokens(0, dev_u32(g["block_ids"]), dev_u32(g["offsets"]), k, k)
    raw = st.read_blocks(0, 0, dev_u32([0, 1, 2]))
    assert raw.dtype == F32
    assert raw.cpu().reshape(-1).tolist() == g["raw_cache"]
    plan = HipGatherPlan([(g["tables"][0], 3), (g["tables"][1], 1)])
    ok = torch.zeros(2 * 1 * 3 * 2, device="cuda")
    ov = torch.zeros_like(ok)
    st.gather(0, plan, ok, ov)
    got = ok.cpu().tolist()
    assert got == ov.cpu().tolist()
    assert got[:6] == g["gather_prefix_a"]
    assert got[6:8] == g["gather_prefix_b"]
    u = golden["reference_kats"]["untouched_slots"]
    st2 = HipKvStorage(1, 1, 4, 1, 2, dtype=F32)
    t = torch.tensor(u["k"], dtype=torch.float32).reshape(1, 1, 2).cuda()
    st2.write_tokens(0, dev_u32([0]), dev_u32([2]), t, t)
    ok = torch.zeros(8, device="cuda")
    st2.gather(0, HipGatherPlan([([0], 4)]), ok, torch.zeros_like(ok))
    assert ok.cpu().tolist() == u["gather"]


@pytest.mark.parametrize("nkv,hd,bs", [(5, 64, 16), (1, 256, 16), (3, 2, 2),
                                       (2, 12, 3), (8, 128, 32)])
def test_f32_append_gather_copy_bit_exact(nkv, hd, bs):
    rng = np.random.default_rng(hd + nkv)
    nb = 29
    st = HipKvStorage(2, nb, bs, nkv, hd, dtype=F32)
    ref = orc.KvCache(nb, bs, nkv, hd, orc.F32)
    slots = rng.permutation(nb * bs)[: nb * bs // 2]
    k = (rng.standard_normal((len(slots), nkv, hd)) * 100).astype(np.float32)
    v = rng.standard_normal((len(slots), nkv, hd)).astype(np.float32)
    k[0, 0, 0], v[0, 0, 0] = np.inf, -0.0
    k[1, 0, 0] = 1e-42  # an f32 subnormal: f32 rows are copied, never rounded
    st.write_tokens(1, dev_u32(slots // bs), dev_u32(slots % bs),
                    torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    ref.write_tokens(slots // bs, slots % bs, k, v)
    # f16 source rows widen exactly (every f16 is an f32)
    s16 = rng.permutation(nb * bs)[:7]
    k16 = rng.standard_normal((7, nkv, hd)).astype(np.float16)
    k16[0, 0, 0] = np.float16(6e-8)  # an f16 subnormal
    st.write_tokens(1, dev_u32(s16 // bs), dev_u32(s16 % bs),
                    torch.from_numpy(k16).cuda(), torch.from_numpy(-k16).cuda())
    ref.write_tokens(s16 // bs, s16 % bs, k16.astype(np.float32),
                     (-k16).astype(np.float32))
    ids = dev_u32(np.arange(nb))
    assert np.array_equal(_bits(st.read_blocks(1, 0, ids).cpu().numpy()),
                          _bits(ref.k))
    assert np.array_equal(_bits(st.read_blocks(1, 1, ids).cpu().numpy()),
                          _bits(ref.v))
    assert st.read_blocks(0, 0, ids).eq(0).all()  # the other layer untouched
    # gather into f32 (bit for bit) through the padded plan, ragged lengths
    tabs = [rng.permutation(nb)[:5].tolist(), rng.permutation(nb)[:3].tolist()]
    plan = HipGatherPlan([(tabs[0], 5 * bs - 1), (tabs[1], 2 * bs + 1)])
    n = 2 * nkv * plan.ctx_len * hd
    ok = torch.empty(n, device="cuda")
    ov = torch.empty(n, device="cuda")
    st.gather(1, plan, ok, ov)
    wk, wv = ref.gather(plan.block_idx.cpu().numpy().view(np.uint32), 2,
                        plan.max_blocks, plan.ctx_len)
    assert np.array_equal(_bits(ok.cpu().numpy()), _bits(wk.reshape(-1)))
    assert np.array_equal(_bits(ov.cpu().numpy()), _bits(wv.reshape(-1)))
    with pytest.raises(RvkvError, match="an f32 cache gathers into F32 only"):
        st.gather(1, plan, ok.half(), ov.half())
    # checksums over the f32 bytes agree with the oracle's
    cs = st.block_checksums(1, 0, ids).cpu().numpy().view(np.uint64)
    assert np.array_equal(cs, ref.checksums(0, np.arange(nb)))
    cv = st.block_checksums(1, 1, ids).cpu().numpy().view(np.uint64)
    assert np.array_equal(cv, ref.checksums(1, np.arange(nb)))
    # copy-on-write: every layer, K and V, bit for bit
    src, dst = int(slots[0] // bs), int(slots[1] // bs)
    if src == dst:
        dst = (src + 1) % nb
    st.copy_blocks(dev_u32([src]), dev_u32([dst]))
    ref.copy_blocks([src], [dst])
    assert np.array_equal(_bits(st.read_blocks(1, 0, ids).cpu().numpy()),
                          _bits(ref.k))
    assert np.array_equal(_bits(st.read_blocks(1, 1, ids).cpu().numpy()),
                          _bits(ref.v))


def _f32_pool(bs, nkv, hd, lens, seed):
    cfg = W.Config("f32", 9, 1, nkv, nkv, hd, bs, len(lens))
    db = W.ragged_batch(cfg, lens, seed=seed, extra_blocks=3)
    st = HipKvStorage(1, db.num_blocks, bs, nkv, hd, dtype=F32)
    ref = orc.KvCache(db.num_blocks, bs, nkv, hd, orc.F32)
    rng = np.random.default_rng(seed)
    n = db.num_blocks * bs
    k = rng.standard_normal((n, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((n, nkv, hd)).astype(np.float32)
    slots = np.arange(n)
    st.write_tokens(0, dev_u32(slots // bs), dev_u32(slots % bs),
                    torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    ref.write_tokens(slots // bs, slots % bs, k, v)
    return db, st, ref


@pytest.mark.parametrize("G,hd", [(3, 64), (2, 128), (4, 256), (7, 32),
                                  (1, 64), (8, 128)])
def test_f32_decode_vs_oracle(G, hd):
    """Uniform and planned decode (windows, an empty sequence, sequences
    long enough to split) and the decode step (the append fused into the
    decode launch; f32 and f16 source rows) over an f32 cache, against
    float64 attention over the same cells."""
    bs, nkv = 16, 2
    lens = np.array([1, 17, 300, 2500, 64, 5], np.uint32)
    db, st, ref = _f32_pool(bs, nkv, hd, lens, seed=G * 7 + hd)
    H = G * nkv
    rng = np.random.default_rng(hd - G)
    qn = rng.standard_normal((len(lens), H, hd)).astype(np.float32)
    q = torch.from_numpy(qn).cuda()
    padded = db.padded_tables()
    tab = dev_u32(padded)
    tables = padded.reshape(-1)
    ctx = lens.copy()
    ctx[5] = 0  # an empty sequence: zero output
    for window in (0, 100):
        out = st.paged_decode(0, q, tab, dev_u32(ctx), int(ctx.max()),
                              window=window)
        want = orc.paged_decode_f64(ref, qn, tables, db.max_blocks, ctx,
                                    window=window)
        assert np.abs(out.cpu().numpy() - want).max() < ATOL_F32, window
        assert out[5].eq(0).all()
    plan = HipDecodePlan(st, ctx, H)
    out = st.paged_decode_planned(0, plan, q, tab, dev_u32(ctx))
    want = orc.paged_decode_f64(ref, qn, tables, db.max_blocks, ctx)
    assert np.abs(out.cpu().numpy() - want).max() < ATOL_F32
    # decode step: each sequence's new row lands at slot ctx-1, bit for bit,
    # and is attended to in the same call
    nk = rng.standard_normal((len(lens), nkv, hd)).astype(np.float32)
    nv = rng.standard_normal((len(lens), nkv, hd)).astype(np.float32)
    plan.update(lens)
    for use_plan in (False, True):
        got = st.decode_step(0, torch.from_numpy(nk).cuda(),
                             torch.from_numpy(nv).cuda(),
                             dev_u32(db.slot_block), dev_u32(db.slot_off), q,
                             tab, dev_u32(lens), int(lens.max()),
                             plan=plan if use_plan else None)
        want = orc.decode_step(ref, db.slot_block, db.slot_off, nk, nv,
                               tables, db.max_blocks, lens, qn)
        assert np.abs(got.cpu().numpy() - want).max() < ATOL_F32, use_plan
        ids = dev_u32(np.arange(db.num_blocks))
        assert np.array_equal(_bits(st.read_blocks(0, 0, ids).cpu().numpy()),
                              _bits(ref.k))
        assert np.array_equal(_bits(st.read_blocks(0, 1, ids).cpu().numpy()),
                              _bits(ref.v))
        nk, nv = nv, nk
    # f16 source rows: widened exactly into the f32 cells
    nk16 = rng.standard_normal((len(lens), nkv, hd)).astype(np.float16)
    nv16 = rng.standard_normal((len(lens), nkv, hd)).astype(np.float16)
    got = st.decode_step(0, torch.from_numpy(nk16).cuda(),
                         torch.from_numpy(nv16).cuda(), dev_u32(db.slot_block),
                         dev_u32(db.slot_off), q, tab, dev_u32(lens),
                         int(lens.max()), plan=plan)
    want = orc.decode_step(ref, db.slot_block, db.slot_off,
                           nk16.astype(np.float32), nv16.astype(np.float32),
                           tables, db.max_blocks, lens, qn)
    assert np.abs(got.cpu().numpy() - want).max() < ATOL_F32
    ids = dev_u32(np.arange(db.num_blocks))
    assert np.array_equal(_bits(st.read_blocks(0, 0, ids).cpu().numpy()),
                          _bits(ref.k))
    assert np.array_equal(_bits(st.read_blocks(0, 1, ids).cpu().numpy()),
                          _bits(ref.v))


def test_f32_smollm2_config():
    """configs[0] (SmolLM2-360M attention: 15 q heads over 5 KV heads,
    head_dim 64, 8 sequences with ctx in [17, 512]) at the reference's own
    cache dtype: the decode step against the oracle's restatement of
    rvllm's CPU path (write_tokens, padded gather, batch_mask and
    gqa_attention in f32, src/model.rs:628-644)."""
    db = W.smollm2_batch()
    c = db.cfg
    rng = W.Rng(c.seed)
    nb, bs = db.num_blocks, c.block_size
    st = HipKvStorage(1, nb, bs, c.n_kv_heads, c.head_dim, dtype=F32)
    ref = orc.KvCache(nb, bs, c.n_kv_heads, c.head_dim, orc.F32)
    slots = np.arange(nb * bs)
    k = rng.normal((nb * bs, c.n_kv_heads, c.head_dim))
    v = rng.normal((nb * bs, c.n_kv_heads, c.head_dim))
    st.write_tokens(0, dev_u32(slots // bs), dev_u32(slots % bs),
                    torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    ref.write_tokens(slots // bs, slots % bs, k, v)
    nk = rng.normal((db.batch, c.n_kv_heads, c.head_dim))
    nv = rng.normal((db.batch, c.n_kv_heads, c.head_dim))
    q = rng.normal((db.batch, c.n_heads, c.head_dim))
    out = st.decode_step(0, torch.from_numpy(nk).cuda(),
                         torch.from_numpy(nv).cuda(), dev_u32(db.slot_block),
                         dev_u32(db.slot_off), torch.from_numpy(q).cuda(),
                         dev_u32(db.padded_tables()), dev_u32(db.ctx_lens),
                         int(db.ctx_lens.max()))
    want = orc.decode_step(ref, db.slot_block, db.slot_off, nk, nv,
                           db.padded_tables().reshape(-1), db.max_blocks,
                           db.ctx_lens, q)
    assert np.abs(out.cpu().numpy() - want).max() < ATOL_F32
    ids = dev_u32(np.arange(nb))
    assert np.array_equal(_bits(st.read_blocks(0, 1, ids).cpu().numpy()),
                          _bits(ref.v))


