"""CPU-side checks of the product library: it loads, exports exactly what
include/rvkv.h declares, validates arguments before touching the device, and
its host block manager behaves as rvllm's engine expects of
kv-cache-scheduler (src/engine.rs:737-973 is the behavioural spec)."""
import ctypes
import os
import re

import numpy as np

import pytest

from rvllm_amd import _lib
from rvllm_amd.block_manager import BlockManager
from rvllm_amd._lib import RvkvError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "rvkv.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(rvkv_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    declared = _declared_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(L, name), f"librvkv.so does not export {name}"
    assert declared == set(_lib.SIGNATURES), \
        "ctypes signatures out of sync with include/rvkv.h"


def test_pool_create_validates_before_any_device_call():
    L = _lib.load()
    h = ctypes.c_void_p()
    rc = L.rvkv_pool_create(0, 8, 16, 1, 64, _lib.RVKV_F16, None,
                            ctypes.byref(h))
    assert rc == _lib.RVKV_EINVAL
    assert L.rvkv_last_error().decode().startswith("pool_create: ")
    rc = L.rvkv_pool_create(1, 8, 16, 1, 64, 7, None, ctypes.byref(h))
    assert rc != _lib.RVKV_OK
    assert L.rvkv_last_error().decode().startswith("pool_create: ")


def test_entry_points_reject_null_pool_with_reference_style_messages():
    L = _lib.load()
    assert L.rvkv_append(None, 0, None, None, 2, None, None, 1) == -1
    assert L.rvkv_last_error().decode() == "kv_write: pool is NULL"
    assert L.rvkv_gather(None, 0, None, 1, 1, 1, None, None, 2) == -1
    assert L.rvkv_last_error().decode().startswith("kv_gather: ")
    assert L.rvkv_paged_decode(None, 0, None, None, None, 1, 1, 1, 1, 1.0, 0,
                               None, None, 0) == -1
    assert L.rvkv_last_error().decode().startswith("paged_decode: ")
    assert L.rvkv_copy_blocks(None, None, None, 1) == -1
    assert L.rvkv_decode_workspace_bytes(None, 1, 1, 1) == 0


def test_check_raises_with_library_message():
    L = _lib.load()
    L.rvkv_copy_blocks(None, None, None, 1)
    with pytest.raises(RvkvError, match="copy_blocks: pool is NULL"):
        _lib.check(-1)


# ---- block manager ---------------------------------------------------------
def test_slot_mapping_is_logical_to_physical():
    bm = BlockManager(16, 4)
    s = bm.add_seq(10)  # 3 blocks
    t = bm.table(s)
    assert len(t) == 3 and bm.available() == 13
    for pos in range(10):
        assert bm.slot(s, pos) == (t[pos // 4], pos % 4)
    with pytest.raises(RvkvError):
        bm.slot(s, 12)


def test_append_allocates_at_block_boundaries_only():
    bm = BlockManager(8, 4)
    s = bm.add_seq(3)
    assert bm.available() == 7
    blk, off, cow = bm.append_slot(s)  # position 3: same block
    assert (off, cow) == (3, None) and bm.available() == 7
    blk2, off2, cow2 = bm.append_slot(s)  # position 4: new block
    assert off2 == 0 and cow2 is None and bm.available() == 6
    assert bm.table(s) == [blk, blk2]
    assert bm.num_tokens(s) == 5


def test_drain_returns_every_block():
    """pool.available() returns to its start after finish/abort
    (src/engine.rs:834, 851)."""
    bm = BlockManager(16, 4)
    ids = [bm.add_seq(n) for n in (1, 5, 9, 16)]
    for i in ids:
        for _ in range(3):
            bm.append_slot(i)
    for i in ids:
        bm.free_seq(i)
    assert bm.available() == 16
    with pytest.raises(RvkvError):
        bm.free_seq(ids[0])


def test_pool_exhaustion_is_reported_not_fatal():
    """A 4x4 pool fits 16 tokens (src/engine.rs:889-903 counts 14 decode
    tokens after a 3-token prompt before PoolFull... the pool itself runs
    dry exactly at 16)."""
    bm = BlockManager(4, 4)
    s = bm.add_seq(3)
    for _ in range(13):
        bm.append_slot(s)
    assert bm.num_tokens(s) == 16 and bm.available() == 0
    with pytest.raises(RvkvError):
        bm.append_slot(s)
    with pytest.raises(RvkvError):
        bm.add_seq(1)
    bm.free_seq(s)
    assert bm.available() == 4


def test_prefix_sharing_refcounts_and_cow():
    bm = BlockManager(32, 4)
    owner = bm.add_seq(12)  # 3 full blocks
    t_owner = bm.table(owner)
    # A sharer of the first 8 tokens, aligned: blocks 0,1 shared.
    a = bm.fork_seq(owner, 8, 8)
    assert bm.table(a) == t_owner[:2]
    assert [bm.refcount(b) for b in t_owner] == [2, 2, 1]
    # A sharer of 6 tokens: its last block (t_owner[1]) is shared + partial.
    b = bm.fork_seq(owner, 6, 6)
    assert bm.refcount(t_owner[1]) == 3
    blk, off, cow = bm.append_slot(b)  # position 6 lands in a shared block
    assert cow is not None and cow[0] == t_owner[1]
    assert blk == cow[1] and off == 2
    assert bm.refcount(t_owner[1]) == 2 and bm.refcount(blk) == 1
    assert bm.table(b) == [t_owner[0], blk]
    # The aligned sharer starts a fresh block: no copy.
    _, off_a, cow_a = bm.append_slot(a)
    assert off_a == 0 and cow_a is None
    for s in (owner, a, b):
        bm.free_seq(s)
    assert bm.available() == 32


def test_fork_rejects_unaligned_prefix_with_private_tail():
    bm = BlockManager(8, 4)
    owner = bm.add_seq(8)
    with pytest.raises(RvkvError):
        bm.fork_seq(owner, 6, 7)


def test_shuffled_free_list_is_a_permutation_and_seeded():
    def order(seed):
        bm = BlockManager(64, 16)
        bm.shuffle_free(seed)
        s = bm.add_seq(64 * 16)
        return bm.table(s)
    a, b, c = order(1), order(1), order(2)
    assert a == b and a != c and sorted(a) == list(range(64))


def test_batch_slots_and_tables_match_single_calls():
    import numpy as np
    bm = BlockManager(64, 4)
    bm.shuffle_free(3)
    owner = bm.add_seq(8)
    a = bm.add_seq(3)
    b = bm.fork_seq(owner, 8, 8)
    c = bm.fork_seq(owner, 6, 6)  # partial shared last block -> CoW
    seqs = [owner, a, b, c]
    blocks, offs, cs, cd = bm.append_slots(seqs)
    assert len(cs) == 1 and cd[0] == bm.table(c)[1]
    for s, blk, off in zip(seqs, blocks, offs):
        pos = bm.num_tokens(s) - 1
        assert bm.slot(s, pos) == (blk, off)
    tables, lens = bm.fill_tables(seqs, 5)
    for i, s in enumerate(seqs):
        t = bm.table(s)
        assert list(tables[i, :len(t)]) == t
        assert (tables[i, len(t):] == t[-1]).all()
        assert lens[i] == bm.num_tokens(s)
    with pytest.raises(RvkvError):
        bm.fill_tables(seqs, 1)  # a table longer than max_blocks


def test_rope_table_matches_oracle():
    """rvllm_amd.rope vs the oracle's powf/cosf/sinf restatement of
    src/model.rs:224-250: one f32 ulp (6e-8 below 1) everywhere, positions
    up to 2^17, with and without Llama-3 factors."""
    from oracle import oracle as orc
    from rvllm_amd.rope import rope_cos_sin
    rng = np.random.default_rng(0)
    pos = np.concatenate([np.arange(64), [4095, 8191, 32767, 131071],
                          rng.integers(0, 1 << 17, 500)])
    for hd, theta, fac in [(64, 5e5, None), (128, 1e6, None),
                           (64, 5e5, np.linspace(1, 8, 32)),
                           (256, 1e4, None)]:
        c, s = rope_cos_sin(theta, hd, pos, fac)
        oc, os_ = orc.rope_cos_sin(theta, hd, pos, factors=fac)
        assert c.dtype == np.float32 and c.shape == (len(pos), hd // 2)
        assert np.max(np.abs(c - oc)) <= 6e-8
        assert np.max(np.abs(s - os_)) <= 6e-8


def test_kernels_have_no_inline_assembly():
    """The HIP sources hold no inline assembly: the compiler inserts the
    wait states the hardware needs between dependent instructions (an
    MFMA's write of a register and a VALU read of it, for one) only for
    instructions it can see."""
    csrc = os.path.join(os.path.dirname(_lib.__file__), "csrc")
    pat = re.compile(r"\basm\s*(volatile\s*)?\(|__asm__")
    found = []
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h", ".cpp")):
            with open(os.path.join(csrc, name)) as f:
                for i, line in enumerate(f, 1):
                    if pat.search(line.split("//")[0]):
                        found.append(f"{name}:{i}")
    assert not found, found


def test_bench_cpu_sample_keeps_the_batch_shape():
    """bench.py's CPU-baseline sample: the first sequences over a compact
    pool, shared blocks kept shared, tables and slots renumbered alike, and
    the same per-sequence bytes as in the full batch."""
    import bench
    from rvllm_amd import workloads as W
    db = W.qwen25_batch(batch=64)
    sub, ids = bench.sample_batch(W, db, 20)
    assert sub.batch == 20 and len(set(ids.tolist())) == len(ids)
    for t_new, t_old in zip(sub.tables, db.tables[:20]):
        assert np.array_equal(ids[t_new], t_old)
    assert np.array_equal(ids[sub.slot_block], db.slot_block[:20])
    assert sub.unique_kv_tokens() == W.DecodeBatch(
        db.cfg, db.num_blocks, db.ctx_lens[:20], db.tables[:20],
        db.slot_block[:20], db.slot_off[:20]).unique_kv_tokens()


def test_integration_sys_listing_matches_the_header():
    """The Rust -sys listing a maintainer would copy declares exactly the
    functions of include/rvkv.h, no more and no fewer."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    header = open(os.path.join(root, "include", "rvkv.h")).read()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    declared = set(re.findall(r"\b(rvkv_[a-z0-9_]+)\s*\(", header))
    listing = open(os.path.join(root, "INTEGRATION.md")).read()
    bound = set(re.findall(r"pub fn (rvkv_[a-z0-9_]+)", listing))
    assert bound == declared, (sorted(bound - declared),
                               sorted(declared - bound))
