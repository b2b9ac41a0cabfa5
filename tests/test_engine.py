"""The reference engine's behaviour tests (src/engine.rs:737-973), run
against rvllm_amd.engine over the native scheduler, with the reference's
CountingBackend stand-in (src/engine.rs:644-700): the next token is the
last input token + 1 (mod 1000), no KV involved. Plus scheduler-level
checks of the prefix cache, eviction, copy-on-write and preemption.

The scheduler's exact allocation/eviction policy (kv-cache-scheduler 0.2.0)
is not in the container: parity is pinned through these behaviour tests
only.
"""
from types import SimpleNamespace

import numpy as np
import pytest

from rvllm_amd.engine import (Engine, EngineConfig, ExceedsKvCapacity,
                              EmptyPrompt, FinishReason, PromptTooLong,
                              Request, RequestSpec, ZeroMaxTokens, run)
from rvllm_amd.scheduler import Scheduler


class CountingBackend:
    def __init__(self, context_length: int):
        self.config = SimpleNamespace(context_length=context_length)
        self.max_batch_seen = 0
        self.released = []
        self.items = []
        self.copies = []

    def forward_sample(self, items, last_only, samplers):
        assert len(items) == len(samplers)
        self.max_batch_seen = max(self.max_batch_seen, len(items))
        self.items.append((last_only, items))
        return [(it.tokens[-1] + 1) % 1000 for it in items]

    def release(self, seq_id):
        self.released.append(seq_id)

    def copy_blocks(self, src, dst):
        self.copies.append((list(src), list(dst)))


def cfg(num_blocks, max_running):
    return EngineConfig(block_size=4, num_blocks=num_blocks,
                        max_running=max_running)


def req(tokens, max_tokens, stop=()):
    return Request(list(tokens), max_tokens, tuple(stop))


def drain(engine):
    out = []
    while engine.has_work():
        out.extend(engine.step())
    return out


def tokens_of(events, sid):
    return [e.token for e in events if e.id == sid]


# ---- src/engine.rs:737-973 ---------------------------------------------------
def test_first_sampled_token_is_emitted():
    engine = Engine(CountingBackend(64), cfg(16, 8))
    sid = engine.add_request(req([10, 11, 12], 3))
    ev = drain(engine)
    assert tokens_of(ev, sid) == [13, 14, 15]
    assert ev[-1].finish == FinishReason.LENGTH
    assert ev[0].ttft is not None and ev[1].ttft is None


def test_stop_token_ends_generation():
    engine = Engine(CountingBackend(64), cfg(16, 8))
    sid = engine.add_request(req([10], 50, stop=[13]))
    ev = drain(engine)
    assert tokens_of(ev, sid) == [11, 12, 13]
    assert ev[-1].finish == FinishReason.STOP
    assert engine.backend.released == [sid]


def test_max_tokens_one_finishes_at_prefill():
    engine = Engine(CountingBackend(64), cfg(16, 8))
    sid = engine.add_request(req([5, 6], 1))
    ev = engine.step()
    assert tokens_of(ev, sid) == [7]
    assert ev[0].finish == FinishReason.LENGTH
    assert not engine.has_work()


def test_max_running_queues_the_rest_fifo():
    engine = Engine(CountingBackend(64), cfg(64, 2))
    ids = [engine.add_request(req([100 * (i + 1)], 4)) for i in range(5)]
    events = engine.step()
    assert engine.num_running() == 2 and engine.num_waiting() == 3
    finish_order = []
    while engine.has_work():
        for e in engine.step():
            if e.finish is not None:
                finish_order.append(e.id)
            events.append(e)
    assert finish_order == ids
    assert engine.backend.max_batch_seen <= 2
    for i, sid in enumerate(ids):
        p = 100 * (i + 1)
        assert tokens_of(events, sid) == list(range(p + 1, p + 5))


def test_outputs_do_not_depend_on_batching():
    def alone(prompt):
        e = Engine(CountingBackend(64), cfg(16, 8))
        sid = e.add_request(req([prompt], 5))
        return tokens_of(drain(e), sid)
    engine = Engine(CountingBackend(64), cfg(16, 8))
    a = engine.add_request(req([10], 5))
    b = engine.add_request(req([200], 5))
    ev = drain(engine)
    assert tokens_of(ev, a) == alone(10)
    assert tokens_of(ev, b) == alone(200)
    assert engine.backend.max_batch_seen == 2


def test_preemption_still_completes_every_request():
    # 6 blocks of 4 slots can't hold three 10-token sequences at once.
    engine = Engine(CountingBackend(64), cfg(6, 8))
    ids = [engine.add_request(req([10 * (i + 1)], 9)) for i in range(3)]
    ev = drain(engine)
    for i, sid in enumerate(ids):
        start = 10 * (i + 1) + 1
        assert tokens_of(ev, sid) == list(range(start, start + 9))
    assert engine.scheduler.available() == 6
    released = engine.backend.released
    assert all(sid in released for sid in ids)
    assert len(released) > len(ids)
    assert engine.scheduler.metrics()[2] > 0  # preemptions happened


def test_abort_frees_running_and_waiting():
    engine = Engine(CountingBackend(64), cfg(16, 1))
    a = engine.add_request(req([1, 2, 3], 50))
    b = engine.add_request(req([4, 5, 6], 50))
    engine.step()
    assert (engine.num_running(), engine.num_waiting()) == (1, 1)
    engine.abort(a)
    engine.abort(b)
    assert engine.backend.released == [a, b]
    assert not engine.has_work()
    assert engine.scheduler.available() == 16
    assert not engine.scheduler.has(a) and not engine.scheduler.has(b)
    engine.abort(a)  # idempotent


def test_rejects_requests_that_can_never_run():
    engine = Engine(CountingBackend(32), cfg(4, 8))  # 16 slots
    with pytest.raises(EmptyPrompt):
        engine.add_request(req([], 5))
    with pytest.raises(ZeroMaxTokens):
        engine.add_request(req([1], 0))
    with pytest.raises(PromptTooLong):
        engine.add_request(req([1] * 40, 5))
    with pytest.raises(ExceedsKvCapacity):
        engine.add_request(req([1] * 10, 20))
    big = Engine(CountingBackend(8), cfg(16, 8))  # clamped, not rejected
    sid = big.add_request(req([1, 2], 100))
    assert len(tokens_of(drain(big), sid)) == 6


def test_continuable_request_stops_when_the_pool_is_full():
    engine = Engine(CountingBackend(64), cfg(4, 8))
    sid = engine.add_continuable_request(req([1, 2, 3], 40))
    ev = drain(engine)
    mine = [e for e in ev if e.id == sid]
    assert mine[-1].finish == FinishReason.POOL_FULL
    assert len(mine) == 14
    assert not engine.has_work()
    assert engine.scheduler.available() == 4
    nxt = engine.add_continuable_request(req([mine[-1].token], 3))
    ev = drain(engine)
    assert sum(1 for e in ev if e.id == nxt) == 3


def test_continuable_request_must_leave_room_for_its_first_token():
    engine = Engine(CountingBackend(64), cfg(4, 8))
    with pytest.raises(ExceedsKvCapacity):
        engine.add_continuable_request(req([1] * 16, 5))
    engine.add_continuable_request(req([1] * 15, 5))


def test_plain_requests_still_reserve_their_whole_answer():
    engine = Engine(CountingBackend(64), cfg(4, 8))
    with pytest.raises(ExceedsKvCapacity):
        engine.add_request(req([1, 2, 3], 40))


def test_run_wrapper_honours_arrival_steps():
    res = run(CountingBackend(64), [RequestSpec([1], 3, 0),
                                    RequestSpec([50], 3, 2)],
              cfg(16, 8), stop_tokens=[999])
    assert res.generated == [[2, 3, 4], [51, 52, 53]]
    assert res.stats.output_tokens == 6


def test_run_wrapper_stops_on_any_stop_token():
    res = run(CountingBackend(64), [RequestSpec([1], 5), RequestSpec([50], 3)],
              cfg(16, 8), stop_tokens=[999, 3])
    assert res.generated == [[2, 3], [51, 52, 53]]


# ---- what the forward calls see ----------------------------------------------
def test_items_carry_slots_tables_and_positions():
    """Prefill items run the whole prompt at position 0; decode items run
    the last sampled token at position num_tokens, written to
    logical_to_physical(position) (src/engine.rs:372-382, 440-447)."""
    engine = Engine(CountingBackend(64), cfg(16, 8))
    sid = engine.add_request(req([7, 8, 9, 10, 11], 3))
    drain(engine)
    (lo0, pre), (lo1, d1), (lo2, d2) = engine.backend.items
    assert lo0 and not lo1 and not lo2
    p = pre[0]
    assert p.tokens == [7, 8, 9, 10, 11] and p.position_offset == 0
    assert p.read_num_tokens == 5 and len(p.read_blocks) == 2
    assert [w[1] for w in p.write_positions] == [0, 1, 2, 3, 0]
    assert p.write_positions[4][0] == p.read_blocks[1]
    assert d1[0].tokens == [12] and d1[0].position_offset == 5
    assert d1[0].read_num_tokens == 6 and d1[0].write_positions == [
        (d1[0].read_blocks[1], 1)]
    assert d2[0].tokens == [13] and d2[0].position_offset == 6


# ---- prefix cache --------------------------------------------------------------
def test_prefix_cache_reuses_full_blocks_and_skips_their_tokens():
    engine = Engine(CountingBackend(128), cfg(32, 8))
    prompt = list(range(100, 111))  # 11 tokens: 2 full blocks + 3
    a = engine.add_request(req(prompt, 2))
    drain(engine)
    b = engine.add_request(req(prompt[:9] + [555, 556], 2))
    ev = drain(engine)
    assert tokens_of(ev, b) == [557, 558]
    last_only, items = engine.backend.items[-2]
    assert last_only and items[0].position_offset == 8
    assert items[0].tokens == [108, 555, 556]
    hits, total, _ = engine.scheduler.metrics()
    assert (hits, total) == (2, 4)


def test_prefix_cache_never_matches_the_last_token_block():
    sch = Scheduler(16, 4)
    a = sch.add_request(list(range(8)))
    sch.prefill(a)
    sch.finish_sequence(a)
    assert sch.match_prefix(list(range(8)))[1] != []
    assert len(sch.match_prefix(list(range(8)))[1]) == 1  # (8 - 1) // 4
    assert len(sch.match_prefix(list(range(9)))[1]) == 2


def test_cached_blocks_count_as_available_and_evict_lru():
    sch = Scheduler(4, 2)
    a = sch.add_request([1, 2, 3, 4, 5])  # blocks [1,2] [3,4] [5]
    sch.prefill(a)
    assert sch.available() == 1
    sch.finish_sequence(a)
    assert sch.available() == 4
    assert len(sch.match_prefix([1, 2, 3, 4, 9])[1]) == 2
    # Needing all 4 blocks evicts the cached ones.
    b = sch.add_request([7, 7, 7, 7, 7, 7, 7, 7])
    sch.prefill(b)
    assert sch.available() == 0
    assert sch.match_prefix([1, 2, 3, 4, 9]) == (0, [])
    assert sch.total_allocs == 3 + 4


def test_shared_blocks_are_refcounted():
    sch = Scheduler(16, 4)
    a = sch.add_request(list(range(9)))
    sch.prefill(a)
    b = sch.add_request(list(range(8)) + [77])
    assert sch.prefill(b) == 2
    ba, bb = sch.blocks(a), sch.blocks(b)
    assert ba[:2] == bb[:2] and ba[2] != bb[2]
    assert [sch.refcount(x) for x in ba[:2]] == [2, 2]
    sch.finish_sequence(a)
    assert [sch.refcount(x) for x in bb[:2]] == [1, 1]
    sch.finish_sequence(b)
    assert sch.available() == 16


def test_fork_then_step_copies_the_shared_tail_block():
    sch = Scheduler(8, 4)
    a = sch.add_request([1, 2, 3, 4, 5, 6])  # tail block half full
    sch.prefill(a)
    b = sch.fork(a)
    tail = sch.blocks(a)[1]
    assert sch.refcount(tail) == 2
    sch.step()
    src, dst = sch.take_cow()
    assert len(src) == 1 and src[0] == tail
    # the first writer got the copy, the other keeps the original
    assert sch.blocks(a)[1] == dst[0] and sch.blocks(b)[1] == tail
    assert sch.refcount(tail) == 1 and sch.refcount(int(dst[0])) == 1
    assert sch.blocks(a)[0] == sch.blocks(b)[0]
    assert sch.take_cow()[0].size == 0


def test_step_preempts_from_the_back_and_requeues_in_front():
    sch = Scheduler(3, 2)
    ids = [sch.add_request([10 * i, 10 * i + 1]) for i in range(3)]
    for s in ids:
        sch.prefill(s)
    assert sch.available() == 0
    sch.step()  # every sequence needs a new block; none is free
    assert sch.running == [ids[0]]
    assert sch.waiting == [ids[1], ids[2]]
    assert sch.metrics()[2] == 2
    assert sch.num_tokens(ids[0]) == 3 and sch.num_tokens(ids[1]) == 0


def test_set_tokens_protects_tokens_with_kv():
    sch = Scheduler(8, 4)
    a = sch.add_request([1, 2, 3])
    sch.prefill(a)
    sch.step()
    sch.set_tokens(a, [1, 2, 3, 9])  # the placeholder may change
    with pytest.raises(Exception):
        sch.set_tokens(a, [1, 5, 3, 9])


def test_random_workload_keeps_the_pool_consistent():
    """Seeded random admissions, steps, finishes and aborts: blocks are
    never lost or double-owned, and finished pools drain to full."""
    rng = np.random.default_rng(7)
    engine = Engine(CountingBackend(512), cfg(40, 6))
    live = []
    for step in range(300):
        if rng.random() < 0.3:
            n = int(rng.integers(1, 30))
            base = int(rng.integers(0, 4)) * 100  # shared prefixes
            toks = [base + (i % 7) for i in range(n)]
            try:
                live.append(engine.add_request(req(toks, int(
                    rng.integers(1, 20)))))
            except ExceedsKvCapacity:
                pass
        if live and rng.random() < 0.05:
            engine.abort(live.pop(int(rng.integers(0, len(live)))))
        engine.step()
        sch = engine.scheduler
        owned = {}
        for sid in sch.running:
            for b in sch.blocks(sid):
                owned[b] = owned.get(b, 0) + 1
        for b, n in owned.items():
            assert sch.refcount(b) == n
        assert sch.available() + len(owned) <= 40
    drain(engine)
    assert engine.scheduler.available() == 40
