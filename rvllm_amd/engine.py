"""Continuous-batching engine over the native scheduler: the host loop of
rvllm's src/engine.rs restated in Python around rvkv_sched_* (csrc/
scheduler.cpp).

`Engine` is steppable like the reference's: add_request (or
add_continuable_request) queues a request; every step admits waiting
requests FIFO (one prefill forward each, up to max_running and as far as
the block pool allows, reusing prefix-cached blocks), then runs one batched
decode forward over every running sequence, preempting (recompute) when the
pool runs dry. `run` drives a fixed request set to completion.

Everything device-specific sits behind a `Backend` (forward_sample +
release, src/engine.rs:28-46), plus copy_blocks for the copy-on-write pairs
the scheduler hands out (forked sequences writing into a shared block).
Cited behaviour: src/engine.rs:224-539 (engine), 549-632 (run).
"""
from __future__ import annotations

import enum
import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

from .scheduler import Scheduler


class FinishReason(enum.Enum):
    STOP = "stop"
    LENGTH = "length"
    # The pool is full and this request is the only one running, so it can't
    # grow (continuable requests only), src/engine.rs:133-140.
    POOL_FULL = "pool_full"


class RequestError(ValueError):
    """A request that can never run (src/engine.rs:150-178)."""


class EmptyPrompt(RequestError):
    def __init__(self):
        super().__init__("prompt is empty")


class ZeroMaxTokens(RequestError):
    def __init__(self):
        super().__init__("max_tokens must be at least 1")


class PromptTooLong(RequestError):
    def __init__(self, prompt: int, context: int):
        super().__init__(f"prompt is {prompt} tokens, which does not fit the "
                         f"model's {context}-token context")
        self.prompt, self.context = prompt, context


class ExceedsKvCapacity(RequestError):
    def __init__(self, tokens: int, capacity: int):
        super().__init__(f"request needs {tokens} tokens of KV cache but the "
                         f"pool only holds {capacity}")
        self.tokens, self.capacity = tokens, capacity


@dataclass
class EngineConfig:
    block_size: int
    num_blocks: int
    max_running: int = 1 << 62


@dataclass
class Request:
    tokens: List[int]
    max_tokens: int
    stop_tokens: Sequence[int] = ()
    sampler: object = None


@dataclass
class TokenEvent:
    id: int
    token: int
    finish: Optional[FinishReason]
    ttft: Optional[float]  # seconds, on a request's first token


@dataclass
class BatchItem:
    """One sequence's slice of a forward call (src/model.rs BatchItem):
    the tokens to run, the slot each one is written to, the sequence's block
    table and how many tokens attention reads, and the position of the
    first token."""
    seq_id: int
    tokens: List[int]
    write_positions: List[Tuple[int, int]]
    read_blocks: List[int]
    read_num_tokens: int
    position_offset: int


@dataclass
class EngineStats:
    prefill_time: float = 0.0
    prefill_tokens: int = 0
    decode_time: float = 0.0
    decode_steps: int = 0


@dataclass
class _SeqState:
    prompt_len: int
    max_tokens: int
    stop_tokens: Tuple[int, ...]
    sampler: object
    continuable: bool
    num_generated: int = 0
    last_token: int = 0


class Engine:
    def __init__(self, backend, cfg: EngineConfig):
        self.backend = backend
        self.cfg = cfg
        self.scheduler = Scheduler(cfg.num_blocks, cfg.block_size)
        self.seqs: Dict[int, _SeqState] = {}
        self.stats = EngineStats()

    # -- queries (src/engine.rs:237-282) -------------------------------------
    def context_length(self) -> int:
        return int(self.backend.config.context_length)

    def max_sequence_tokens(self) -> int:
        return min(self.cfg.num_blocks * self.cfg.block_size,
                   self.context_length())

    def num_running(self) -> int:
        return self.scheduler.num_running()

    def num_waiting(self) -> int:
        return self.scheduler.num_waiting()

    def has_work(self) -> bool:
        return self.num_running() > 0 or self.num_waiting() > 0

    # -- requests (src/engine.rs:284-341) ------------------------------------
    def add_request(self, req: Request) -> int:
        return self._enqueue(req, False)

    def add_continuable_request(self, req: Request) -> int:
        return self._enqueue(req, True)

    def _enqueue(self, req: Request, continuable: bool) -> int:
        if not req.tokens:
            raise EmptyPrompt()
        if req.max_tokens == 0:
            raise ZeroMaxTokens()
        context = self.context_length()
        prompt_len = len(req.tokens)
        if prompt_len >= context:
            raise PromptTooLong(prompt_len, context)
        max_tokens = min(req.max_tokens, context - prompt_len)
        capacity = self.cfg.num_blocks * self.cfg.block_size
        if continuable:
            if prompt_len >= capacity:  # the first token needs room too
                raise ExceedsKvCapacity(prompt_len + 1, capacity)
        elif prompt_len + max_tokens > capacity:
            raise ExceedsKvCapacity(prompt_len + max_tokens, capacity)
        seq_id = self.scheduler.add_request(req.tokens)
        self.seqs[seq_id] = _SeqState(prompt_len, max_tokens,
                                      tuple(req.stop_tokens), req.sampler,
                                      continuable)
        return seq_id

    def abort(self, seq_id: int) -> None:
        if self.seqs.pop(seq_id, None) is None:
            return
        self.scheduler.remove(seq_id)
        self.backend.release(seq_id)

    # -- the loop (src/engine.rs:343-539) ------------------------------------
    def step(self) -> List[TokenEvent]:
        events: List[TokenEvent] = []
        self._admit_waiting(events)
        self._decode(events)
        return events

    def _admit_waiting(self, events: List[TokenEvent]) -> None:
        sch, bs = self.scheduler, self.cfg.block_size
        while sch.num_running() < self.cfg.max_running:
            waiting = sch.waiting
            if not waiting:
                break
            seq_id = waiting[0]
            tokens = sch.tokens(seq_id)
            needed = -(-len(tokens) // bs)
            if sch.available() < needed:
                break
            _, matched = sch.match_prefix(tokens)
            skip = min(len(matched) * bs, len(tokens) - 1)
            t0 = time.perf_counter()
            sch.prefill(seq_id)
            item = BatchItem(
                seq_id, tokens[skip:],
                [sch.logical_to_physical(seq_id, i)
                 for i in range(skip, len(tokens))],
                sch.blocks(seq_id), sch.num_tokens(seq_id), skip)
            state = self.seqs[seq_id]
            nxt = self.backend.forward_sample([item], True,
                                              [state.sampler])[0]
            dt = time.perf_counter() - t0
            self.stats.prefill_time += dt
            self.stats.prefill_tokens += len(tokens) - skip
            first = state.num_generated == 0
            self._emit(seq_id, int(nxt), dt if first else None, events)

    def _decode(self, events: List[TokenEvent]) -> None:
        sch = self.scheduler
        running = sch.running
        if not running:
            return
        t0 = time.perf_counter()
        offsets = {sid: sch.num_tokens(sid) for sid in running}
        sch.step()
        src, dst = sch.take_cow()
        if len(src):
            self.backend.copy_blocks(src, dst)
        still = set(sch.running)
        # Preempted sequences: rebuild token_ids as prompt + every token
        # sampled so far so they re-prefill cleanly (src/engine.rs:424-438).
        for sid in running:
            if sid not in still:
                self.backend.release(sid)
                st = self.seqs[sid]
                real_len = st.prompt_len + st.num_generated
                toks = sch.tokens(sid)[:real_len - 1] + [st.last_token]
                sch.set_tokens(sid, toks)
        items: List[BatchItem] = []
        for sid in running:
            if sid not in still:
                continue
            st = self.seqs[sid]
            toks = sch.tokens(sid)
            toks[-1] = st.last_token
            sch.set_tokens(sid, toks)
            pos = offsets[sid]
            items.append(BatchItem(sid, [st.last_token],
                                   [sch.logical_to_physical(sid, pos)],
                                   sch.blocks(sid), sch.num_tokens(sid), pos))
        if not items:
            return
        samplers = [self.seqs[it.seq_id].sampler for it in items]
        next_ids = self.backend.forward_sample(items, False, samplers)
        for it, nxt in zip(items, next_ids):
            self._emit(it.seq_id, int(nxt), None, events)
        self.stats.decode_time += time.perf_counter() - t0
        self.stats.decode_steps += 1

    def _cannot_grow(self, seq_id: int) -> bool:
        sch = self.scheduler
        return (sch.running == [seq_id]
                and sch.num_tokens(seq_id) % self.cfg.block_size == 0
                and sch.available() == 0)

    def _emit(self, seq_id: int, token: int, ttft: Optional[float],
              events: List[TokenEvent]) -> None:
        st = self.seqs[seq_id]
        st.num_generated += 1
        st.last_token = token
        if token in st.stop_tokens:
            finish = FinishReason.STOP
        elif st.num_generated >= st.max_tokens:
            finish = FinishReason.LENGTH
        elif st.continuable and self._cannot_grow(seq_id):
            finish = FinishReason.POOL_FULL
        else:
            finish = None
        if finish is not None:
            self.scheduler.finish_sequence(seq_id)
            self.scheduler.remove(seq_id)
            del self.seqs[seq_id]
            self.backend.release(seq_id)
        events.append(TokenEvent(seq_id, token, finish, ttft))


# -- the fixed-request-set driver (src/engine.rs:540-632) ---------------------
@dataclass
class RequestSpec:
    tokens: List[int]
    max_tokens: int
    arrival_step: int = 0


@dataclass
class RunStats:
    steps: int = 0
    elapsed: float = 0.0
    output_tokens: int = 0
    prefix_hits: int = 0
    prefix_total: int = 0
    total_block_allocs: int = 0
    preemptions: int = 0
    prefill_time: float = 0.0
    prefill_tokens: int = 0
    decode_time: float = 0.0
    decode_steps: int = 0
    ttft: List[float] = field(default_factory=list)


@dataclass
class RunResult:
    generated: List[List[int]]
    stats: RunStats


def run(backend, requests: Sequence[RequestSpec], cfg: EngineConfig,
        stop_tokens: Sequence[int] = (), sampler_factory=None) -> RunResult:
    engine = Engine(backend, cfg)
    order = sorted(range(len(requests)), key=lambda i: requests[i].arrival_step)
    nxt = 0
    req_of: Dict[int, int] = {}
    generated: List[List[int]] = [[] for _ in requests]
    ttft = [0.0] * len(requests)
    t0 = time.perf_counter()
    step = 0
    while True:
        while nxt < len(order) and requests[order[nxt]].arrival_step <= step:
            i = order[nxt]
            nxt += 1
            sid = engine.add_request(Request(
                list(requests[i].tokens), requests[i].max_tokens,
                tuple(stop_tokens),
                sampler_factory() if sampler_factory else None))
            req_of[sid] = i
        if not engine.has_work() and nxt == len(order):
            break
        for ev in engine.step():
            i = req_of[ev.id]
            generated[i].append(ev.token)
            if ev.ttft is not None:
                ttft[i] = ev.ttft
        step += 1
    hits, total, pre = engine.scheduler.metrics()
    st = RunStats(
        steps=step, elapsed=time.perf_counter() - t0,
        output_tokens=sum(len(g) for g in generated), prefix_hits=hits,
        prefix_total=total,
        total_block_allocs=engine.scheduler.total_allocs, preemptions=pre,
        prefill_time=engine.stats.prefill_time,
        prefill_tokens=engine.stats.prefill_tokens,
        decode_time=engine.stats.decode_time,
        decode_steps=engine.stats.decode_steps, ttft=ttft)
    return RunResult(generated, st)
