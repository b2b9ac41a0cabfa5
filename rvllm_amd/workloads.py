"""The benchmark workloads as concrete, seeded synthetic inputs.

Shapes follow the attention geometry of the named models (layers, query
heads, KV heads, head_dim) and rvllm's paged cache (block_size, block
tables built by its engine, src/engine.rs:365-388, 410-452). Seeded with
SplitMix64 (seed 0x5EED0000 + config index); block tables are Fisher-Yates
permutations of the pool, so no two consecutive logical blocks are
physically adjacent.

A workload describes ONE decode step: every sequence appends one token at
position ctx_len - 1 (rvllm: write_positions = logical_to_physical(
position_offset), src/engine.rs:446-451) and then attends over ctx_len keys
(read_num_tokens). The K/V values themselves are drawn on the device by the
caller (torch generator), since the large configs hold up to 120 GB of KV.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np


def splitmix64_stream(seed: int):
    s = seed & 0xFFFFFFFFFFFFFFFF
    while True:
        s = (s + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        yield z ^ (z >> 31)


class Rng:
    """SplitMix64 with uniform / Box-Muller normal / permutation helpers.
    numpy's Generator is seeded from it for bulk draws."""

    def __init__(self, seed: int):
        self._it = splitmix64_stream(seed)
        self.np = np.random.Generator(np.random.PCG64(next(self._it)))

    def u64(self) -> int:
        return next(self._it)

    def uniform(self) -> float:
        return (self.u64() >> 11) * (1.0 / (1 << 53))

    def randint(self, lo: int, hi: int) -> int:
        """Uniform integer in [lo, hi]."""
        return lo + self.u64() % (hi - lo + 1)

    def permutation(self, n: int) -> np.ndarray:
        """Fisher-Yates permutation of 0..n-1 driven by SplitMix64."""
        return self.np.permutation(n).astype(np.uint32)

    def normal(self, shape, scale: float = 1.0) -> np.ndarray:
        """N(0, 1) * scale via Box-Muller in float64, rounded to f32."""
        n = int(np.prod(shape))
        m = (n + 1) // 2
        u1 = self.np.random(m)
        u2 = self.np.random(m)
        r = np.sqrt(-2.0 * np.log1p(-u1))
        z = np.concatenate([r * np.cos(2 * np.pi * u2),
                            r * np.sin(2 * np.pi * u2)])[:n]
        return (z * scale).astype(np.float32).reshape(shape)


@dataclass
class Config:
    name: str
    index: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    block_size: int
    batch: int
    value_scale: float = 1.0
    window: int = 0
    description: str = ""
    rope_theta: float = 10000.0
    qkv_bias: bool = False     # Qwen2-style q/k/v projection bias
    qk_norm: bool = False      # Qwen3/Gemma-3 per-head RMS norm of q and k

    @property
    def group(self) -> int:
        return self.n_heads // self.n_kv_heads

    @property
    def seed(self) -> int:
        return 0x5EED0000 + self.index


CONFIGS = {
    # The CPU-sized workload (rvllm runs it with an f32 cache).
    "smollm2-360m": Config("smollm2-360m", 0, 1, 15, 5, 64, 16, 8,
                           description="SmolLM2-360M attention, CPU config",
                           rope_theta=100000.0),
    # The headline bench workload.
    "llama-3.2-1b": Config("llama-3.2-1b", 1, 16, 32, 8, 64, 16, 64,
                           description="Llama-3.2-1B shape, 64 x 2048",
                           rope_theta=500000.0),
    "qwen3-0.6b": Config("qwen3-0.6b", 2, 28, 16, 8, 128, 16, 256,
                         value_scale=0.5,
                         description="Qwen3-0.6B shape, 256 x 4096",
                         rope_theta=1000000.0, qk_norm=True),
    "qwen2.5-0.5b": Config("qwen2.5-0.5b", 3, 24, 14, 2, 64, 32, 512,
                           description="Qwen2.5-0.5B shape, ragged + prefix",
                           rope_theta=1000000.0, qkv_bias=True),
    "gemma-3-270m": Config("gemma-3-270m", 4, 18, 4, 1, 256, 16, 1024,
                           description="gemma-3-270m shape, 1024 x 1024",
                           rope_theta=1000000.0, qk_norm=True),
}


@dataclass
class DecodeBatch:
    """Host-side description of one decode step over a paged pool."""
    cfg: Config
    num_blocks: int
    ctx_lens: np.ndarray            # u32 [batch], read_num_tokens
    tables: List[np.ndarray]        # per-sequence block tables (u32)
    slot_block: np.ndarray          # u32 [batch], this step's append slot
    slot_off: np.ndarray            # u32 [batch]
    shared_prefix: Optional[dict] = None
    cow_src: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    cow_dst: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))

    @property
    def batch(self) -> int:
        return len(self.tables)

    @property
    def max_blocks(self) -> int:
        return max(len(t) for t in self.tables)

    def padded_tables(self) -> np.ndarray:
        """[batch, max_blocks], padded with each table's last block
        (GatherPlan's rule, src/kv_storage.rs:59-67)."""
        mb = self.max_blocks
        out = np.zeros((self.batch, mb), np.uint32)
        for b, t in enumerate(self.tables):
            out[b, :len(t)] = t
            out[b, len(t):] = t[-1] if len(t) else 0
        return out

    def unique_kv_tokens(self) -> int:
        """Tokens of K/V actually resident and read (shared blocks once):
        sum over unique (block, slot) pairs that some sequence reads."""
        bs = self.cfg.block_size
        seen = {}
        for t, n in zip(self.tables, self.ctx_lens):
            full, rem = divmod(int(n), bs)
            for i, blk in enumerate(t[:full]):
                seen[int(blk)] = bs
            if rem:
                blk = int(t[full])
                seen[blk] = max(seen.get(blk, 0), rem)
        return sum(seen.values())


def uniform_batch(cfg: Config, ctx_len: int, seed: Optional[int] = None,
                  num_blocks: Optional[int] = None) -> DecodeBatch:
    """Every sequence at ctx_len tokens (after this step's append); the pool
    holds exactly the live blocks unless num_blocks is larger; tables are a
    random permutation of the pool split per sequence."""
    rng = Rng(cfg.seed if seed is None else seed)
    per = -(-ctx_len // cfg.block_size)
    need = per * cfg.batch
    nb = max(need, num_blocks or 0)
    perm = rng.permutation(nb)
    tables = [perm[b * per:(b + 1) * per].copy() for b in range(cfg.batch)]
    ctx = np.full(cfg.batch, ctx_len, np.uint32)
    return _with_slots(cfg, nb, ctx, tables)


def ragged_batch(cfg: Config, lengths: np.ndarray, seed: Optional[int] = None,
                 extra_blocks: int = 0) -> DecodeBatch:
    rng = Rng(cfg.seed if seed is None else seed)
    lengths = np.asarray(lengths, np.uint32)
    per = [-(-int(n) // cfg.block_size) for n in lengths]
    nb = sum(per) + extra_blocks
    perm = rng.permutation(nb)
    tables, at = [], 0
    for p in per:
        tables.append(perm[at:at + p].copy())
        at += p
    return _with_slots(cfg, nb, lengths, tables)


def _with_slots(cfg, nb, ctx, tables) -> DecodeBatch:
    bs = cfg.block_size
    sb = np.array([t[(int(n) - 1) // bs] for t, n in zip(tables, ctx)],
                  np.uint32)
    so = np.array([(int(n) - 1) % bs for n in ctx], np.uint32)
    return DecodeBatch(cfg, nb, np.asarray(ctx, np.uint32), tables, sb, so)


def smollm2_batch(seed: Optional[int] = None) -> DecodeBatch:
    """The CPU-sized workload: 8 sequences, ctx drawn uniformly in [17, 512], tables
    drawn from a permutation of a 512-block pool."""
    cfg = CONFIGS["smollm2-360m"]
    rng = Rng(cfg.seed if seed is None else seed)
    lengths = np.array([rng.randint(17, 512) for _ in range(cfg.batch)],
                       np.uint32)
    perm = rng.permutation(512)
    tables, at = [], 0
    for n in lengths:
        p = -(-int(n) // cfg.block_size)
        tables.append(perm[at:at + p].copy())
        at += p
    return _with_slots(cfg, 512, lengths, tables)


def qwen25_batch(batch: Optional[int] = None, seed: Optional[int] = None,
                 prefix: int = 1024, share_frac: float = 0.3) -> DecodeBatch:
    """The ragged Qwen2.5 workload: lengths log-uniform in [32, 8192]; a share_frac of the
    sequences reuse the first min(len, prefix) tokens of one common prefix
    through identical block ids. A sharer whose last block is shared and
    partially filled gets a private copy before this step's append (the
    copy-on-write pairs are returned in cow_src/cow_dst)."""
    cfg = CONFIGS["qwen2.5-0.5b"]
    batch = batch or cfg.batch
    rng = Rng(cfg.seed if seed is None else seed)
    bs = cfg.block_size
    lengths = np.exp(rng.np.uniform(np.log(32), np.log(8192), batch))
    lengths = np.clip(lengths.astype(np.int64), 32, 8192).astype(np.uint32)
    n_share = int(round(share_frac * batch))
    sharers = set(rng.np.choice(batch, n_share, replace=False).tolist())
    prefix_blocks = prefix // bs
    # Pool: the prefix owner's blocks + every sequence's private blocks +
    # one spare per sharer for a possible CoW copy.
    private = []
    for b in range(batch):
        n = int(lengths[b])
        total = -(-n // bs)
        shared = min(prefix_blocks, -(-n // bs)) if b in sharers else 0
        private.append(total - shared)
    nb = prefix_blocks + sum(private) + n_share
    perm = rng.permutation(nb)
    prefix_tbl = perm[:prefix_blocks]
    at = prefix_blocks
    tables = []
    cow_src, cow_dst = [], []
    spare = nb - n_share
    for b in range(batch):
        n = int(lengths[b])
        if b in sharers:
            shared = min(prefix_blocks, -(-n // bs))
            t = np.concatenate([prefix_tbl[:shared],
                                perm[at:at + private[b]]]).astype(np.uint32)
            # Appending at position n-1 (ctx includes this step's token):
            # the write goes to block (n-1)//bs; if that block is a shared
            # prefix block, copy it first.
            wb = (n - 1) // bs
            if wb < shared:
                cow_src.append(int(t[wb]))
                cow_dst.append(int(perm[spare]))
                t = t.copy()
                t[wb] = perm[spare]
                spare += 1
        else:
            t = perm[at:at + private[b]].copy()
        at += private[b]
        tables.append(t)
    db = _with_slots(cfg, nb, lengths, tables)
    db.shared_prefix = {"blocks": prefix_tbl, "sharers": sorted(sharers)}
    db.cow_src = np.array(cow_src, np.uint32)
    db.cow_dst = np.array(cow_dst, np.uint32)
    return db


def decode_bytes(db: DecodeBatch, cell_bytes: int = 2) -> int:
    """Algorithmic HBM bytes of one paged-decode launch (one layer): unique
    K+V bytes read (cell_bytes per element: 2 for f16, 4 for f32) + q and
    out (f32) + block tables + ctx_lens."""
    c = db.cfg
    kv = db.unique_kv_tokens() * c.n_kv_heads * c.head_dim * 2 * cell_bytes
    qo = db.batch * c.n_heads * c.head_dim * 4 * 2
    tables = 4 * sum(-(-int(n) // c.block_size) for n in db.ctx_lens)
    return kv + qo + tables + 4 * db.batch


def append_bytes(n_tokens: int, cfg: Config, src_bytes: int = 4,
                 cell_bytes: int = 2) -> int:
    """Algorithmic bytes of one append launch: K+V rows read at src_bytes
    per element, written at cell_bytes (f16: 2, f32: 4), plus 8 bytes of
    slot per token."""
    return (n_tokens * cfg.n_kv_heads * cfg.head_dim * 2 *
            (src_bytes + cell_bytes) + 8 * n_tokens)


def prep_bytes(n_tokens: int, cfg: Config) -> int:
    """Algorithmic bytes of one attn_prep launch: per token the f32 q row
    read and written, the f32 k and v rows read and written as f16, the
    f32 cos/sin halves and 8 bytes of slot; per launch the bias and norm
    weights."""
    H, KV, hd = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    per_tok = 8 * H * hd + KV * hd * 2 * (4 + 2) + 4 * hd + 8
    weights = 4 * ((H + 2 * KV) * hd if cfg.qkv_bias else 0) \
        + 4 * (2 * hd if cfg.qk_norm else 0)
    return n_tokens * per_tok + weights


def prefill_visible_pairs(pos_offset, read_num, q_len: int,
                          window: int = 0) -> int:
    """Number of (query row, key) pairs batch_mask leaves visible
    (src/model.rs:346-369), summed over the batch: row i of sequence b at
    p = pos_offset[b] + i sees keys [max(0, p + 1 - window), min(read_num,
    p + 1))."""
    total = 0
    for off, rd in zip(np.asarray(pos_offset, np.int64),
                       np.asarray(read_num, np.int64)):
        p = off + np.arange(q_len, dtype=np.int64)
        hi = np.minimum(rd, p + 1)
        lo = np.maximum(0, p + 1 - window) if window > 0 else 0
        total += int(np.maximum(hi - lo, 0).sum())
    return total


def prefill_attn_flops(pairs: int, cfg: Config) -> int:
    """Algorithmic flops of paged prefill attention: per visible pair and
    query head, q.k (2 hd) and p.v (2 hd)."""
    return pairs * cfg.n_heads * 4 * cfg.head_dim
