"""Writes tests/golden/kats.json: the reference's known-answer vectors for the
paged-KV path, plus float64 expectations for the reference's paged-attention
test cases.

Nothing here imports or runs the reference (it is Rust; there is no
toolchain). Two kinds of vectors:

1. Literal known answers from the reference's own tests, transcribed with
   their file:line (inputs and expected outputs are the numbers written in
   those tests).
2. The six shape cases of ``attn_decode_matches_reference``
   (src/metal/ops.rs:676-766): inputs come from that test's deterministic
   xorshift generator (src/metal/ops.rs:513-525, restated in ``values``),
   block tables are its reversed permutations, sequence b has ctx - 2b real
   tokens and the last q_len of them are queries (causal). The expected
   outputs are computed here by an independent float64 brute force in numpy,
   exactly as that test computes ``want``.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# (n_kv_heads, group, head_dim, batch, q_len, ctx_len), src/metal/ops.rs:684-691
METAL_CASES = [
    (2, 3, 64, 2, 1, 100),
    (2, 5, 64, 2, 1, 40),
    (1, 9, 32, 1, 2, 33),
    (2, 2, 6, 3, 2, 17),
    (1, 4, 128, 2, 3, 70),
    (2, 2, 200, 1, 1, 300),
]
METAL_BLOCK_SIZE = 16


def values(n: int, seed: int) -> np.ndarray:
    """xorshift32 values in [-1, 1) (src/metal/ops.rs:513-525): state =
    seed*2654435761 + 12345 (wrapping u32); per value state ^= state<<13,
    >>17, <<5; value = (state as f32 / u32::MAX as f32) * 2 - 1 in f32."""
    state = (seed * 2654435761 + 12345) & 0xFFFFFFFF
    out = np.empty(n, dtype=np.float32)
    denom = np.float32(4294967295.0)  # u32::MAX as f32 == 2^32
    for i in range(n):
        state ^= (state << 13) & 0xFFFFFFFF
        state ^= state >> 17
        state ^= (state << 5) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(state) / denom) * np.float32(2.0) \
            - np.float32(1.0)
    return out


def metal_case_inputs(case: int):
    """Inputs of case `case`: dict with q [rows, n_heads*hd], cache_k/v
    [num_blocks, bs, n_kv, hd] (f32), block_idx [batch*max_blocks], mask."""
    n_kv, group, hd, batch, q_len, ctx = METAL_CASES[case]
    bs = METAL_BLOCK_SIZE
    n_heads = n_kv * group
    rows = batch * q_len
    max_blocks = -(-ctx // bs)
    num_blocks = batch * max_blocks
    block_idx = np.array([num_blocks - 1 - (b * max_blocks + i)
                          for b in range(batch) for i in range(max_blocks)],
                         dtype=np.uint32)
    q = values(rows * n_heads * hd, 10 + case)
    ck = values(num_blocks * bs * n_kv * hd, 20 + case)
    cv = values(num_blocks * bs * n_kv * hd, 30 + case)
    mask = np.zeros(rows * ctx, dtype=np.float32)
    for b in range(batch):
        valid = ctx - 2 * b
        for qi in range(q_len):
            for j in range(ctx):
                if j >= valid or j + q_len > valid + qi:
                    mask[(b * q_len + qi) * ctx + j] = -np.inf
    return dict(n_kv=n_kv, group=group, hd=hd, batch=batch, q_len=q_len,
                ctx=ctx, bs=bs, n_heads=n_heads, max_blocks=max_blocks,
                num_blocks=num_blocks, block_idx=block_idx, q=q,
                cache_k=ck.reshape(num_blocks, bs, n_kv, hd),
                cache_v=cv.reshape(num_blocks, bs, n_kv, hd),
                mask=mask.reshape(rows, ctx))


def metal_case_expected(c) -> np.ndarray:
    """float64 brute force, as src/metal/ops.rs:719-745 computes `want`."""
    n_heads, hd, bs = c["n_heads"], c["hd"], c["bs"]
    q = c["q"].astype(np.float64).reshape(-1, n_heads, hd)
    ck = c["cache_k"].astype(np.float64)
    cv = c["cache_v"].astype(np.float64)
    scale = np.float64(np.float32(1.0) / np.sqrt(np.float32(hd)))
    want = np.zeros((c["batch"] * c["q_len"], n_heads, hd))
    for b in range(c["batch"]):
        blocks = c["block_idx"][b * c["max_blocks"]:(b + 1) * c["max_blocks"]]
        pos = np.arange(c["ctx"])
        blk = blocks[pos // bs].astype(np.int64)
        for qi in range(c["q_len"]):
            row = b * c["q_len"] + qi
            for h in range(n_heads):
                kvh = h // c["group"]
                K = ck[blk, pos % bs, kvh]  # [ctx, hd]
                V = cv[blk, pos % bs, kvh]
                s = (K @ q[row, h]) * scale + c["mask"][row].astype(np.float64)
                e = np.exp(s - s.max())
                want[row, h] = (e @ V) / e.sum()
    return want.astype(np.float32)


def reference_kats():
    """Literal known answers of the reference's tests."""
    return {
        # src/kv_storage.rs:193-224, src/cuda/kv_storage.rs:178-219,
        # src/cuda/ops.rs:1220-1259: 3 blocks x 2 slots, n_kv 1, hd 2.
        "round_trip_across_blocks": {
            "source": "src/kv_storage.rs:193-224",
            "num_blocks": 3, "block_size": 2, "n_kv": 1, "hd": 2,
            "k": [10.0, 10.5, 11.0, 11.5, 12.0, 12.5, 20.0, 20.5],
            "block_ids": [0, 0, 1, 2], "offsets": [0, 1, 0, 0],
            "tables": [[0, 1], [2]], "n_tokens": [3, 1],
            "plan_block_idx": [0, 1, 2, 2],  # src/cuda/ops.rs:1222-1226
            "ctx_len": 3,
            "gather_prefix_a": [10.0, 10.5, 11.0, 11.5, 12.0, 12.5],
            "gather_prefix_b": [20.0, 20.5],
            # raw cache after the write, src/cuda/ops.rs:1106-1114
            "raw_cache": [10.0, 10.5, 11.0, 11.5, 12.0, 12.5, 0.0, 0.0,
                          20.0, 20.5, 0.0, 0.0],
        },
        # src/kv_storage.rs:226-237, src/cuda/ops.rs:1117-1157
        "untouched_slots": {
            "source": "src/kv_storage.rs:226-237",
            "num_blocks": 1, "block_size": 4, "n_kv": 1, "hd": 2,
            "k": [1.0, 1.5], "block_ids": [0], "offsets": [2],
            "tables": [[0]], "n_tokens": [4],
            "gather": [0.0, 0.0, 0.0, 0.0, 1.0, 1.5, 0.0, 0.0],
        },
        # src/kv_storage.rs:239-255
        "clone_independence": {
            "source": "src/kv_storage.rs:239-255",
            "num_blocks": 1, "block_size": 2, "n_kv": 1, "hd": 2,
            "k": [1.0, 1.5], "block_ids": [0], "offsets": [0],
            "after_write": [1.0, 1.5], "snapshot": [0.0, 0.0],
        },
        # src/model.rs:879-923, src/cuda/cublas_ops.rs:263-352 (tol 1e-2)
        "gqa_hand_computed": {
            "source": "src/model.rs:879-923",
            "batch": 1, "n_heads": 2, "n_kv": 1, "q_len": 2, "ctx_len": 2,
            "hd": 2,
            "k": [1.0, 0.0, 0.0, 1.0], "v": [10.0, 0.0, 0.0, 20.0],
            "q": [1.0, 0.0, 1.0, 0.0, 0.0, 1.0, 0.0, 1.0],
            "position_offset": [0], "read_num_tokens": [2],
            "expected": [10.0, 0.0, 6.698, 6.604, 10.0, 0.0, 3.302, 13.396],
            "tol": 1e-2,
        },
        # src/model.rs:1184-1197: window 2, four queries from position 0.
        "mask_window": {
            "source": "src/model.rs:1184-1197",
            "position_offset": [0], "read_num_tokens": [4], "q_len": 4,
            "ctx_len": 4, "window": 2,
            "expected": [[0, "-inf", "-inf", "-inf"], [0, 0, "-inf", "-inf"],
                         ["-inf", 0, 0, "-inf"], ["-inf", "-inf", 0, 0]],
        },
        # src/model.rs:951-975 shape: 2 seqs (5 and 3 real tokens padded to
        # 5), 4 q heads over 2 kv heads, q_len 2 at offsets 3 and 1; the
        # reference checks against a naive per-head computation at 1e-5.
        "naive_per_head_shape": {
            "source": "src/model.rs:951-975",
            "batch": 2, "n_heads": 4, "n_kv": 2, "q_len": 2, "ctx_len": 5,
            "hd": 4, "position_offset": [3, 1], "read_num_tokens": [5, 3],
            "tol": 1e-5,
        },
    }


def main() -> None:
    metal = []
    for i in range(len(METAL_CASES)):
        c = metal_case_inputs(i)
        metal.append({
            "case": i,
            "shape": list(METAL_CASES[i]),
            "source": "src/metal/ops.rs:676-766",
            "expected": metal_case_expected(c).reshape(-1).tolist(),
            "tol": 1e-4,
        })
    doc = {"reference_kats": reference_kats(), "metal_attn_decode": metal}
    path = os.path.join(HERE, "kats.json")
    with open(path, "w") as f:
        json.dump(doc, f)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
