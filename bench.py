"""Benchmark of the paged KV-cache decode path on one MI355X.

A step is one decode step of the whole model's KV path: for every layer,
append each sequence's new K/V row (f32 source rounded to f16) into its
slot, then paged GQA decode attention over the full context. Inputs are
resident in HBM before the timed region. Prints one JSON line.

Default workload: the Qwen3-0.6B shape at the target size (28 layers, 16 q
heads / 8 KV heads, head_dim 128, block_size 16, 256 sequences x 4096
tokens: a 112 GiB pool, block tables a random permutation of a pool sized
for exactly the live tokens) - the largest single-GPU config. Other configs:
--config llama-3.2-1b (64 x 2048; --batch 256 --ctx 4096 for the target
size) | gemma-3-270m | qwen2.5-0.5b.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16/bf16, no sparsity
METRIC = "paged-decode attn HBM GB/s (% of peak) + decode tok/s, 1 MI355X"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default=None,
                   help="workload (default: qwen3-0.6b; gemma-3-270m for "
                   "--churn; qwen2.5-0.5b for --cow)")
    p.add_argument("--batch", type=int, default=0,
                   help="override the number of sequences (uniform configs)")
    p.add_argument("--ctx", type=int, default=0,
                   help="context length of the uniform configs (llama, "
                   "qwen3, gemma); 0 = the config's own")
    p.add_argument("--no-cpu", action="store_true",
                   help="skip the CPU baseline leg")
    p.add_argument("--no-secondary", dest="secondary", action="store_false",
                   help="default run only: skip the secondary records "
                   "(Llama-3.2-1B 256 x 4096, the Qwen3 prefill append, the "
                   "200-step churn)")
    p.add_argument("--f32-cache", dest="f32_cache", action="store_true",
                   default=None,
                   help="f32 cache cells, the reference's own (default for "
                   "smollm2-360m, whose reference path is f32; else f16)")
    p.add_argument("--f16-cache", dest="f32_cache", action="store_false")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="wall-clock budget of the CPU baseline sample")
    p.add_argument("--plan", dest="plan", action="store_true", default=None,
                   help="decode through a per-step decode plan (default: "
                        "only for ragged batches)")
    p.add_argument("--no-plan", dest="plan", action="store_false")
    p.add_argument("--unfused", action="store_true",
                   help="append and decode as two launches per layer "
                        "(rvkv_append + rvkv_paged_decode) instead of the "
                        "fused rvkv_decode_step")
    p.add_argument("--churn", action="store_true",
                   help="continuous-batching churn (gemma-3-270m shape): each "
                        "step 10%% of sequences finish and as many are "
                        "admitted with 64-token prompts, over a fragmented "
                        "pool; --steps counts engine steps")
    p.add_argument("--prefill", choices=["f32", "f16"], default=None,
                   help="time the prefill append instead (Qwen3 shape: "
                        "every sequence's whole context scattered into the "
                        "paged cache, all layers; source dtype f32 or f16)")
    p.add_argument("--prefill-attn", action="store_true",
                   help="time whole-prompt paged prefill attention over the "
                   "uniform batch of --config (default batch 16)")
    p.add_argument("--gather", choices=["f32", "f16"], default=None,
                   help="time the block-table gather (rvkv_gather) of the "
                        "decode workload of --config into rvllm's padded "
                        "[batch, n_kv, ctx, hd] layout, all layers")
    p.add_argument("--cow", action="store_true",
                   help="time the copy-on-write block copy (rvkv_copy_blocks, "
                        "all layers, K and V) of the prefix sharers' pairs of "
                        "--config (default qwen2.5-0.5b), or of --cow-blocks "
                        "random pairs")
    p.add_argument("--cow-blocks", type=int, default=0)
    p.add_argument("--engine", action="store_true",
                   help="run the continuous-batching engine (native scheduler "
                        "+ GPU attention-only model of --config's attention "
                        "shape) over a request set with shared prefixes; "
                        "reports output tok/s")
    p.add_argument("--prep", action="store_true",
                   help="time the fused attention prep + append over the "
                   "prefill batch of --config instead")
    p.add_argument("--graph", action="store_true",
                   help="time the step as one HIP graph replay (all layers' "
                        "append + decode launches captured once)")
    p.add_argument("--traffic-pass", action="store_true",
                   help="internal: a short headline decode after a 2 GiB "
                        "device copy, run under rocprofv3 --pmc by the "
                        "default run to measure HBM traffic per launch")
    p.add_argument("--no-traffic", dest="traffic", action="store_false",
                   help="default run only: skip the live counter passes "
                        "(traffic then comes from profiles/)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only time a plain 2 GiB device-to-device copy (the "
                        "achievable-bandwidth and PMC-counter reference)")
    a = p.parse_args()
    if a.config is None:
        a.config = ("gemma-3-270m" if a.churn else
                    "qwen2.5-0.5b" if a.cow else "qwen3-0.6b")
    return a


def copy_calibration(torch, steps):
    """Times torch's device copy of a 2 GiB buffer into another: 4 GiB of
    HBM traffic per launch (read + write)."""
    n = (2 << 30) // 4
    a = torch.randn(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    print(json.dumps({"copy_calibration": {
        "bytes_per_launch": 2 * n * 4, "avg_launch_ms": round(ms, 4),
        "GB/s": round(2 * n * 4 / (ms * 1e-3) / 1e9, 1)}}), flush=True)


def read_ceiling(torch, nbytes, steps):
    """The plain streaming-read rate at one launch's size: the read probe
    (16-byte non-temporal loads, 16384 contiguous slices, nothing written)
    timed with HIP
    events over buffers of `nbytes`, rotated so at least 1.5 GiB separates
    two reads of one buffer (no MALL reuse, as for the layer launches)."""
    import ctypes

    from rvllm_amd import _lib
    lib = _lib.load_calib()
    nb = (int(nbytes) + 15) // 16 * 16
    n_buf = max(2, -(-(3 << 29) // nb))
    bufs = [torch.zeros(nb // 4, dtype=torch.int32, device="cuda")
            for _ in range(n_buf)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def sweep(wg):
        for b in bufs:
            _lib.check_calib(lib.rvkv_calib_read_probe(
                ctypes.c_void_p(b.data_ptr()), nb, wg, None, stream))

    # The best workgroup count depends on the size: the best of three.
    best = None
    for wg in (2048, 16384, 65536):
        sweep(wg)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            sweep(wg)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / (steps * n_buf)
        if best is None or ms < best[0]:
            best = (ms, wg)
    del bufs
    ms, wg = best
    return {"bytes_per_launch": nb, "avg_launch_ms": round(ms, 5),
            "GB/s": round(nb / (ms * 1e-3) / 1e9, 2), "workgroups": wg}


def paged_ceiling(torch, nbytes, tile_bytes, steps):
    """The plain read of a paged layer: every tile (tile_bytes, one
    (block, head) tile of the cache) of a buffer of `nbytes` read once in a
    random order, as a decode reads a randomly permuted pool, one wave per
    workgroup with eight 1 KB loads in flight, nothing computed (the paged
    probe). Buffers rotate so no launch finds its data in the MALL; the best
    of two workgroup counts."""
    import ctypes

    from rvllm_amd import _lib
    lib = _lib.load_calib()
    n_ids = max(1, int(nbytes) // tile_bytes)
    nb = n_ids * tile_bytes
    n_buf = max(2, -(-(3 << 29) // nb))
    bufs = [torch.zeros(nb // 4, dtype=torch.int32, device="cuda")
            for _ in range(n_buf)]
    rng = np.random.default_rng(7)
    ids = [torch.from_numpy(rng.permutation(n_ids).astype(np.int32)).cuda()
           for _ in range(n_buf)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def sweep(wg):
        for b, t in zip(bufs, ids):
            _lib.check_calib(lib.rvkv_calib_paged_probe(
                ctypes.c_void_p(b.data_ptr()), tile_bytes,
                ctypes.c_void_p(t.data_ptr()), n_ids, wg, stream))

    best = None
    for wg in (2048, 8192):
        sweep(wg)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            sweep(wg)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / (steps * n_buf)
        if best is None or ms < best[0]:
            best = (ms, wg)
    del bufs, ids
    ms, wg = best
    return {"bytes_per_launch": nb, "tile_bytes": tile_bytes,
            "avg_launch_ms": round(ms, 5),
            "GB/s": round(nb / (ms * 1e-3) / 1e9, 2), "workgroups": wg}


def copy_ceiling(torch, nbytes, read_frac, steps):
    """The plain streaming-copy rate at one launch's size and read/write mix:
    the copy probe (16-byte non-temporal loads and stores, contiguous on both
    sides) moving `nbytes` in total, split read:write as 2:1, 1:1 or 1:2
    (whichever is nearest read_frac), over buffers rotated so no launch
    finds its data in the MALL."""
    import ctypes

    from rvllm_amd import _lib
    lib = _lib.load_calib()
    ra, wa = min(((2, 1), (1, 1), (1, 2)),
                 key=lambda r: abs(r[0] / (r[0] + r[1]) - read_frac))
    unit = 32 * ra * wa  # keeps both sides whole 16-byte units
    rd = int(nbytes) * ra // (ra + wa) // unit * unit
    wr = rd * wa // ra
    n_buf = max(2, -(-(3 << 29) // (rd + wr)))
    srcs = [torch.zeros(rd // 4, dtype=torch.int32, device="cuda")
            for _ in range(n_buf)]
    dsts = [torch.empty(wr // 4, dtype=torch.int32, device="cuda")
            for _ in range(n_buf)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def sweep(wg):
        for a, b in zip(srcs, dsts):
            _lib.check_calib(lib.rvkv_calib_copy_probe(
                ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                rd, wr, wg, stream))

    # The best workgroup count varies with size and mix (and is noisy): the
    # best of five.
    best = None
    for wg in (2048, 4096, 16384, 65536, 262144):
        sweep(wg)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            sweep(wg)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / (steps * n_buf)
        if best is None or ms < best[0]:
            best = (ms, wg)
    del srcs, dsts
    ms, wg = best
    return {"read_bytes": rd, "write_bytes": wr, "avg_launch_ms": round(ms, 5),
            "GB/s": round((rd + wr) / (ms * 1e-3) / 1e9, 2), "workgroups": wg}


def with_copy_ceiling(torch, res, read_frac, steps):
    """Adds roofline.stream_copy_ceiling (and the launch's fraction of it)
    to a byte mover's record."""
    r = res["roofline"]
    cc = copy_ceiling(torch, r["algorithmic_bytes_per_launch"], read_frac,
                      steps)
    cc["frac"] = round(r["achieved"] / cc["GB/s"], 4)
    r["stream_copy_ceiling"] = cc
    return res


def measured_traffic(config, batch, unfused, ctx=0):
    """HBM bytes per decode launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, each scaled by the same counter's reading for a copy of
    known size) for this workload, from the committed summary, or None."""
    if batch or ctx:
        return None
    if unfused:
        return None
    name = "decode_step_traffic.json"
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            rec = json.load(f).get(config)
    except (OSError, ValueError):
        return None
    return rec.get("traffic_bytes_per_launch") if rec else None


def build_workload(W, name, batch=0, ctx=0):
    c = W.CONFIGS[name]
    if batch:
        import dataclasses
        c = dataclasses.replace(c, batch=batch)
    if name == "llama-3.2-1b":
        return W.uniform_batch(c, ctx or 2048)
    if name == "qwen3-0.6b":
        return W.uniform_batch(c, ctx or 4096)
    if name == "gemma-3-270m":
        return W.uniform_batch(c, ctx or 1024)
    if name == "qwen2.5-0.5b":
        return W.qwen25_batch(batch=c.batch)
    if name == "smollm2-360m":
        return W.smollm2_batch()
    raise SystemExit(f"unknown config {name}")


def fill_pool(torch, st, seed, scale):
    """Writes N(0,1)*scale f16 rows into every slot of every layer through
    the append kernel (f16 source), drawn on the device."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    bs, nkv, hd = st.block_size, st.n_kv_heads, st.head_dim
    total = st.num_blocks * bs
    chunk = max(1, (1 << 28) // (nkv * hd * 2))  # 256 MiB of f16 per tensor
    for layer in range(st.n_layers):
        for t0 in range(0, total, chunk):
            n = min(chunk, total - t0)
            s = torch.arange(t0, t0 + n, device="cuda", dtype=torch.int64)
            blk = (s // bs).to(torch.int32)
            off = (s % bs).to(torch.int32)
            k = torch.randn((n, nkv, hd), generator=g, device="cuda",
                            dtype=torch.float16)
            v = torch.randn((n, nkv, hd), generator=g, device="cuda",
                            dtype=torch.float16)
            if scale != 1.0:
                k.mul_(scale)
                v.mul_(scale)
            st.write_tokens(layer, blk, off, k, v)
        torch.cuda.synchronize()


def sample_batch(W, db, n_seq):
    """The first n_seq sequences of db over a compact pool: their blocks
    (shared ones once) renumbered 0..n-1 in first-use order. Returns the
    sub-batch and the original ids of its blocks."""
    tabs = db.tables[:n_seq]
    ids = []
    remap = {}
    for t in tabs:
        for blk in t:
            if int(blk) not in remap:
                remap[int(blk)] = len(ids)
                ids.append(int(blk))
    new_tabs = [np.array([remap[int(x)] for x in t], np.uint32) for t in tabs]
    ctx = np.asarray(db.ctx_lens[:n_seq], np.uint32)
    sub = W.DecodeBatch(db.cfg, len(ids), ctx, new_tabs,
                        np.array([remap[int(x)] for x in
                                  db.slot_block[:n_seq]], np.uint32),
                        np.asarray(db.slot_off[:n_seq], np.uint32))
    return sub, np.asarray(ids, np.uint32)


def cpu_baseline(orc, W, st, db, budget_s, f32=False):
    """The oracle's restatement of rvllm's CPU decode path (append + padded
    gather + batch_mask + gqa_attention, f32 math over the cache) on the
    host cores: layer 0 of a bounded sample of the same workload (its first
    sequences, the cache blocks they read copied from the GPU pool),
    repeated within budget_s, on every core this process may run on, and a
    shorter single-thread sample. Returns the cpu_baseline dict; tok/s is
    extrapolated to the whole batch and every layer."""
    import torch
    c = db.cfg
    threads = len(os.sched_getaffinity(0))
    # About 1 s of multi-threaded work per repetition at ~10 GB/s; the
    # single-thread leg uses an eighth of that sample.
    cell = 4 if f32 else 2
    full_bytes = W.decode_bytes(db, cell)
    n_seq = db.batch
    while n_seq > 1 and full_bytes * n_seq / db.batch > 2e9:
        n_seq //= 2
    n_seq = max(n_seq, min(db.batch, threads))

    def prepare(n):
        sub, ids = sample_batch(W, db, n)
        cache = orc.KvCache(sub.num_blocks, c.block_size, c.n_kv_heads,
                            c.head_dim, orc.F32 if f32 else orc.F16)
        dev_ids = torch.from_numpy(ids.view(np.int32)).cuda()
        for which, dst in ((0, cache.k), (1, cache.v)):
            blocks = st.read_blocks(0, which, dev_ids).cpu()
            if f32:
                dst[:] = blocks.numpy()
            else:
                dst[:] = blocks.view(torch.int16).numpy().view(np.uint16)
        rng = W.Rng(c.seed + 99)
        nk = rng.normal((n, c.n_kv_heads, c.head_dim))
        nv = rng.normal((n, c.n_kv_heads, c.head_dim))
        q = rng.normal((n, c.n_heads, c.head_dim))
        return sub, cache, nk, nv, q

    def timed(sub, cache, nk, nv, q, nthr, budget, max_reps):
        idx = sub.padded_tables().reshape(-1)
        reps, t_total = 0, 0.0
        while reps < 1 or (t_total < budget and reps < max_reps):
            t0 = time.perf_counter()
            orc.decode_step(cache, sub.slot_block, sub.slot_off, nk, nv, idx,
                            sub.max_blocks, sub.ctx_lens, q, n_threads=nthr)
            t_total += time.perf_counter() - t0
            reps += 1
        return t_total / reps, reps

    sub, cache, nk, nv, q = prepare(n_seq)
    per_rep, reps = timed(sub, cache, nk, nv, q, threads, budget_s, 1000)
    sub_bytes = (W.decode_bytes(sub, cell) +
                 W.append_bytes(sub.batch, c, cell_bytes=cell))
    gbs = sub_bytes / per_rep / 1e9
    n1 = max(1, n_seq // 8)
    sub1, cache1, nk1, nv1, q1 = prepare(n1)
    per_rep1, reps1 = timed(sub1, cache1, nk1, nv1, q1, 1,
                            min(3.0, budget_s / 4), 100)
    sub1_bytes = (W.decode_bytes(sub1, cell) +
                  W.append_bytes(sub1.batch, c, cell_bytes=cell))
    # Whole batch, all layers, at the sample's rate.
    layer_bytes = (W.decode_bytes(db, cell) +
                   W.append_bytes(db.batch, c, cell_bytes=cell))
    layer_s = layer_bytes / (gbs * 1e9)
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": threads,
        "host_cpu_count": os.cpu_count(),
        "kind": "port",
        "sample": (f"oracle decode_step (rvllm CPU path restated in C: "
                   f"write_tokens + padded gather + batch_mask + "
                   f"gqa_attention, f32 math over "
                   f"{'f32' if f32 else 'f16'} cells) on layer 0 of the "
                   f"first {n_seq} of "
                   f"{db.batch} sequences of the same workload, "
                   f"{reps} repetitions of {per_rep * 1e3:.1f} ms on "
                   f"{threads} threads; tok/s extrapolated to {db.batch} "
                   f"sequences x {c.n_layers} layers"),
        "tok_per_s": round(db.batch / (layer_s * c.n_layers), 2),
        "ms_per_layer": round(layer_s * 1e3, 3),
        "single_thread": {
            "value": round(sub1_bytes / per_rep1 / 1e9, 3),
            "sample_sequences": n1,
            "ms_per_repetition": round(per_rep1 * 1e3, 3),
            "repetitions": reps1,
        },
    }


def prompt_slots(torch, db):
    """Device slot lists (block id, offset) of every prompt token of the
    batch, in sequence order, plus each token's position."""
    bs = db.cfg.block_size
    sb, so, ps = [], [], []
    for t, n in zip(db.tables, db.ctx_lens):
        pos = np.arange(int(n))
        sb.append(np.asarray(t, np.uint32)[pos // bs])
        so.append((pos % bs).astype(np.uint32))
        ps.append(pos)
    dev = lambda a: torch.from_numpy(np.concatenate(a).view(np.int32)).cuda()
    return dev(sb), dev(so), np.concatenate(ps)


def run_prefill_attn(args, torch, W):
    """Whole-prompt prefill attention over the paged cache: every sequence
    of the config's uniform batch (its prompt already in the cache, as
    after the prefill append) attends causally from all ctx positions,
    pos_offset 0 and read_num = ctx, one rvkv_paged_prefill per layer.
    Matrix-core bound: priced in flops against the f16 dense MFMA peak."""
    from rvllm_amd.kv_storage import HipKvStorage
    batch = args.batch or 16
    db = build_workload(W, args.config, batch, args.ctx)
    c = db.cfg
    if len(set(int(x) for x in db.ctx_lens)) != 1:
        raise SystemExit("--prefill-attn needs a uniform-length config")
    L = int(db.ctx_lens[0])
    st = HipKvStorage(c.n_layers, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim)
    fill_pool(torch, st, c.seed, c.value_scale)
    tables = torch.from_numpy(db.padded_tables().view(np.int32)).cuda()
    zero = torch.zeros(db.batch, dtype=torch.int32, device="cuda")
    read = torch.full((db.batch,), L, dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(c.seed + 1)
    q = torch.randn((db.batch, L, c.n_heads, c.head_dim), generator=g,
                    device="cuda")
    out = torch.empty_like(q)
    window = c.window

    def step():
        for layer in range(c.n_layers):
            st.paged_prefill(layer, q, tables, zero, read, out=out,
                             window=window)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    launch_ms = e0.elapsed_time(e1) / (args.steps * c.n_layers)
    pairs = W.prefill_visible_pairs(np.zeros(db.batch), db.ctx_lens, L,
                                    window)
    flops = W.prefill_attn_flops(pairs, c)
    achieved = flops / (launch_ms * 1e-3) / 1e12
    kv_bytes = int(db.ctx_lens.astype(np.int64).sum()) * c.n_kv_heads * \
        c.head_dim * 4
    qo_bytes = db.batch * L * c.n_heads * c.head_dim * 8
    res = {
        "metric": "paged prefill attention TFLOP/s, 1 MI355X",
        "value": round(flops * c.n_layers / dt / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA, f32 accumulate (f32 q/out, f16 cache)",
        "data": "synthetic N(0,1)*scale KV and q, seeded permuted tables",
        "config": {
            "workload": f"{c.name} whole-prompt prefill attention: "
                        f"{db.batch} seqs x {L} tokens, causal, "
                        f"{c.n_layers} layers, {c.n_heads} q / "
                        f"{c.n_kv_heads} kv heads, head_dim {c.head_dim}, "
                        f"block_size {c.block_size}",
            "global_batch": db.batch,
            "seq_len": L,
            "parallelism": "single GPU",
        },
        "tok_per_s": round(db.batch * L / dt, 1),
        "roofline": {
            "bound": "mfma",
            "kernel": f"prefill_kernel<{c.head_dim}>",
            "achieved": round(achieved, 2),
            "peak": MFMA_F16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
            "traffic": None,
            "algorithmic_flops_per_launch": flops,
            "min_hbm_bytes_per_launch": kv_bytes + qo_bytes,
            "avg_launch_ms": round(launch_ms, 5),
        },
    }
    print(json.dumps(res), flush=True)


def _time_launches(torch, fn, n_launch, steps, warmup):
    """(wall seconds per step, HIP-event ms per launch) of `steps` calls of
    fn (each making n_launch launches) after `warmup` untimed ones."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    return dt, e0.elapsed_time(e1) / (steps * n_launch)


def _hbm_line(metric, value_bytes_per_step, dt, launch_ms, per_launch,
              kernel, args, config, dtype):
    achieved = per_launch / (launch_ms * 1e-3) / 1e9
    return {
        "metric": metric,
        "value": round(value_bytes_per_step / dt / 1e9, 2),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic N(0,1)*scale f16 KV, seeded permuted block tables",
        "config": config,
        "roofline": {"bound": "hbm", "kernel": kernel,
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "algorithmic_bytes_per_launch": per_launch,
                     "avg_launch_ms": round(launch_ms, 5)},
    }


def run_engine(args, torch, W):
    """The serving loop end to end: rvllm_amd.engine.run (admission with
    prefix-cache reuse, one prefill forward per admitted request, batched
    decode forwards, recompute preemption) over the native scheduler, with
    the GPU backend of rvllm_amd.attn_model: an attention-only decoder with
    --config's attention shape (layers, heads, head_dim, block_size), a
    2048-wide residual stream and a 32000-token vocabulary, seeded random
    weights. Requests: --batch (default 64) prompts of 512 tokens, 30 %
    opening with one shared 256-token prefix, 64 new tokens each, all
    arriving at step 0. --steps counts repetitions of the whole run."""
    from rvllm_amd.attn_model import AttnModelConfig, HipBackend, init_weights
    from rvllm_amd.engine import EngineConfig, RequestSpec, run
    c = W.CONFIGS[args.config]
    n_req = args.batch or 64
    prompt, new_tok, shared_len = 512, 64, 256
    mcfg = AttnModelConfig(
        vocab=32000, hidden=2048, n_layers=c.n_layers, n_heads=c.n_heads,
        n_kv_heads=c.n_kv_heads, head_dim=c.head_dim,
        qkv_bias=c.qkv_bias, qk_norm=c.qk_norm, rope_theta=c.rope_theta,
        context_length=4096, seed=c.seed)
    bs = c.block_size
    num_blocks = n_req * (-(-(prompt + new_tok) // bs)) + 64
    backend = HipBackend(mcfg, init_weights(mcfg), num_blocks, bs)
    rng = np.random.default_rng(c.seed)
    shared = rng.integers(0, mcfg.vocab, shared_len).tolist()
    specs = []
    for i in range(n_req):
        head = shared if rng.random() < 0.3 else []
        tail = rng.integers(0, mcfg.vocab, prompt - len(head)).tolist()
        specs.append(RequestSpec(head + tail, new_tok))
    ecfg = EngineConfig(block_size=bs, num_blocks=num_blocks)
    import gc
    gc.collect()
    gc.freeze()  # start-up objects out of the collector's view (as churn)
    for _ in range(max(args.warmup, 1)):
        run(backend, specs[:4], ecfg)
    torch.cuda.synchronize()
    res_runs = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        res_runs.append(run(backend, specs, ecfg))
    dt = (time.perf_counter() - t0) / args.steps
    st = res_runs[-1].stats
    out_tok = st.output_tokens
    res = {
        "metric": "engine output tok/s (attention-only model), 1 MI355X",
        "value": round(out_tok / dt, 1),
        "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 KV, f32 activations",
        "data": "synthetic prompts (30 % share a 256-token prefix), seeded "
                "random weights",
        "config": {
            "workload": f"{c.name} attention shape: {c.n_layers} layers, "
                        f"{c.n_heads} q / {c.n_kv_heads} kv heads, head_dim "
                        f"{c.head_dim}, block_size {bs}; hidden 2048, vocab "
                        f"32000; {n_req} requests x {prompt} prompt + "
                        f"{new_tok} new tokens",
            "global_batch": n_req, "seq_len": prompt + new_tok,
            "parallelism": "single GPU"},
        "engine": {
            "engine_steps": st.steps, "output_tokens": out_tok,
            "prefill_tokens": st.prefill_tokens,
            "prefill_s": round(st.prefill_time, 4),
            "decode_steps": st.decode_steps,
            "decode_step_ms": round(1e3 * st.decode_time /
                                    max(st.decode_steps, 1), 3),
            "prefix_hits": st.prefix_hits, "prefix_total": st.prefix_total,
            "preemptions": st.preemptions,
            "ttft_mean_ms": round(1e3 * float(np.mean(st.ttft)), 2)},
    }
    print(json.dumps(res), flush=True)


def run_gather(args, torch, W):
    """The reference's attention read path, materialised: every sequence's
    K and V gathered through its block table into rvllm's padded
    [batch, n_kv, ctx_len, hd] (f32 as kv_gather.cu writes it, or f16 raw
    bits), one rvkv_gather per layer over the decode workload of --config.
    Algorithmic bytes: the cache rows read (f16) + the padded outputs
    written + the tables."""
    from rvllm_amd.kv_storage import HipGatherPlan, HipKvStorage
    db = build_workload(W, args.config, args.batch, args.ctx)
    c = db.cfg
    st = HipKvStorage(c.n_layers, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim)
    fill_pool(torch, st, c.seed, c.value_scale)
    plan = HipGatherPlan([(db.tables[b], int(db.ctx_lens[b]))
                          for b in range(db.batch)])
    dt_out = torch.float32 if args.gather == "f32" else torch.float16
    n_out = db.batch * c.n_kv_heads * plan.ctx_len * c.head_dim
    ok = torch.empty(n_out, dtype=dt_out, device="cuda")
    ov = torch.empty(n_out, dtype=dt_out, device="cuda")

    def step():
        for layer in range(c.n_layers):
            st.gather(layer, plan, ok, ov)

    dt, launch_ms = _time_launches(torch, step, c.n_layers, args.steps,
                                   args.warmup)
    # Rows read: each sequence's own tokens (padding positions re-read its
    # last block, already counted); rows written: the whole padded output.
    read = int(db.ctx_lens.sum()) * c.n_kv_heads * c.head_dim * 2 * 2
    per_launch = (read + 2 * n_out * ok.element_size() +
                  4 * db.batch * plan.max_blocks)
    res = _hbm_line(
        "block-table gather HBM GB/s, 1 MI355X", per_launch * c.n_layers, dt,
        launch_ms, per_launch, f"gather_kernel (out {args.gather})", args,
        {"workload": f"{c.name}: gather of {db.batch} seqs, padded ctx "
                     f"{plan.ctx_len}, {c.n_kv_heads} kv heads, head_dim "
                     f"{c.head_dim}, block_size {c.block_size}, "
                     f"{c.n_layers} layers",
         "global_batch": db.batch, "seq_len": plan.ctx_len,
         "parallelism": "single GPU"},
        f"f16 cache -> {args.gather}")
    st.close()
    del ok, ov
    torch.cuda.empty_cache()
    with_copy_ceiling(torch, res, read / per_launch, max(args.steps // 4, 3))
    print(json.dumps(res), flush=True)


def run_cow(args, torch, W):
    """Copy-on-write block copies: the prefix sharers' (shared -> private)
    pairs of the --config workload (Qwen2.5 by default: sharers whose last
    block is a partial shared one), or --cow-blocks random distinct pairs;
    one rvkv_copy_blocks covers every layer, K and V. Algorithmic bytes:
    each copied block read and written, all layers, K and V."""
    from rvllm_amd.kv_storage import HipKvStorage
    name = args.config
    db = build_workload(W, name, args.batch, args.ctx)
    c = db.cfg
    st = HipKvStorage(c.n_layers, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim)
    if args.cow_blocks:
        rng = np.random.default_rng(c.seed + 11)
        pick = rng.permutation(db.num_blocks)[:2 * args.cow_blocks]
        src, dst = pick[:args.cow_blocks], pick[args.cow_blocks:]
    else:
        src, dst = db.cow_src, db.cow_dst
    if len(src) == 0:
        raise SystemExit(f"{name} has no copy-on-write pairs; use "
                         "--cow-blocks N")

    def u32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32)
                                .view(np.int32).copy()).cuda()

    s_t, d_t = u32(src), u32(dst)
    dt, launch_ms = _time_launches(
        torch, lambda: st.copy_blocks(s_t, d_t), 1, args.steps, args.warmup)
    block_bytes = c.block_size * c.n_kv_heads * c.head_dim * 2
    per_launch = len(src) * block_bytes * 2 * c.n_layers * 2 + 8 * len(src)
    res = _hbm_line(
        "copy-on-write block copy HBM GB/s, 1 MI355X", per_launch, dt,
        launch_ms, per_launch, "copy_blocks_kernel", args,
        {"workload": f"{c.name}: {len(src)} block pairs x {c.n_layers} "
                     f"layers x K/V, block {block_bytes} B",
         "global_batch": len(src), "seq_len": c.block_size,
         "parallelism": "single GPU"},
        "f16 (bit copy)")
    st.close()
    torch.cuda.empty_cache()
    with_copy_ceiling(torch, res, 0.5, max(args.steps // 4, 3))
    print(json.dumps(res), flush=True)


def run_prep(args, torch, W):
    """Fused attention prep over a prefill batch: per token, q/k/v rows
    (f32, as the QKV projection leaves them) get the bias, the per-head
    RMS norm (q and k) and RoPE, q is written back in f32 and k/v are
    appended into the f16 cache at the token's slot; one rvkv_attn_prep per
    layer. Bias and norm weights are used when the model has them
    (Qwen2.5: bias, Qwen3: QK norm)."""
    from rvllm_amd.kv_storage import HipKvStorage
    from rvllm_amd.rope import rope_cos_sin
    db = build_workload(W, args.config, args.batch, args.ctx)
    c = db.cfg
    st = HipKvStorage(c.n_layers, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim)
    sb, so, pos = prompt_slots(torch, db)
    n_tok = sb.numel()
    H, KV, hd = c.n_heads, c.n_kv_heads, c.head_dim
    g = torch.Generator(device="cuda")
    g.manual_seed(c.seed)
    rnd = lambda *shape: torch.randn(shape, generator=g, device="cuda")
    q, k, v = rnd(n_tok, H, hd), rnd(n_tok, KV, hd), rnd(n_tok, KV, hd)
    q_out = torch.empty_like(q)
    cs, sn = rope_cos_sin(c.rope_theta, hd, pos)
    cs, sn = torch.from_numpy(cs).cuda(), torch.from_numpy(sn).cuda()
    opt = {}
    if c.qkv_bias:
        opt.update(q_bias=rnd(H * hd), k_bias=rnd(KV * hd),
                   v_bias=rnd(KV * hd))
    if c.qk_norm:
        opt.update(q_norm=rnd(hd), k_norm=rnd(hd))

    def step():
        for layer in range(c.n_layers):
            st.attn_prep(layer, q, k, v, cs, sn, sb, so, eps=1e-6,
                         q_out=q_out, **opt)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    launch_ms = e0.elapsed_time(e1) / (args.steps * c.n_layers)
    per_launch = W.prep_bytes(n_tok, c)
    achieved = per_launch / (launch_ms * 1e-3) / 1e9
    res = {
        "metric": "attention prep + append HBM GB/s, 1 MI355X",
        "value": round(per_launch * c.n_layers / dt / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 q/k/v -> f32 q, f16 cache",
        "data": "synthetic N(0,1) rows and weights, seeded permuted tables",
        "config": {
            "workload": f"{c.name} attn prep: {n_tok} tokens "
                        f"({db.batch} seqs x {int(db.ctx_lens.max())}) x "
                        f"{c.n_layers} layers, {H} q / {KV} kv heads, "
                        f"head_dim {hd}, bias {c.qkv_bias}, "
                        f"qk_norm {c.qk_norm}",
            "global_batch": db.batch,
            "seq_len": int(db.ctx_lens.max()),
            "parallelism": "single GPU",
        },
        "tok_per_s": round(n_tok / dt, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": f"attn_prep_kernel<{hd}>",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": per_launch,
            "avg_launch_ms": round(launch_ms, 5),
        },
    }
    st.close()
    del q, k, v, q_out
    torch.cuda.empty_cache()
    rd = 4 * H * hd + 8 * KV * hd  # q, k, v in (per token)
    wr = 4 * H * hd + 4 * KV * hd  # q out, k/v cells
    with_copy_ceiling(torch, res, rd / (rd + wr), max(args.steps // 4, 3))
    print(json.dumps(res), flush=True)


def run_prefill(args, torch, W, st=None):
    """Scatter-only prefill append: every sequence's ctx tokens (K and V
    rows [tokens, n_kv, hd] of the source dtype) appended into its
    block-table slots, one rvkv_append per layer (the slot lists are built
    once, like the engine's write_positions). The source rows are one
    device buffer reused by every layer (each layer's write goes to its own
    pool, and the source is far larger than the 256 MB MALL). st: an
    existing pool of this workload's shape to write into (kept open)."""
    from rvllm_amd.kv_storage import HipKvStorage
    db = build_workload(W, args.config, args.batch, args.ctx)
    c = db.cfg
    own = st is None
    if own:
        st = HipKvStorage(c.n_layers, db.num_blocks, c.block_size,
                          c.n_kv_heads, c.head_dim)
    bs = c.block_size
    sb, so, _ = prompt_slots(torch, db)
    n_tok = sb.numel()
    dt_src = torch.float32 if args.prefill == "f32" else torch.float16
    g = torch.Generator(device="cuda")
    g.manual_seed(c.seed)
    k = (torch.randn((n_tok, c.n_kv_heads, c.head_dim), generator=g,
                     device="cuda") * c.value_scale).to(dt_src)
    v = (torch.randn((n_tok, c.n_kv_heads, c.head_dim), generator=g,
                     device="cuda") * c.value_scale).to(dt_src)

    def step():
        for layer in range(c.n_layers):
            st.write_tokens(layer, sb, so, k, v)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    launch_ms = e0.elapsed_time(e1) / (args.steps * c.n_layers)
    src_bytes = 4 if args.prefill == "f32" else 2
    per_launch = W.append_bytes(n_tok, c, src_bytes)
    achieved = per_launch / (launch_ms * 1e-3) / 1e9
    res = {
        "metric": "prefill append (scatter) HBM GB/s, 1 MI355X",
        "value": round(per_launch * c.n_layers / dt / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{args.prefill} source -> f16 cache",
        "data": "synthetic N(0,1)*scale rows, seeded permuted block tables",
        "config": {
            "workload": f"{c.name} prefill append: {n_tok} tokens "
                        f"({db.batch} seqs x {int(db.ctx_lens.max())}) x "
                        f"{c.n_layers} layers, {c.n_kv_heads} kv heads, "
                        f"head_dim {c.head_dim}, block_size {bs}",
            "global_batch": db.batch,
            "seq_len": int(db.ctx_lens.max()),
            "parallelism": "single GPU",
        },
        "tok_per_s": round(n_tok / dt, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": f"append_kernel<8, {args.prefill == 'f32'}>",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": per_launch,
            "avg_launch_ms": round(launch_ms, 5),
        },
    }
    if own:
        st.close()
    del k, v, sb, so
    torch.cuda.empty_cache()
    return with_copy_ceiling(torch, res, src_bytes / (src_bytes + 2),
                             max(args.steps // 2, 3))


def run_churn(args, torch, W):
    """The churn workload: gemma-3-270m shape, 1024 sequences starting at
    1024 tokens; every engine step 10% finish and 10% are admitted with
    64-token prompts (prefill append), then all decode one token (fused
    append + decode per layer under a per-step decode plan). The pool is
    1.25x the initial live blocks, with a seeded-shuffled free list."""
    from rvllm_amd.engine_sim import ChurnDriver
    c = W.CONFIGS[args.config]
    batch = args.batch or c.batch
    drv = ChurnDriver(c, batch, 1024, prompt_len=64, churn=0.10,
                      steps=args.warmup + args.steps + 1)
    # A serving loop's host: the objects made at start-up leave the garbage
    # collector's view, so a full collection during the run does not stall
    # the step it lands in (one such pause measured 36 ms).
    import gc
    gc.collect()
    gc.freeze()
    for _ in range(args.warmup):
        drv.step()
    evs = [torch.cuda.Event(enable_timing=True)
           for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    b0 = drv.bytes_moved
    step_bytes_each = []
    t0 = time.perf_counter()
    evs[0].record()
    for i in range(args.steps):
        b_before = drv.bytes_moved
        drv.step()
        step_bytes_each.append(drv.bytes_moved - b_before)
        evs[i + 1].record()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    step_ms = [evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)]
    step_median_ms = float(np.median(step_ms))
    # The run in five phases of consecutive steps: GPU time (step events)
    # and bytes, so the long-context start and the short-context end show.
    phases = []
    for idx in np.array_split(np.arange(args.steps), 5):
        if len(idx) == 0:
            continue
        ms = float(np.sum([step_ms[i] for i in idx]))
        by = float(np.sum([step_bytes_each[i] for i in idx]))
        phases.append({"steps": f"{int(idx[0])}-{int(idx[-1])}",
                       "ms_per_step": round(ms / len(idx), 4),
                       "GB_per_step": round(by / len(idx) / 1e9, 4),
                       "GB/s": round(by / (ms * 1e-3) / 1e9, 1)})
    step_bytes = (drv.bytes_moved - b0) / args.steps
    # Per-launch decode time at the final state (back-to-back over layers).
    st, plan = drv.st, drv.plan
    from rvllm_amd.engine_sim import NSTAGE
    db = drv.devb[(drv.step_index - 1) % NSTAGE]
    lens = drv.last[1]
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    reps = max(args.steps // 10, 3)
    e0.record()
    for _ in range(reps):
        for layer in range(c.n_layers):
            st.decode_step(layer, drv.nk[layer], drv.nv[layer], db["sb"],
                           db["so"], drv.q[layer], db["tables"], db["ctx"],
                           plan=plan, out=drv.out[layer])
    e1.record()
    torch.cuda.synchronize()
    dec_ms = e0.elapsed_time(e1) / (reps * c.n_layers)
    dec_bytes = drv.decode_bytes(lens) + W.append_bytes(batch, c)
    achieved = dec_bytes / (dec_ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": round(step_bytes / dt / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "ms_per_step_median": round(step_median_ms, 4),
        "phases": phases,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 KV, f32 accumulate",
        "data": "synthetic: K/V/q ~ N(0,1), seeded churn and free list",
        "config": {
            "workload": f"{c.name} churn: {c.n_layers} layers, {c.n_heads} q / "
                        f"{c.n_kv_heads} kv heads, head_dim {c.head_dim}, "
                        f"block_size {c.block_size}, {batch} seqs from 1024 "
                        f"tokens, 10% finish/admit (64-token prompts) per "
                        f"step, pool {drv.num_blocks} blocks (1.25x live, "
                        f"shuffled free list)",
            "global_batch": batch,
            "seq_len": int(lens.max()),
            "parallelism": "single GPU",
            "decode_plan_items": plan.items,
        },
        "pct_of_peak": round(100 * step_bytes / dt / 1e9 / HBM_PEAK_GBS, 2),
        "tok_per_s": round(batch / dt, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_part_kernel (fused append, decode plan) at the "
                      "final step's lengths",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": dec_bytes,
            "avg_launch_ms": round(dec_ms, 5),
        },
    }
    rc = read_ceiling(torch, dec_bytes, max(args.steps // 10, 3))
    rc["frac"] = round(achieved / rc["GB/s"], 4)
    res["roofline"]["stream_read_ceiling"] = rc
    pc = paged_ceiling(torch, drv.decode_bytes(lens),
                       c.block_size * c.head_dim * 2, max(args.steps // 10, 3))
    pc["frac"] = round(achieved / pc["GB/s"], 4)
    res["roofline"]["paged_read_ceiling"] = pc
    drv.close()
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); the "
              "paged KV path shards by sequence or KV head with no exchange "
              "inside it, so run one process per GPU.", file=sys.stderr)
        sys.exit(2)
    import torch

    from rvllm_amd import workloads as W
    from rvllm_amd.kv_storage import HipKvStorage

    torch.cuda.set_device(0)
    if args.copy_calibration:
        copy_calibration(torch, max(args.steps, 5))
        return
    if args.traffic_pass:
        traffic_pass(args, torch, W)
        return
    if args.churn:
        print(json.dumps(run_churn(args, torch, W)), flush=True)
        return
    if args.prefill:
        print(json.dumps(run_prefill(args, torch, W)), flush=True)
        return
    if args.prep:
        run_prep(args, torch, W)
        return
    if args.prefill_attn:
        run_prefill_attn(args, torch, W)
        return
    if args.gather:
        run_gather(args, torch, W)
        return
    if args.engine:
        run_engine(args, torch, W)
        return
    if args.cow:
        run_cow(args, torch, W)
        return
    secondary = (args.secondary and args.config == "qwen3-0.6b"
                 and not args.batch and not args.ctx and not args.f32_cache
                 and not args.unfused and not args.graph and args.plan is None)
    res = run_decode(args, torch, W, cpu=not args.no_cpu, keep_pool=secondary)
    if secondary:
        # configs[2]'s prefill append into the headline's own pool (the
        # same Qwen3 shape): a second 112 GiB pool is never made.
        st = res.pop("_pool")
        pre = run_prefill(argparse.Namespace(**{
            **vars(args), "config": "qwen3-0.6b", "batch": 0, "ctx": 0,
            "prefill": "f32", "steps": max(args.steps // 2, 5),
            "warmup": min(args.warmup, 2)}), torch, W, st=st)
        st.close()
        torch.cuda.empty_cache()
        pre = _secondary(pre, "configs[2] prefill append (scatter only, f32 "
                              "source rows), into the headline's pool")
        pre["command"] = ("python3 bench.py (after the headline, same "
                          "process); alone: python3 bench.py --prefill f32")
        res["secondary"] = secondary_records(args, torch, W) + [pre]
        if args.traffic:
            live = live_traffic(args)
            if live is not None:
                res["roofline"]["traffic"] = live.pop("traffic")
                res["roofline"]["traffic_source"] = live
    print(json.dumps(res), flush=True)


def _secondary(res, role):
    """The part of a workload's record a secondary entry keeps."""
    keep = ("metric", "value", "unit", "steps", "warmup", "ms_per_step",
            "ms_per_step_median", "phases", "dtype", "config", "pct_of_peak",
            "tok_per_s", "roofline")
    out = {"role": role}
    out.update({k: res[k] for k in keep if k in res})
    return out


PAUSE_AFTER_FREE_S = 15.0


def _child_record(args, extra):
    """Runs bench.py with `extra` arguments in a child process (a fresh
    process, as a separate bench invocation would be) and returns its JSON
    record. The parent has freed its own pools before this."""
    import subprocess
    cmd = [sys.executable, os.path.abspath(__file__), "--no-cpu"] + extra
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if p.returncode != 0:
        raise SystemExit(f"secondary run {' '.join(extra)} failed "
                         f"({p.returncode}): {p.stderr[-2000:]}")
    return json.loads(p.stdout.strip().splitlines()[-1])


def secondary_records(args, torch, W):
    """The rest of the north star's target workloads, run within the same
    bench invocation as the headline (as rvllm's bench sweeps its workloads
    in one run), each in a child process of its own: configs[4]'s 200-step
    churn and the Llama-3.2-1B shape at 256 x 4096. (configs[2]'s prefill
    append runs in this process, on the headline's pool.)"""
    jobs = [
        (["--churn", "--steps", "200", "--warmup", "3"],
         "configs[4] churn, 200 engine steps"),
        (["--config", "llama-3.2-1b", "--batch", "256", "--ctx", "4096",
          "--steps", str(args.steps), "--warmup", str(args.warmup)],
         "north-star shape 2: Llama-3.2-1B, 256 seqs x 4096 tokens, fused "
         "decode step"),
    ]
    out = []
    for extra, role in jobs:
        # A workload started within ~10 s of a large pool's release ran
        # 10-20 % slower (the churn: 0.84 vs 0.72 ms per step right after
        # the 112 GiB pool was freed, 0.72 after 10, 25 or 45 s); each run
        # starts after a pause.
        time.sleep(PAUSE_AFTER_FREE_S)
        rec = _child_record(args, extra)
        rec = _secondary(rec, role)
        rec["command"] = "python3 bench.py --no-cpu " + " ".join(extra)
        if args.traffic and "--batch" in extra:
            live = live_traffic(args, extra[:6])
            if live is not None:
                rec["roofline"]["traffic"] = live.pop("traffic")
                rec["roofline"]["traffic_source"] = live
        out.append(rec)
    return out


def traffic_pass(args, torch, W):
    """What the counter passes of live_traffic profile: two launches of the
    calibration library's copy probe, each reading 2 GiB and writing 2 GiB
    (the counters' scale), then the headline decode for a few steps (no
    ceilings, no CPU leg)."""
    import ctypes

    from rvllm_amd import _lib
    lib = _lib.load_calib()
    n = 2 << 30
    a = torch.zeros(n // 4, dtype=torch.int32, device="cuda")
    b = torch.empty_like(a)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for _ in range(2):
        _lib.check_calib(lib.rvkv_calib_copy_probe(
            ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
            n, n, 16384, stream))
    torch.cuda.synchronize()
    del a, b
    torch.cuda.empty_cache()
    run_decode(argparse.Namespace(**{**vars(args), "steps": 2, "warmup": 1}),
               torch, W, cpu=False)


def live_traffic(args, extra=None):
    """HBM bytes per headline decode launch, measured in this run: two child
    processes run the traffic pass under rocprofv3 --pmc, one with
    FETCH_SIZE and one with WRITE_SIZE (KiB per dispatch); each is scaled by
    what the same counter reads for a copy probe launch that reads 2 GiB
    and writes 2 GiB, in the same pass. Returns
    {traffic, ...details} or None (the profiler missing or failing; the
    record then keeps the committed profile's figure)."""
    import csv
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return None
    per = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        time.sleep(PAUSE_AFTER_FREE_S)
        d = tempfile.mkdtemp(prefix="rvkv_pmc_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "--kernel-include-regex",
               "decode_part_kernel|prefill_kernel|decode_reduce_kernel|"
               "copy_probe_kernel",
               "-f", "csv", "-d", d, "-o", "run", "--", sys.executable,
               os.path.abspath(__file__), "--traffic-pass", "--no-cpu"] + (
                   extra if extra is not None else ["--config", args.config])
        # (its own process group, so a pass that overruns is ended with
        # the bench child it started)
        p = subprocess.Popen(cmd, stdout=subprocess.DEVNULL,
                             stderr=subprocess.DEVNULL, cwd="/tmp",
                             env={**os.environ, "TMPDIR": "/tmp"},
                             start_new_session=True)
        try:
            p.wait(timeout=150)
        except subprocess.TimeoutExpired:
            os.killpg(p.pid, 9)
            p.wait()
            shutil.rmtree(d, ignore_errors=True)
            return None
        rows = []
        for root, _, files in os.walk(d):
            for fn in files:
                if fn.endswith("counter_collection.csv"):
                    with open(os.path.join(root, fn)) as f:
                        rows += list(csv.DictReader(f))
        shutil.rmtree(d, ignore_errors=True)
        if p.returncode != 0 or not rows:
            return None
        vals = {"copy": [], "part": [], "reduce": []}
        for r in rows:
            if r.get("Counter_Name") != counter:
                continue
            k = r.get("Kernel_Name", "")
            key = ("copy" if "copy_probe_kernel" in k else
                   "reduce" if "decode_reduce" in k else
                   "part" if ("decode_part" in k or "prefill_kernel" in k)
                   else None)
            if key:
                vals[key].append(float(r["Counter_Value"]))
        if not vals["copy"] or not vals["part"]:
            return None
        copy_kib = sum(vals["copy"]) / len(vals["copy"])
        launch_kib = (sum(vals["part"]) + sum(vals["reduce"])) / len(
            vals["part"])
        scale = (2 << 30) / (copy_kib * 1024)
        per[counter] = {"kib_per_launch": round(launch_kib, 1),
                        "copy_kib": round(copy_kib, 1),
                        "scale": round(scale, 6),
                        "dispatches": len(vals["part"])}
    traffic = sum(v["kib_per_launch"] * 1024 * v["scale"]
                  for v in per.values())
    return {"traffic": int(round(traffic)),
            "how": "rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, on "
                   "python3 bench.py --traffic-pass (child processes of "
                   "this run, after the timed runs); KiB per decode launch "
                   "x (2 GiB / the same counter's KiB for one copy-probe "
                   "launch reading and writing 2 GiB)",
           **{c.lower(): v for c, v in per.items()}}


def run_decode(args, torch, W, cpu, keep_pool=False):
    """The decode step of --config (append + paged decode per layer, fused
    by default) timed over --steps; returns the record (keep_pool: the pool
    is left open, in record["_pool"])."""
    from rvllm_amd.kv_storage import HipKvStorage
    db = build_workload(W, args.config, args.batch, args.ctx)
    c = db.cfg
    f32 = (args.f32_cache if args.f32_cache is not None
           else c.name == "smollm2-360m")
    cell = 4 if f32 else 2
    st = HipKvStorage(c.n_layers, db.num_blocks, c.block_size, c.n_kv_heads,
                      c.head_dim,
                      dtype=torch.float32 if f32 else torch.float16)
    fill_pool(torch, st, c.seed, c.value_scale)

    def u32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32)
                                .view(np.int32).copy()).cuda()

    if len(db.cow_src):  # prefix sharers move onto private copies first
        st.copy_blocks(u32(db.cow_src), u32(db.cow_dst))
    tables = u32(db.padded_tables())
    ctx = u32(db.ctx_lens)
    sb, so = u32(db.slot_block), u32(db.slot_off)
    max_ctx = int(db.ctx_lens.max())
    g = torch.Generator(device="cuda")
    g.manual_seed(c.seed + 7)
    L, B = c.n_layers, db.batch
    q = [torch.randn((B, c.n_heads, c.head_dim), generator=g, device="cuda")
         for _ in range(L)]
    nk = [torch.randn((B, c.n_kv_heads, c.head_dim), generator=g,
                      device="cuda") for _ in range(L)]
    nv = [torch.randn((B, c.n_kv_heads, c.head_dim), generator=g,
                      device="cuda") for _ in range(L)]
    out = [torch.empty_like(q[0]) for _ in range(L)]
    ws = st.alloc_workspace(B, c.n_heads, max_ctx)
    part = st.decode_partition_tokens(B, c.n_heads, max_ctx)
    # Ragged batches use the per-forward decode plan, rebuilt every step from
    # the host-side context lengths (as the engine's GatherPlan is).
    plan = None
    if args.plan or (args.plan is None and
                     int(db.ctx_lens.min()) != int(db.ctx_lens.max())):
        from rvllm_amd.kv_storage import HipDecodePlan
        plan = HipDecodePlan(st, db.ctx_lens, c.n_heads)
        if args.graph:
            raise SystemExit("--graph cannot capture the per-step plan "
                             "rebuild; use --no-plan with --graph")

    # The library's choice for groups of four and more at head_dim 64 on an
    # f16 pool, with or without a plan: the matrix-core decode.
    mfma = (not f32 and c.head_dim == 64 and
            c.n_heads // c.n_kv_heads >= 4 and
            os.environ.get("RVKV_DECODE_MFMA", "") != "0")
    if mfma:
        decode_kernels = ("prefill_kernel<64, 1> in decode mode (matrix "
                          "cores" + ("" if args.unfused else
                                     ", fused append (rvkv_decode_step)")
                          + ") + decode_reduce_kernel for split sequences"
                          " or partitions")
    else:
        decode_kernels = ("decode_part_kernel (+ decode_reduce_kernel for "
                          "split sequences)" + ("" if args.unfused else
                                                ", fused append "
                                                "(rvkv_decode_step)"))

    def decode(layer):
        if args.unfused:
            if plan is not None:
                st.paged_decode_planned(layer, plan, q[layer], tables, ctx,
                                        out=out[layer])
            else:
                st.paged_decode(layer, q[layer], tables, ctx, max_ctx,
                                out=out[layer], ws=ws)
        else:  # append + decode in one launch
            st.decode_step(layer, nk[layer], nv[layer], sb, so, q[layer],
                           tables, ctx, max_ctx, plan=plan, out=out[layer],
                           ws=ws)

    host_tables = db.padded_tables()

    def step():
        if plan is not None:
            plan.update(db.ctx_lens, host_tables)
        for layer in range(L):
            if args.unfused:
                st.write_tokens(layer, sb, so, nk[layer], nv[layer])
            decode(layer)

    run = step
    if args.graph:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            st.set_stream(side)
            step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            st.set_stream(torch.cuda.current_stream())
            step()
        st.set_stream(torch.cuda.current_stream())
        run = graph.replay

    for _ in range(args.warmup):
        run()
    # Step events (recording does not synchronise) give the median step.
    evs = [torch.cuda.Event(enable_timing=True)
           for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    evs[0].record()
    for i in range(args.steps):
        run()
        evs[i + 1].record()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    step_median_ms = float(np.median([evs[i].elapsed_time(evs[i + 1])
                                      for i in range(args.steps)]))

    # Per-launch decode duration: HIP events on the pool's stream (torch's
    # current stream) around `steps` rounds of back-to-back decode launches
    # over all layers (each launch reads a different layer's pool, so no
    # launch finds the previous one's data in the 256 MB MALL).
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        for layer in range(L):
            decode(layer)
    e1.record()
    torch.cuda.synchronize()
    dec_ms = e0.elapsed_time(e1) / (args.steps * L)

    traffic = None if f32 else measured_traffic(args.config, args.batch,
                                                args.unfused, args.ctx)
    app_bytes = W.append_bytes(B, c, cell_bytes=cell)
    # The fused launch also moves the appended rows (f32 in, f16 out; an f32
    # pool runs the append and the decode as two launches, timed together).
    dec_bytes = W.decode_bytes(db, cell) + (0 if args.unfused else app_bytes)
    step_bytes = L * (W.decode_bytes(db, cell) + app_bytes)
    achieved = dec_bytes / (dec_ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": round(step_bytes / dt / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "ms_per_step_median": round(step_median_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 KV, f32 math" if f32 else "f16 KV, f32 accumulate",
        "data": "synthetic: K/V ~ N(0,1)*scale (f16 values), q ~ N(0,1) "
                "f32, seeded random-permutation block tables",
        "config": {
            "workload": f"{c.name}: {c.description.split(',')[0]}"
                        f"{'' if not (args.batch or args.ctx) else ' (resized)'}; "
                        f"{L} layers, "
                        f"{c.n_heads} q / {c.n_kv_heads} kv heads, head_dim "
                        f"{c.head_dim}, block_size {c.block_size}, "
                        f"{B} seqs, max ctx {max_ctx}",
            "global_batch": B,
            "seq_len": max_ctx,
            "parallelism": "single GPU",
            "launch": "hip graph" if args.graph else "eager",
            "partition_tokens": None if plan is not None else part,
            "decode_plan_items": plan.items if plan is not None else None,
        },
        "pct_of_peak": round(100 * step_bytes / dt / 1e9 / HBM_PEAK_GBS, 2),
        "tok_per_s": round(B / dt, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": decode_kernels,
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": dec_bytes,
            "avg_launch_ms": round(dec_ms, 5),
        },
    }
    # Context for frac: the best plain read of the same bytes per launch,
    # contiguous and as randomly placed cache tiles.
    if getattr(args, "traffic_pass", False):
        return res
    rc = read_ceiling(torch, dec_bytes, max(args.steps, 3))
    rc["frac"] = round(achieved / rc["GB/s"], 4)
    res["roofline"]["stream_read_ceiling"] = rc
    tile = c.block_size * c.head_dim * cell
    if tile % 1024 == 0:
        pc = paged_ceiling(torch, W.decode_bytes(db, cell), tile,
                           max(args.steps // 2, 3))
        pc["frac"] = round(achieved / pc["GB/s"], 4)
        res["roofline"]["paged_read_ceiling"] = pc
    if cpu:
        from oracle import oracle as orc
        res["cpu_baseline"] = cpu_baseline(orc, W, st, db, args.cpu_seconds,
                                             f32=f32)
    if plan is not None:
        plan.close()
    if keep_pool:
        res["_pool"] = st
    else:
        st.close()
    return res


if __name__ == "__main__":
    main()
