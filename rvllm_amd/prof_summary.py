"""Summaries of rocprofv3 CSV output for the paged-KV kernels.

    python -m rvllm_amd.prof_summary stats <kernel_stats.csv> [--cmd "..."]
    python -m rvllm_amd.prof_summary traffic --fetch <counter_collection.csv>
        --write <counter_collection.csv> --copy-fetch <...> --copy-write <...>
        --copy-bytes N --kernel "decode_part_kernel[|other|...]"
        [--launch-bytes N]

`stats` prints a markdown table of per-kernel calls / average / total time.
`traffic` prints the mean FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of
the named kernel, scales each by (known bytes / counter bytes) of a plain
device copy, and reports HBM bytes per launch as JSON.
"""
from __future__ import annotations

import argparse
import csv
import json
import sys
from collections import defaultdict


def kernel_stats(path):
    rows = list(csv.DictReader(open(path)))
    out = []
    for r in rows:
        out.append((r["Name"], int(r["Calls"]), float(r["AverageNs"]),
                    float(r["TotalDurationNs"]), float(r["Percentage"]),
                    float(r["MinNs"]), float(r["MaxNs"])))
    return out


def counter_means(path, counter):
    agg = defaultdict(list)
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] == counter:
            agg[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in agg.items()}


def _pick(means, needle):
    hits = {k: v for k, v in means.items() if needle in k}
    if not hits:
        raise SystemExit(f"no kernel matching {needle!r}")
    return max(hits.items(), key=lambda kv: kv[1])


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="mode", required=True)
    a = sub.add_parser("stats")
    a.add_argument("csv")
    a.add_argument("--cmd", default="")
    a.add_argument("--top", type=int, default=8)
    b = sub.add_parser("traffic")
    for k in ("fetch", "write", "copy_fetch", "copy_write"):
        b.add_argument("--" + k.replace("_", "-"), required=True)
    b.add_argument("--copy-bytes", type=float, required=True)
    b.add_argument("--kernel", default="decode_part_kernel")
    b.add_argument("--copy-kernel", default="copyBuffer")
    b.add_argument("--launch-bytes", type=float, default=0.0)
    args = ap.parse_args(argv)
    if args.mode == "stats":
        if args.cmd:
            print(f"Command: `{args.cmd}`\n")
        print("| kernel | calls | avg us | total ms | % | min us | max us |")
        print("|---|---|---|---|---|---|---|")
        for n, c, avg, tot, pct, mn, mx in kernel_stats(args.csv)[:args.top]:
            n = n if len(n) < 90 else n[:87] + "..."
            print(f"| `{n}` | {c} | {avg / 1e3:.2f} | {tot / 1e6:.3f} | "
                  f"{pct:.1f} | {mn / 1e3:.2f} | {mx / 1e3:.2f} |")
        return
    # --kernel may list several kernels ("|"-separated: kernel names hold
    # commas) that together make one launch of the measured call; their
    # per-dispatch means add.
    fm = counter_means(args.fetch, "FETCH_SIZE")
    wm = counter_means(args.write, "WRITE_SIZE")
    names, fetch, write = [], 0.0, 0.0
    for needle in args.kernel.split("|"):
        kf, f = _pick(fm, needle)
        _, w = _pick(wm, needle)
        names.append(kf)
        fetch += f
        write += w
    kf = " + ".join(names)
    _, cfetch = _pick(counter_means(args.copy_fetch, "FETCH_SIZE"),
                      args.copy_kernel)
    _, cwrite = _pick(counter_means(args.copy_write, "WRITE_SIZE"),
                      args.copy_kernel)
    half = args.copy_bytes / 2  # a copy reads and writes half the bytes each
    f_scale = half / (cfetch * 1024)
    w_scale = half / (cwrite * 1024)
    traffic = fetch * 1024 * f_scale + write * 1024 * w_scale
    rec = {"kernel": kf, "fetch_kib": fetch, "write_kib": write,
           "copy_fetch_kib": cfetch, "copy_write_kib": cwrite,
           "fetch_scale": f_scale, "write_scale": w_scale,
           "traffic_bytes_per_launch": round(traffic)}
    if args.launch_bytes:
        rec["algorithmic_bytes_per_launch"] = args.launch_bytes
        rec["traffic_over_algorithmic"] = traffic / args.launch_bytes
    json.dump(rec, sys.stdout, indent=1)
    print()


if __name__ == "__main__":
    main()
