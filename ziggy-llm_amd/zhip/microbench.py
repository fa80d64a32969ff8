"""Standalone dequant-matvec microbenchmark (batch 1).

Formats Q4_K, Q6_K and Q8_0; shapes (rows x cols) 4096x4096, 14336x4096,
4096x14336 and 128256x4096; weights N(0, 0.02) quantized by this package,
x ~ N(0, 1).  One matrix is quantized on the host, uploaded, and replicated
on the device into at least 1 GiB of distinct copies; launches rotate over
the copies so every launch streams its weights from HBM rather than the
256 MB Infinity Cache.  Each launch is timed with its own HIP events.
GB/s counts the weight bytes plus x and y (rows*cols*bytes_per_weight +
4*(rows+cols)).

Usage: python -m zhip.microbench [--iters N] [--formats q4_k,q6_k,q8_0]
                                 [--shapes 4096x4096,14336x4096] [--out FILE.md]
Prints one JSON object per case; --out also writes them as a markdown table.
"""
from __future__ import annotations

import argparse
import json
import math

import numpy as np

from . import hip, synth
from .gguf import Q4_K, Q6_K, Q8_0, row_bytes

SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]
FORMATS = {"q4_k": Q4_K, "q6_k": Q6_K, "q8_0": Q8_0}
HBM_PEAK_GBS = 8000.0


def run(ctx: hip.Context, ttype: int, rows: int, cols: int, iters: int, min_bytes: int = 1 << 30) -> dict:
    rb = row_bytes(ttype, cols)
    mbytes = rb * rows
    stride = (mbytes + 4095) // 4096 * 4096
    copies = max(2, math.ceil(min_bytes / stride))
    q = np.zeros(mbytes, np.uint8)
    synth.fill_tensor(q, ttype, rows, cols, seed=rows * 31 + cols)
    src = ctx.buffer(q)
    mats = ctx.empty(stride * copies)
    for c in range(copies):
        ctx.copy(src, 0, mats, c * stride, mbytes)
    src.free()
    x = ctx.buffer(synth.normal_row(5, 0, cols, 0.0, 1.0))
    y = ctx.empty(rows * 4)
    ctx.time_matvec(ttype, mats, copies, stride, x, y, rows, cols, min(copies, 8))  # warm-up
    ns = ctx.time_matvec(ttype, mats, copies, stride, x, y, rows, cols, max(iters, copies))
    nbytes = mbytes + 4 * (rows + cols)
    mats.free()
    gbs = nbytes / ns
    return {"format": {Q4_K: "q4_k", Q6_K: "q6_k", Q8_0: "q8_0"}[ttype], "rows": rows, "cols": cols,
            "copies": copies, "bytes": nbytes, "avg_us": round(ns / 1e3, 3), "gbs": round(gbs, 1),
            "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--formats", default="q4_k,q6_k,q8_0")
    ap.add_argument("--shapes", default=",".join(f"{r}x{c}" for r, c in SHAPES),
                    help="comma-separated ROWSxCOLS list")
    ap.add_argument("--out", help="also write the results as a markdown table")
    args = ap.parse_args()
    shapes = [tuple(int(v) for v in s.split("x")) for s in args.shapes.split(",")]
    ctx = hip.Context(0)
    results = []
    for f in args.formats.split(","):
        for rows, cols in shapes:
            r = run(ctx, FORMATS[f], rows, cols, args.iters)
            results.append(r)
            print(json.dumps(r), flush=True)
    ctx.close()
    if args.out:
        lines = ["# Dequant-matvec microbenchmark (batch 1), one MI355X", "",
                 "Command (from ziggy-llm_amd/):", "",
                 f"    python3 -m zhip.microbench --iters {args.iters} --formats {args.formats} "
                 f"--shapes {args.shapes} --out <file>", "",
                 "Each launch streams one of >= 1 GiB of distinct weight copies from HBM and is timed with its own",
                 "HIP events; GB/s counts the weight bytes plus x and y.", "",
                 "| format | rows x cols | weight + x + y bytes | avg us | GB/s | % of 8 TB/s |", "|---|---|---|---|---|---|"]
        for r in results:
            lines.append(f"| {r['format']} | {r['rows']} x {r['cols']} | {r['bytes']} | {r['avg_us']} | {r['gbs']} | "
                         f"{100 * r['frac_of_peak']:.1f} |")
        with open(args.out, "w") as fh:
            fh.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
