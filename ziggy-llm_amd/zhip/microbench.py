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

Two probes of the launch structure (no quantized work; they time the hardware):
  --chain [--position P]  the Llama-3.1-8B-shaped decode step's byte plan (each launch's weight or K/V
                          bytes at position P, in launch order) as one streaming kernel, as a HIP graph
                          of one streaming kernel per launch, and as a graph of as many empty kernels;
  --sync                  one-way hand-off latency between two CUs and the latency of a barrier of a
                          CU-sized grid, inside one launch.
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


def step_plan(spec, position: int) -> list:
    """Bytes each launch of one decode step streams, in launch order: the step-begin kernel (one
    embedding row), per layer q/k/v, attention (K/V rows 0..position), o_proj, gate/up and down, then the
    output head (the session's step graph, zh_session.cpp enqueue_step)."""
    t = {x.name: x for x in spec.tensors()}
    kv = spec.n_kv * spec.head_dim * 2 * 2 * (position + 1)
    plan = [row_bytes(t["token_embd.weight"].ttype, spec.hidden)]
    for i in range(spec.n_layers):
        b = lambda n: t[f"blk.{i}.{n}.weight"].nbytes  # noqa: E731
        plan += [b("attn_q") + b("attn_k") + b("attn_v"), kv, b("attn_output"), b("ffn_gate") + b("ffn_up"),
                 b("ffn_down")]
    plan.append(t["output.weight"].nbytes)
    return plan


def chain(args) -> dict:
    spec = synth.llama8b_spec(context=args.position + 16)
    plan = step_plan(spec, args.position)
    ctx = hip.Context(0)
    r = ctx.probe_chain(plan, reps=args.reps)
    ctx.close()
    gbs = lambda ms: r.bytes / (ms * 1e-3) / 1e9  # noqa: E731
    out = {"probe": "chain", "model": spec.name, "position": args.position, "kernels": r.kernels,
           "workgroups": r.workgroups, "bytes": r.bytes,
           "one_kernel_ms": round(r.one_kernel_ms, 4), "one_kernel_gbs": round(gbs(r.one_kernel_ms), 1),
           "chain_ms": round(r.chain_ms, 4), "chain_gbs": round(gbs(r.chain_ms), 1),
           "empty_chain_ms": round(r.empty_chain_ms, 4),
           "empty_us_per_kernel": round(1e3 * r.empty_chain_ms / r.kernels, 3)}
    print(json.dumps(out), flush=True)
    if args.out:
        lines = ["# Launch-structure probe: the decode step's byte plan, one MI355X", "",
                 "Command (from ziggy-llm_amd/):", "",
                 f"    python3 -m zhip.microbench --chain --position {args.position} --reps {args.reps} --out <file>",
                 "",
                 f"Plan: the {spec.name} step at position {args.position}: {r.kernels} launches (step begin, per "
                 "layer q/k/v, attention K/V, o_proj, gate/up, down, then the output head), each streaming its "
                 "bytes in shares of whole 128-byte lines over a grid of one workgroup per CU. Best of "
                 f"{args.reps} runs after a warm-up, HIP events around each.", "",
                 "| form | ms | GB/s | % of 8 TB/s |", "|---|---|---|---|",
                 f"| one streaming kernel over all {r.bytes} bytes | {out['one_kernel_ms']} | "
                 f"{out['one_kernel_gbs']} | {100 * out['one_kernel_gbs'] / HBM_PEAK_GBS:.1f} |",
                 f"| {r.kernels} streaming kernels in a graph | {out['chain_ms']} | {out['chain_gbs']} | "
                 f"{100 * out['chain_gbs'] / HBM_PEAK_GBS:.1f} |",
                 f"| {r.kernels} empty kernels in a graph | {out['empty_chain_ms']} | - | - |", "",
                 f"Empty kernels: {out['empty_us_per_kernel']} us per launch."]
        with open(args.out, "w") as fh:
            fh.write("\n".join(lines) + "\n")
    return out


def sync(args) -> dict:
    ctx = hip.Context(0)
    r = ctx.probe_sync(args.rounds)
    ctx.close()
    out = {"probe": "sync", "workgroups": r.workgroups, "timed_out": bool(r.timed_out), "rounds": args.rounds,
           "handoff_relaxed_us": round(r.handoff_relaxed_us, 3), "handoff_acqrel_us": round(r.handoff_acqrel_us, 3),
           "barrier_flags_us": round(r.barrier_flags_us, 3), "barrier_counter_us": round(r.barrier_counter_us, 3)}
    print(json.dumps(out), flush=True)
    if r.timed_out:
        raise SystemExit("a probe wait ran out of its bound: the figures are not valid")
    if args.out:
        lines = ["# In-launch dependency latencies, one MI355X", "", "Command (from ziggy-llm_amd/):", "",
                 f"    python3 -m zhip.microbench --sync --rounds {args.rounds} --out <file>", "",
                 f"Averages over {args.rounds} rounds, timed on the device (s_memrealtime, 100 MHz).", "",
                 "| dependency | us |", "|---|---|",
                 f"| one-way hand-off between two CUs, relaxed device-scope store and load | {out['handoff_relaxed_us']} |",
                 f"| the same, release store and acquire load | {out['handoff_acqrel_us']} |",
                 f"| barrier of {r.workgroups} workgroups: arrival words polled by one wavefront | "
                 f"{out['barrier_flags_us']} |",
                 f"| barrier of {r.workgroups} workgroups: one arrival counter | {out['barrier_counter_us']} |"]
        with open(args.out, "w") as fh:
            fh.write("\n".join(lines) + "\n")
    return out


def row_load(args) -> dict:
    ctx = hip.Context(0)
    r = ctx.probe_row_load(args.reps)
    ctx.close()
    out = {"probe": "row_load", "workgroups": r.workgroups, "values": r.values, "reps": args.reps,
           "slot_us": [round(v, 3) for v in r.slot_us], "coalesced_us": [round(v, 3) for v in r.coalesced_us],
           "lds_us": [round(v, 3) for v in r.lds_us]}
    print(json.dumps(out), flush=True)
    if args.out:
        kb = r.values * 4 // 1024
        lines = ["# Input-row load patterns, one MI355X", "", "Command (from ziggy-llm_amd/):", "",
                 f"    python3 -m zhip.microbench --row-load --reps {args.reps} --out <file>", "",
                 f"{r.workgroups} workgroups of 256 lanes (two per CU); each brings a {r.values}-float row "
                 f"({kb} KiB), written by the launch before, into every lane's registers (each wavefront holds "
                 "the whole row, 64 floats a lane), optionally with a second row of the same size (RMSNorm "
                 "weights). Median over workgroups of the time from the first load to every lane holding its "
                 f"values (s_memrealtime, 100 MHz); median of {args.reps} launches.", "",
                 "| load pattern | row alone, us | row + second row, us |", "|---|---|---|",
                 f"| every lane loads its own 256-byte slot (16-byte loads 256 bytes apart) | "
                 f"{out['slot_us'][0]} | {out['slot_us'][1]} |",
                 f"| coalesced 16-byte loads, same bytes per wavefront | {out['coalesced_us'][0]} | "
                 f"{out['coalesced_us'][1]} |",
                 f"| once per workgroup, coalesced, through LDS; slots read there | {out['lds_us'][0]} | "
                 f"{out['lds_us'][1]} |"]
        with open(args.out, "w") as fh:
            fh.write("\n".join(lines) + "\n")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--chain", action="store_true", help="the decode step's launch-structure probe")
    ap.add_argument("--sync", action="store_true", help="in-launch dependency latencies")
    ap.add_argument("--row-load", action="store_true", help="input-row load patterns")
    ap.add_argument("--position", type=int, default=4096)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--rounds", type=int, default=2000)
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--formats", default="q4_k,q6_k,q8_0")
    ap.add_argument("--shapes", default=",".join(f"{r}x{c}" for r, c in SHAPES),
                    help="comma-separated ROWSxCOLS list")
    ap.add_argument("--out", help="also write the results as a markdown table")
    args = ap.parse_args()
    if args.chain or args.sync or args.row_load:
        if args.chain:
            chain(args)
        if args.sync:
            sync(args)
        if args.row_load:
            row_load(args)
        return
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
