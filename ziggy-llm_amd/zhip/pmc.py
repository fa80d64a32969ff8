"""HBM traffic of the dominant decode kernel from rocprofv3 counters.

Two steps, each its own process:

  probe      the program rocprofv3 profiles: builds the Llama-3.1-8B-shaped
             Q4_K_M model, launches the fused RMSNorm + gate/up + SwiGLU
             kernel `--iters` times (rotating over the 32 layers, so every
             launch streams its 66 MB of weights from HBM), then one device
             copy of a known size used to calibrate the counters.
  summarize  reads the counter CSVs of two profiled runs (FETCH_SIZE, then
             WRITE_SIZE; both in KiB per dispatch) and writes a short
             markdown summary with the per-launch HBM bytes of the kernel,
             each counter scaled by what it reads for the copy:
                 factor_read  = FETCH_SIZE(copy) * 1024 / copy bytes
                 factor_write = WRITE_SIZE(copy) * 1024 / copy bytes
                 traffic      = FETCH_SIZE(kernel) * 1024 / factor_read
                              + WRITE_SIZE(kernel) * 1024 / factor_write

Usage (rocprofv3 runs the program directly after `--`):
  cd /tmp && export TMPDIR=/tmp && cd <repo>
  rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir>/fetch -o pmc -- \\
      python3 -m zhip.pmc probe
  rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir>/write -o pmc -- \\
      python3 -m zhip.pmc probe
  python3 -m zhip.pmc summarize <dir>/fetch <dir>/write --out profiles/<name>.md
  python3 -m zhip.pmc stats <trace dir> --title T --command C --out profiles/<name>.md
             (markdown table of a rocprofv3 --kernel-trace --stats run)
(the module lives in ziggy-llm_amd/, so run from there or put it on PYTHONPATH)
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import statistics
import sys

GATE_UP_KERNEL = "mv_kernel<12, 12, 1, 2"  # Q4_K, Q4_K, IN_NORM, OUT_SWIGLU
COPY_BYTES = 512 << 20


def probe(args) -> None:
    import numpy as np

    from . import hip, synth

    spec = synth.llama8b_spec(context=64)
    img = synth.build(spec, seed=args.seed)
    ctx = hip.Context(0)
    sess = hip.Session(ctx, img, context=64)
    sess.generate(synth.prompt_tokens(args.seed, 4, spec.vocab), 1)
    ns, nb = sess.time_kernel("gate_up", args.iters)
    print(f"gate_up: {ns / 1e3:.2f} us per launch, {nb} algorithmic bytes", flush=True)
    sess.close()
    a = ctx.empty(COPY_BYTES)
    b = ctx.empty(COPY_BYTES)
    ctx.copy(a, 0, b, 0, COPY_BYTES)
    print(f"copy: {COPY_BYTES} bytes", flush=True)
    a.free()
    b.free()
    ctx.close()
    del np


def _per_dispatch(dirname: str, counter: str) -> dict[str, list[float]]:
    files = glob.glob(os.path.join(dirname, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {dirname}")
    sums: dict[tuple[str, str], float] = {}
    for f in files:
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] != counter:
                continue
            key = (r["Dispatch_Id"], r["Kernel_Name"])
            sums[key] = sums.get(key, 0.0) + float(r["Counter_Value"])
    out: dict[str, list[float]] = {}
    for (_, name), v in sums.items():
        out.setdefault(name, []).append(v)
    return out


def _pick(d: dict[str, list[float]], needle: str) -> tuple[str, list[float]]:
    hits = [(k, v) for k, v in d.items() if needle in k]
    if not hits:
        raise SystemExit(f"no dispatch of a kernel matching {needle!r}; kernels: {sorted(d)[:12]}")
    hits.sort(key=lambda kv: -len(kv[1]))
    return hits[0]


def summarize(args) -> None:
    fetch = _per_dispatch(args.fetch_dir, "FETCH_SIZE")
    write = _per_dispatch(args.write_dir, "WRITE_SIZE")
    kname, kf = _pick(fetch, GATE_UP_KERNEL)
    _, kw = _pick(write, GATE_UP_KERNEL)
    cname, cf = _pick(fetch, "copyBuffer")
    _, cw = _pick(write, "copyBuffer")
    # the probe's first launch is a warm-up; the medians are robust to it
    k_fetch, k_write = statistics.median(kf), statistics.median(kw)
    c_fetch, c_write = max(cf), max(cw)
    f_read = c_fetch * 1024 / COPY_BYTES
    f_write = c_write * 1024 / COPY_BYTES
    traffic = k_fetch * 1024 / f_read + k_write * 1024 / f_write
    algo = 66060288  # 2 x 14336 x 4096 Q4_K weights (144 B per 256 values)
    lines = [
        "# HBM traffic per launch: fused RMSNorm + Q4_K gate/up + SwiGLU, Llama-3.1-8B shape",
        "",
        "Counters from two rocprofv3 runs of the same probe (FETCH_SIZE, then WRITE_SIZE;",
        "KiB per dispatch), each scaled by what it reads for a device copy of 512 MiB.",
        "",
        "Commands (from ziggy-llm_amd/, after `cd /tmp && export TMPDIR=/tmp`):",
        "",
        "    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir>/fetch -o pmc -- python3 -m zhip.pmc probe",
        "    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir>/write -o pmc -- python3 -m zhip.pmc probe",
        "    python3 -m zhip.pmc summarize <dir>/fetch <dir>/write --out ../profiles/<this file>",
        "",
        f"- kernel: `{kname[:120]}` ({len(kf)} dispatches)",
        f"- FETCH_SIZE median: {k_fetch:.1f} KiB; WRITE_SIZE median: {k_write:.1f} KiB",
        f"- copy kernel `{cname[:80]}`: FETCH_SIZE {c_fetch:.1f} KiB, WRITE_SIZE {c_write:.1f} KiB for "
        f"{COPY_BYTES} bytes -> read factor {f_read:.4f}, write factor {f_write:.4f}",
        f"- algorithmic bytes per launch: {algo}",
        f"- traffic_bytes_per_launch: {int(round(traffic))}",
        f"- traffic / algorithmic: {traffic / algo:.4f}",
        "",
    ]
    text = "\n".join(lines)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text)
    print(text)


def stats(args) -> None:
    """Markdown summary of a rocprofv3 --kernel-trace --stats run."""
    files = glob.glob(os.path.join(args.trace_dir, "**", "*kernel_stats.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_stats.csv under {args.trace_dir}")
    rows = list(csv.DictReader(open(files[0])))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    lines = [f"# {args.title}", "", "Command:", "", f"    {args.command}", "",
             "| kernel | calls | avg us | total ms | % |", "|---|---|---|---|---|"]
    for r in rows[: args.top]:
        name = r["Name"].replace("|", "/")
        if len(name) > 90:
            name = name[:87] + "..."
        lines.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['TotalDurationNs']) / 1e6:.2f} | {float(r['Percentage']):.1f} |")
    lines.append("")
    text = "\n".join(lines)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text)
    print(text)


def read_traffic(path: str) -> int | None:
    """traffic_bytes_per_launch from a summary written by `summarize`, or None."""
    try:
        for line in open(path):
            if "traffic_bytes_per_launch:" in line:
                return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("probe")
    p.add_argument("--iters", type=int, default=32)
    p.add_argument("--seed", type=int, default=1)
    s = sub.add_parser("summarize")
    s.add_argument("fetch_dir")
    s.add_argument("write_dir")
    s.add_argument("--out")
    t = sub.add_parser("stats")
    t.add_argument("trace_dir")
    t.add_argument("--title", required=True)
    t.add_argument("--command", required=True)
    t.add_argument("--top", type=int, default=14)
    t.add_argument("--out")
    args = ap.parse_args(argv)
    {"probe": probe, "summarize": summarize, "stats": stats}[args.cmd](args)


if __name__ == "__main__":
    main(sys.argv[1:])
