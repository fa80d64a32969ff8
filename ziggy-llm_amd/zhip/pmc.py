"""HBM traffic of the decode kernels from rocprofv3 counters.

Two steps, each its own process:

  probe      the program rocprofv3 profiles: builds the Llama-3.1-8B-shaped
             Q4_K_M model, fills its binary16 KV cache to --position rows,
             launches each decode kernel (--kernels) `--iters` times (rotating
             over the 32 layers, so every launch streams its weights from
             HBM), then one device copy of a known size used to calibrate the
             counters.  It writes the algorithmic bytes per launch of each
             kernel to --meta (JSON).
  summarize  reads the counter CSVs of two profiled runs (FETCH_SIZE, then
             WRITE_SIZE; both in KiB per dispatch) and writes a short
             markdown summary with the per-launch HBM bytes of each kernel,
             each counter scaled by what it reads for the copy:
                 factor_read  = FETCH_SIZE(copy) * 1024 / copy bytes
                 factor_write = WRITE_SIZE(copy) * 1024 / copy bytes
                 traffic      = FETCH_SIZE(kernel) * 1024 / factor_read
                              + WRITE_SIZE(kernel) * 1024 / factor_write

Usage (rocprofv3 runs the program directly after `--`):
  cd /tmp && export TMPDIR=/tmp && cd <repo>/ziggy-llm_amd
  rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir>/fetch -o pmc -- \\
      python3 -m zhip.pmc probe --meta <dir>/meta.json
  rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir>/write -o pmc -- \\
      python3 -m zhip.pmc probe --meta <dir>/meta.json
  python3 -m zhip.pmc summarize <dir>/fetch <dir>/write <dir>/meta.json --out ../profiles/<name>.md
  python3 -m zhip.pmc stats <trace dir> --title T --command C --out ../profiles/<name>.md
             (markdown table of a rocprofv3 --kernel-trace --stats run)
(the module lives in ziggy-llm_amd/, so run from there or put it on PYTHONPATH)
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import statistics
import json
import sys

COPY_BYTES = 512 << 20
# rocprof names of the Llama-3.1-8B-shaped step's kernels (Q4_K = 12, Q6_K = 14; IN_PLAIN 0 / IN_NORM 1;
# OUT_STORE 0 / OUT_ADD 1 / OUT_SWIGLU 2)
KERNEL_NAMES = {
    "qkv": ["mv_kernel<12, 14, 1, 0, 64"],
    "attention": ["attn_mfma_kernel<128, 4, false>"],
    # q/k/v and the attention in the one launch a decode step runs them in
    "qkv_attention": ["qkv_attn_kernel<12, 14, 128, 4>"],
    "o_proj": ["mv_kernel<12, 12, 0, 1, 64"],
    "gate_up": ["mv_kernel<12, 12, 1, 2, 64"],
    "down": ["mv_kernel<12, 12, 0, 1, 256", "mv_kernel<14, 14, 0, 1, 256"],
}


def probe(args) -> None:
    from . import hip, synth

    ctx_len = args.position + 64
    spec = synth.llama8b_spec(context=ctx_len)
    img = synth.build(spec, seed=args.seed)
    ctx = hip.Context(0)
    sess = hip.Session(ctx, img, context=ctx_len)
    sess.fill_kv_pattern(args.position, seed=1)
    meta = {"position": args.position, "kernels": {}}
    for name in args.kernels.split(","):
        ns, nb = sess.time_kernel(name, args.iters)
        print(f"{name}: {ns / 1e3:.2f} us per launch, {nb} algorithmic bytes (mean over the layers)", flush=True)
        per = {}
        if name == "down":
            # the Q4_K and Q6_K down layers stream different bytes: one entry per rocprof name
            q6 = [i for i in range(spec.n_layers) if synth.q6k_down_rule(i)]
            q4 = [i for i in range(spec.n_layers) if not synth.q6k_down_rule(i)]
            for needle, L in zip(KERNEL_NAMES["down"], (q4[0], q6[0])):
                per[needle] = img.tensors[f"blk.{L}.ffn_down.weight"].nbytes
        else:
            per[KERNEL_NAMES[name][0]] = nb
        meta["kernels"][name] = {"us": ns / 1e3, "algorithmic": per}
    sess.close()
    a = ctx.empty(COPY_BYTES)
    b = ctx.empty(COPY_BYTES)
    ctx.copy(a, 0, b, 0, COPY_BYTES)
    print(f"copy: {COPY_BYTES} bytes", flush=True)
    a.free()
    b.free()
    ctx.close()
    if args.meta:
        os.makedirs(os.path.dirname(os.path.abspath(args.meta)), exist_ok=True)
        with open(args.meta, "w") as fh:
            json.dump(meta, fh, indent=1)


def gemm_probe(args) -> None:
    """The program of the matrix-core counter runs: only the M >= 8 passes, few launches each.
    verify  Qwen3-8B-shaped Q8_0: an 8-token prompt (one batched pass of 7 rows), then --iters verify passes
            of the pending token and 8 seeded drafts (M = 9) at the same position;
    prompt  Llama-3.1-8B-shaped Q4_K_M: one 257-token prompt (one batched pass of 256 rows);
    moe     4 layers of the MoE FFN stack (hidden 2048, 256 IQ4_XS experts of FFN 512, top-8, Q3_K
            shared expert): one 512-row prefill (grouped expert GEMMs)."""
    import numpy as np

    from . import hip, synth

    ctx = hip.Context(0)
    if args.what == "verify":
        spec = synth.qwen3_8b_spec(context=128)
        img = synth.build(spec, seed=args.seed)
        s = hip.Session(ctx, img, context=128)
        _, st = s.generate(synth.prompt_tokens(args.seed, 8, spec.vocab), 0)
        p0, cur = s.position, int(st.next_token)
        drafts = [int(t) for t in synth.prompt_tokens(args.seed + 1, 8, spec.vocab)]
        for i in range(args.iters):
            s.rewind(p0)
            _, n = s.verify(cur, drafts)
            print(f"verify {i} at position {p0}: {n} emitted", flush=True)
        s.close()
    elif args.what == "prompt":
        spec = synth.llama8b_spec(context=320)
        img = synth.build(spec, seed=args.seed)
        s = hip.Session(ctx, img, context=320)
        _, st = s.generate(synth.prompt_tokens(args.seed, 257, spec.vocab), 0)
        print(f"prompt of 257 tokens: {st.prompt_ns / 1e6:.2f} ms", flush=True)
        s.close()
    else:
        spec = synth.moe_config5_spec(4)
        layers = synth.build_moe_stack(spec, seed=args.seed)
        st = hip.MoeStack(ctx, synth.moe_desc(spec), layers)
        xs = np.stack([synth.normal_row(args.seed + 1, t, spec.hidden, 0.0, 1.0) for t in range(512)])
        st.prefill(xs)
        print("moe prefill of 512 rows", flush=True)
        st.close()
    ctx.close()


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
    meta = json.load(open(args.meta))
    cname, cf = _pick(fetch, "copyBuffer")
    _, cw = _pick(write, "copyBuffer")
    c_fetch, c_write = max(cf), max(cw)
    f_read = c_fetch * 1024 / COPY_BYTES
    f_write = c_write * 1024 / COPY_BYTES
    lines = [
        f"# HBM traffic per launch: decode kernels, Llama-3.1-8B shape, KV cache at {meta['position']} positions",
        "",
        "Counters from two rocprofv3 runs of the same probe (FETCH_SIZE, then WRITE_SIZE;",
        "KiB per dispatch), each scaled by what it reads for a device copy of 512 MiB.",
        "",
        "Commands (from ziggy-llm_amd/, after `cd /tmp && export TMPDIR=/tmp`):",
        "",
        f"    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir>/fetch -o pmc -- python3 -m zhip.pmc probe "
        f"--position {meta['position']} --meta <dir>/meta.json",
        f"    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir>/write -o pmc -- python3 -m zhip.pmc probe "
        f"--position {meta['position']} --meta <dir>/meta.json",
        "    python3 -m zhip.pmc summarize <dir>/fetch <dir>/write <dir>/meta.json --out ../profiles/<this file>",
        "",
        f"Copy kernel `{cname[:80]}`: FETCH_SIZE {c_fetch:.1f} KiB, WRITE_SIZE {c_write:.1f} KiB for "
        f"{COPY_BYTES} bytes -> read factor {f_read:.4f}, write factor {f_write:.4f}.",
        "",
        "| kernel | rocprof name | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic bytes | algorithmic bytes "
        "| traffic / algorithmic |",
        "|---|---|---|---|---|---|---|---|",
    ]
    for name, info in meta["kernels"].items():
        for needle, algo in info["algorithmic"].items():
            kname, kf = _pick(fetch, needle)
            _, kw = _pick(write, needle)
            # the probe's first launch is a warm-up; the medians are robust to it
            k_fetch, k_write = statistics.median(kf), statistics.median(kw)
            traffic = k_fetch * 1024 / f_read + k_write * 1024 / f_write
            lines.append(f"| {name} | `{kname[:60]}` | {len(kf)} | {k_fetch:.1f} | {k_write:.1f} | "
                         f"{int(round(traffic))} | {algo} | {traffic / algo:.4f} |")
            if name == "gate_up":
                lines_tail = f"traffic_bytes_per_launch: {int(round(traffic))}"
    lines.append("")
    if "gate_up" in meta["kernels"]:
        lines.append("- " + lines_tail + " (gate_up, the bench's roofline kernel)")
        lines.append("")
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


REQ_COUNTERS = ("TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_sum")


def reqsize(args) -> None:
    """HBM read bytes by request size, from one --pmc run of the four REQ_COUNTERS over the probe:
    bytes = 32 x (32-byte requests) + 64 x (64-byte) + 128 x (128-byte), checked on the copy.  FETCH_SIZE
    prices every request that is not 32 bytes as 64 bytes plus 128 per TCC_BUBBLE; where a kernel's reads
    mix 64- and 128-byte requests, one copy-derived factor misprices some of them, and this split says how
    many."""
    rows = _dispatch_rows(args.pmc_dir)
    meta = json.load(open(args.meta))
    by: dict[str, list[dict]] = {}
    for d in rows.values():
        by.setdefault(d["name"], []).append(d["counters"])

    def med(name_needle, key):
        hits = [(k, v) for k, v in by.items() if name_needle in k]
        if not hits:
            raise SystemExit(f"no dispatch of a kernel matching {name_needle!r}")
        hits.sort(key=lambda kv: -len(kv[1]))
        return hits[0][0], len(hits[0][1]), statistics.median(c.get(key, 0.0) for c in hits[0][1])

    def sized(needle):
        name, n, r32 = med(needle, REQ_COUNTERS[0])
        _, _, r64 = med(needle, REQ_COUNTERS[1])
        _, _, r128 = med(needle, REQ_COUNTERS[2])
        _, _, rall = med(needle, REQ_COUNTERS[3])
        return name, n, r32, r64, r128, rall, 32 * r32 + 64 * r64 + 128 * r128

    # the calibration copy: the copyBuffer dispatch with the most read requests (the probe's small
    # uploads are copies too)
    cands = [(k, c) for k, cs in by.items() if "copyBuffer" in k for c in cs]
    if not cands:
        raise SystemExit("no copyBuffer dispatch")
    cname, cc = max(cands, key=lambda kc: kc[1].get(REQ_COUNTERS[3], 0.0))
    c32, c64, c128, call = (cc.get(k, 0.0) for k in REQ_COUNTERS)
    cbytes = 32 * c32 + 64 * c64 + 128 * c128
    lines = [f"# HBM read requests by size: decode kernels, Llama-3.1-8B shape, KV cache at {meta['position']} positions",
             "", "Command (from ziggy-llm_amd/, after `cd /tmp && export TMPDIR=/tmp`):", "",
             f"    rocprofv3 --pmc {' '.join(REQ_COUNTERS)} --output-format csv -d <dir> -o pmc -- python3 -m zhip.pmc "
             f"probe --position {meta['position']} --kernels {','.join(meta['kernels'])}",
             f"    python3 -m zhip.pmc reqsize <dir> <meta.json> --out ../profiles/<this file>", "",
             "read bytes = 32 x RDREQ_32B + 64 x RDREQ_64B + 128 x RDREQ_128B (median over the dispatches).",
             f"Copy `{cname[:60]}` of {COPY_BYTES} bytes: {c32:.0f} / {c64:.0f} / {c128:.0f} requests of 32 / 64 / "
             f"128 bytes ({call:.0f} in all) -> {cbytes:.0f} read bytes, {cbytes / COPY_BYTES:.4f} of the copy.", "",
             "| kernel | rocprof name | dispatches | 32 B | 64 B | 128 B | all | read bytes | algorithmic bytes "
             "| read / algorithmic |", "|---|---|---|---|---|---|---|---|---|---|"]
    for name, info in meta["kernels"].items():
        for needle, algo in info["algorithmic"].items():
            kname, n, r32, r64, r128, rall, kb = sized(needle)
            lines.append(f"| {name} | `{kname[:50]}` | {n} | {r32:.0f} | {r64:.0f} | {r128:.0f} | {rall:.0f} | "
                         f"{kb:.0f} | {algo} | {kb / algo:.4f} |")
    lines.append("")
    text = "\n".join(lines)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text)
    print(text)


MFMA_F16_PEAK_TFLOPS = 2500.0  # dense binary16 / bf16 matrix-core peak of the MI355X
SIMD_NUM = 1024  # 256 CUs x 4 SIMDs
CLOCK_GHZ = 2.4  # peak engine clock


def _dispatch_rows(dirname: str) -> dict[str, dict]:
    """{dispatch id: {"name", "counters": {name: value}, "ns"}} from a --pmc run.  Counters are collected
    in runs of their own, never with --kernel-trace: that combination once ended a profiled process with
    a SIGSEGV in a profiler thread (no GPU fault)."""
    files = glob.glob(os.path.join(dirname, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {dirname}")
    out: dict[str, dict] = {}
    for f in files:
        for r in csv.DictReader(open(f)):
            d = out.setdefault(r["Dispatch_Id"], {"name": r["Kernel_Name"], "counters": {}, "ns": None})
            c, k, v = d["counters"], r["Counter_Name"], float(r["Counter_Value"])
            # per-instance rows: GPU-wide cycle counts and percentages take the max, event counts add
            c[k] = max(c.get(k, v), v) if k.startswith("GRBM_") or k == "MfmaUtil" else c.get(k, 0.0) + v
            if r.get("Start_Timestamp") and r.get("End_Timestamp"):
                d["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    return out


def mfma(args) -> None:
    """Matrix-core use per kernel shape from one --pmc run of SQ_INSTS_VALU_MFMA_MOPS_F16,
    SQ_INSTS_VALU_MFMA_MOPS_BF16, SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE and MfmaUtil.  One MOPS unit is
    512 flops; MfmaUtil = MFMA-busy cycles summed over the SIMDs / (GPU-active cycles x 1024 SIMDs).  The
    launch time is the counter row's own duration when it has one, else the GPU-active cycles at the
    2.4 GHz peak engine clock (counter collection serialises launches).  Dispatches of one kernel with
    the same flops are one shape."""
    rows = _dispatch_rows(args.pmc_dir)
    groups: dict[tuple[str, int], list[dict]] = {}
    for d in rows.values():
        c = d["counters"]
        mops = c.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) + c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0)
        if mops <= 0:
            continue
        groups.setdefault((d["name"], int(mops)), []).append(d)

    def launch_ns(x):
        if x["ns"]:
            return x["ns"]
        gui = x["counters"].get("GRBM_GUI_ACTIVE", 0.0)
        return gui / CLOCK_GHZ if gui else None

    ranked = sorted(groups.items(), key=lambda kv: -sum((launch_ns(x) or 0) for x in kv[1]))
    lines = [f"# {args.title}", "", "Command:", "", f"    {args.command}", "",
             "One row per kernel shape (the dispatches of one kernel that issue the same matrix-core work).",
             "GFLOP per launch = (SQ_INSTS_VALU_MFMA_MOPS_F16 + _BF16) x 512; us = GRBM_GUI_ACTIVE cycles at",
             f"{CLOCK_GHZ} GHz (counter collection serialises launches); TFLOP/s = GFLOP over that; MFMA busy =",
             f"MfmaUtil (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x {SIMD_NUM} SIMDs)); peak "
             f"{MFMA_F16_PEAK_TFLOPS:.0f} TFLOP/s dense bf16 / binary16.",
             "",
             "| kernel | launches | GFLOP / launch | avg us | TFLOP/s | % of peak | MFMA busy % |",
             "|---|---|---|---|---|---|---|"]
    for (name, mops), ds in ranked[: args.top]:
        flops = mops * 512.0
        ns = [launch_ns(x) for x in ds if launch_ns(x)]
        avg_ns = statistics.median(ns) if ns else None
        util = [x["counters"]["MfmaUtil"] for x in ds if "MfmaUtil" in x["counters"]]
        if not util:
            util = [100.0 * x["counters"].get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) /
                    (x["counters"]["GRBM_GUI_ACTIVE"] * SIMD_NUM) for x in ds if x["counters"].get("GRBM_GUI_ACTIVE")]
        nm = name.replace("|", "/")
        nm = nm[:70] + "..." if len(nm) > 73 else nm
        tf = flops / avg_ns / 1e3 if avg_ns else None
        nan = float("nan")
        lines.append(f"| `{nm}` | {len(ds)} | {flops / 1e9:.3f} | {avg_ns / 1e3 if avg_ns else nan:.2f} | "
                     f"{tf if tf else nan:.1f} | {100 * tf / MFMA_F16_PEAK_TFLOPS if tf else nan:.2f} | "
                     f"{statistics.median(util) if util else nan:.2f} |")
    lines.append("")
    text = "\n".join(lines)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text)
    print(text)


def sq(args) -> None:
    """Instruction mix and stall shares per kernel shape from several --pmc runs of one program (each
    run its own counters; a run's dispatch ids follow the program's launch order, so the runs merge by
    dispatch id).  Dispatches of one kernel and grid with the same matrix-core instruction count are one
    shape.  Per wavefront: instructions by type (SQ_INSTS_*); shares of the wavefront's lifetime
    (SQ_WAVE_CYCLES, in quad cycles like the SQ_ACTIVE_INST_* and SQ_WAIT_* counters): issuing VALU / LDS /
    any instruction, waiting; matrix-core busy cycles per SIMD over the lifetime; LDS bank-conflict cycles
    over LDS-active cycles."""
    runs = [_dispatch_rows(d) for d in args.pmc_dirs]
    grids = {}
    for d in args.pmc_dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                grids[r["Dispatch_Id"]] = int(r.get("Grid_Size") or 0)
    merged: dict[str, dict] = {}
    for run in runs:
        for did, d in run.items():
            m = merged.setdefault(did, {"name": d["name"], "counters": {}})
            if m["name"] != d["name"]:
                raise SystemExit(f"dispatch {did} is {m['name']} in one run and {d['name']} in another")
            m["counters"].update(d["counters"])
    groups: dict[tuple, list[dict]] = {}
    for did, d in merged.items():
        c = d["counters"]
        if not c.get("SQ_WAVES"):
            continue
        key = (d["name"], grids.get(did, 0), int(c.get("SQ_INSTS_MFMA", 0)))
        groups.setdefault(key, []).append(c)
    wanted = [n for n in args.kernels.split(",") if n]
    lines = [f"# {args.title}", "", "Command:", "", f"    {args.command}", "",
             "One row per kernel shape (kernel, grid in threads, matrix-core instructions). Per wavefront:",
             "instructions by type; % of the wavefront's lifetime issuing VALU, LDS or any instruction, and",
             "waiting (SQ_ACTIVE_INST_* and SQ_WAIT_ANY over SQ_WAVE_CYCLES); MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES",
             "per wavefront over its lifetime in cycles; LDS conflict = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE.",
             "Medians over the shape's dispatches.", "",
             "| kernel | grid | launches | VALU | SALU | LDS | MFMA | VMEM rd | % VALU | % LDS | % any | % wait | "
             "% MFMA busy | % LDS conflict |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    med = statistics.median
    rows = sorted(groups.items(), key=lambda kv: -sum(c.get("SQ_WAVE_CYCLES", 0.0) for c in kv[1]))
    for (name, grid, _), cs in rows[: args.top]:
        if wanted and not any(w in name for w in wanted):
            continue

        def pw(k):
            return med([c.get(k, 0.0) / c["SQ_WAVES"] for c in cs])

        def share(k, scale=1.0):
            v = [scale * c.get(k, 0.0) / c["SQ_WAVE_CYCLES"] for c in cs if c.get("SQ_WAVE_CYCLES")]
            return 100.0 * med(v) if v else float("nan")
        conf = [c["SQ_LDS_BANK_CONFLICT"] / c["SQ_LDS_IDX_ACTIVE"] for c in cs if c.get("SQ_LDS_IDX_ACTIVE")]
        nm = name.split("(")[0].replace("void ", "").replace("|", "/")
        lines.append(f"| `{nm}` | {grid} | {len(cs)} | {pw('SQ_INSTS_VALU'):.0f} | {pw('SQ_INSTS_SALU'):.0f} | "
                     f"{pw('SQ_INSTS_LDS'):.0f} | {pw('SQ_INSTS_MFMA'):.0f} | {pw('SQ_INSTS_VMEM_RD'):.0f} | "
                     f"{share('SQ_ACTIVE_INST_VALU'):.1f} | {share('SQ_ACTIVE_INST_LDS'):.1f} | "
                     f"{share('SQ_ACTIVE_INST_ANY'):.1f} | {share('SQ_WAIT_ANY'):.1f} | "
                     f"{share('SQ_VALU_MFMA_BUSY_CYCLES', 0.25):.1f} | "
                     f"{100 * med(conf) if conf else float('nan'):.1f} |")
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
                return int(line.split(":", 1)[1].split()[0])
    except OSError:
        return None
    return None


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("probe")
    p.add_argument("--iters", type=int, default=32)
    p.add_argument("--seed", type=int, default=1)
    p.add_argument("--position", type=int, default=4096)
    p.add_argument("--kernels", default="qkv,attention,qkv_attention,o_proj,gate_up,down")
    p.add_argument("--meta")
    g = sub.add_parser("gemm-probe")
    g.add_argument("what", choices=["verify", "prompt", "moe"])
    g.add_argument("--iters", type=int, default=3)
    g.add_argument("--seed", type=int, default=1)
    s = sub.add_parser("summarize")
    s.add_argument("fetch_dir")
    s.add_argument("write_dir")
    s.add_argument("meta")
    s.add_argument("--out")
    r = sub.add_parser("reqsize")
    r.add_argument("pmc_dir")
    r.add_argument("meta")
    r.add_argument("--out")
    m = sub.add_parser("mfma")
    m.add_argument("pmc_dir")
    m.add_argument("--title", required=True)
    m.add_argument("--command", required=True)
    m.add_argument("--top", type=int, default=24)
    m.add_argument("--out")
    t = sub.add_parser("stats")
    t.add_argument("trace_dir")
    t.add_argument("--title", required=True)
    t.add_argument("--command", required=True)
    t.add_argument("--top", type=int, default=14)
    t.add_argument("--out")
    q = sub.add_parser("sq")
    q.add_argument("pmc_dirs", nargs="+")
    q.add_argument("--title", required=True)
    q.add_argument("--command", required=True)
    q.add_argument("--kernels", default="", help="comma-separated name fragments to keep (default: all)")
    q.add_argument("--top", type=int, default=16)
    q.add_argument("--out")
    args = ap.parse_args(argv)
    {"probe": probe, "gemm-probe": gemm_probe, "summarize": summarize, "reqsize": reqsize, "mfma": mfma, "stats": stats,
     "sq": sq}[args.cmd](args)


if __name__ == "__main__":
    main(sys.argv[1:])
