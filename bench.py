"""Decode benchmark: Llama-3.1-8B-shaped Q4_K_M, batch 1, 4k context, one MI355X.

A "step" is one greedy decode step (one token through every layer and the
output head).  The KV cache is first filled by a 4096-token seeded prompt
(batched passes of up to 256 tokens on the matrix cores, the last prompt token
through the decode step; the reference's runPrompt feeds the same rows token
by token and the K/V rows agree), then W untimed warm-up steps run, then
exactly K timed steps (positions ~4.1k).  tok/s = K / decode wall time, the reference's definition
(runtime/types.zig:220-223).  Weights are random N(0, 0.02) of the
Llama-3.1-8B shape quantized by this package's own Q4_K_M mix; data is
synthetic.

Also reported, on the same JSON line:
  hbm_fraction  -- (weight + KV bytes per token) x tok/s / 8 TB/s;
  roofline      -- the dominant kernel (fused RMSNorm + gate/up + SwiGLU, Q4_K):
                   its algorithmic bytes per launch (66,060,288 B: 2 x 14336 x
                   4096 weights at 144 B per 256) over its mean launch time,
                   measured here with one pair of HIP events on the session
                   stream around back-to-back launches rotating over the 32
                   layers (weights stream from HBM), against the 8 TB/s peak;
                   `traffic` is the HBM bytes per launch from the committed
                   rocprofv3 FETCH_SIZE / WRITE_SIZE summary
                   (profiles/decode_kernels_llama8b_4k_hbm_traffic.md), else null;
  cpu_baseline  -- the CPU oracle (a C restatement of the reference's CPU
                   decode path, same threads policy: 1 + min(11, ncpu - 1))
                   decoding the same model at the same context on host cores;
  other_configs -- the other benchmark configurations in the same run (skip with
                   --no-other-configs): TinyLlama decode of 128 tokens after a
                   32-token prompt; the matvec microbench (Q4_K, Q6_K, Q8_0 at
                   its four shapes); Qwen3-8B Q8_0 decode of 128 tokens at 16k
                   context and its verify step (1 + 8 drafts); the 40-layer MoE
                   stack's decode and 512-row prefill.
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "ziggy-llm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_TFLOPS = 2500.0  # dense bf16 matrix-core peak
# a verify prediction may differ from the decoded draft only within this top-2 logit margin
VERIFY_TIE_ABS, VERIFY_TIE_REL = 1e-3, 1e-4


CPU_MAX_STEPS = 64  # upper bound on the CPU baseline's decode steps


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def context_length(model, prompt, warmup, steps, profile_steps=0):
    """KV rows the run needs.  The GPU decode uses prompt + warmup rows, then 1 + steps more (the pending
    token and the timed steps), then the profiled steps; time_kernel needs one free row after that; the CPU
    baseline fills its cache to pos0 = prompt + warmup + 1 and then decodes up to CPU_MAX_STEPS steps;
    config 4's verify adds three passes of 9 rows (drafts decoded, the position rewound, then verified)."""
    rows = prompt + warmup + 1 + max(steps + 1 + profile_steps, CPU_MAX_STEPS)
    if model == "qwen3":
        rows += 3 * 9
    return rows + 8


def cpu_step_budget(ctx_len, pos0):
    """CPU baseline steps that fit the cache after pos0 (a step at position p needs p < ctx_len)."""
    return max(0, min(CPU_MAX_STEPS, ctx_len - pos0))


def verify_passes(sess, cur, ms_per_step, spec, passes=3):
    """Config 4's speculative-verify step: the pending token and 8 drafts in one batched pass on the
    matrix cores, against the 9 decode steps it replaces.  The drafts are the stream's own next tokens
    (decoded one step at a time with their top-2 logits, then the position rewound), so all are
    accepted.  The pass adds its products in another order than the decode step, so a prediction may
    differ from the decoded draft only where the decode step's top-2 logits are within a near-tie
    margin; any other difference fails the bench.  The median of `passes` passes is reported."""
    times, mismatches, accepted = [], 0, []
    for _ in range(passes):
        p0 = sess.position
        drafts, margins, t = [], [], cur
        for _ in range(8):
            ids, lg = sess.step_shortlist(t, 2)
            drafts.append(int(ids[0]))
            margins.append((float(lg[0]) - float(lg[1]), float(abs(lg[0]))))
            t = int(ids[0])
        sess.rewind(p0)
        t1 = time.perf_counter()
        pred, n = sess.verify(cur, drafts)
        times.append(time.perf_counter() - t1)
        for j, (a, b) in enumerate(zip(pred[:8], drafts)):
            if int(a) != int(b):
                mismatches += 1
                gap, mag = margins[j]
                if gap > VERIFY_TIE_ABS + VERIFY_TIE_REL * mag:
                    raise SystemExit(f"verify pass: prediction {j} is {int(a)}, the decode step's is {b} "
                                     f"with a top-2 margin of {gap:.3g} (not a near-tie)")
        accepted.append(int(n))
        cur = int(pred[n - 1])
    tv = sorted(times)[len(times) // 2]
    # the pass reads every weight once (the output head included) for its 9 rows
    wbytes = spec.weight_bytes_per_token()
    log(f"verify (1 + 8 drafts, MFMA GEMMs): {1e3 * tv:.3f} ms vs {9 * ms_per_step:.3f} ms for 9 decode steps")
    return {"tokens": 9, "drafts": 8, "ms": round(1e3 * tv, 3), "accepted": accepted,
            "prediction_mismatches": mismatches, "tok_s_equiv": round(9 / tv, 1),
            "decode_ms_for_9": round(9 * ms_per_step, 3),
            "weight_bytes": wbytes, "weights_hbm_fraction": round(wbytes / tv / (HBM_PEAK_GBS * 1e9), 4)}


def decode_measure(model, prompt_len, steps, seed, warmup=4, verify=False):
    """A decode run of config 1 (tinyllama) or 4 (qwen3) for the headline line's other_configs: the
    prompt in batched passes, `warmup` untimed steps, `steps` timed greedy steps (one graph replay
    each), and for config 4 the speculative-verify passes (verify_passes)."""
    import numpy as np

    from zhip import hip, synth

    ctx_len = prompt_len + warmup + 1 + steps + 1 + (3 * 9 + 8 if verify else 0) + 8
    spec = {"tinyllama": synth.tinyllama_spec, "qwen3": synth.qwen3_8b_spec}[model](context=ctx_len)
    t0 = time.time()
    img = synth.build(spec, seed=seed)
    ctx = hip.Context(0)
    sess = hip.Session(ctx, img, context=ctx_len)
    prompt = synth.prompt_tokens(seed, prompt_len, spec.vocab)
    _, wst = sess.generate(prompt, warmup)
    _, st = sess.generate(np.array([wst.next_token], np.uint32), steps)
    wall_s = st.wall_ns / 1e9
    tok_s, ms = steps / wall_s, 1e3 * wall_s / steps
    pos0 = prompt_len + warmup + 1
    bpt = spec.weight_bytes_per_token() + spec.kv_bytes_per_token(int(round(pos0 + (steps - 1) / 2.0)))
    frac = bpt * tok_s / (HBM_PEAK_GBS * 1e9)
    out = {"workload": f"{spec.name} greedy decode, batch 1, positions {pos0}-{pos0 + steps - 1} after a "
                       f"{prompt_len}-token prompt",
           "tok_s": round(tok_s, 3), "ms_per_step": round(ms, 4), "hbm_fraction": round(frac, 4),
           "bytes_per_token": bpt, "prompt_ms": round(wst.prompt_ns / 1e6, 3)}
    log(f"{spec.name}: {tok_s:.1f} tok/s ({ms:.3f} ms/step) at positions {pos0}-{pos0 + steps - 1}, "
        f"{100 * frac:.1f}% of HBM peak ({time.time() - t0:.1f}s with the build)")
    if verify:
        out["verify"] = verify_passes(sess, int(st.next_token), ms, spec)
    sess.close()
    ctx.close()
    return out


def matvec_measure(iters):
    """Config 2: the dequant-matvec microbench (zhip.microbench) over its formats and shapes."""
    from zhip import hip, microbench

    ctx = hip.Context(0)
    res = []
    for name, fmt in microbench.FORMATS.items():
        for rows, cols in microbench.SHAPES:
            r = microbench.run(ctx, fmt, rows, cols, iters)
            res.append({k: r[k] for k in ("format", "rows", "cols", "avg_us", "gbs", "frac_of_peak")})
    ctx.close()
    log("matvec microbench: " + ", ".join(f"{r['format']} {r['rows']}x{r['cols']} {r['gbs']:.0f} GB/s" for r in res))
    return res


def other_configs(args):
    """The other benchmark configurations, measured in the same run at their own workloads (shorter samples
    than their own --model lines): 1 TinyLlama decode, 2 the matvec microbench, 4 Qwen3-8B decode at
    16k plus the verify step, 5 the MoE stack's decode and 512-row prefill."""
    out = {"config1_tinyllama": decode_measure("tinyllama", 32, 128, args.seed),
           "config2_matvec": matvec_measure(64),
           "config4_qwen3_16k": decode_measure("qwen3", 16384, 128, args.seed, verify=True)}
    _, _, dec, prefill = moe_measure(args.seed, 64, 4)
    out["config5_moe"] = {"workload": "qwen3.5-moe-ffn-stack, 40 layers, batch-1 decode and a 512-row prefill",
                          "decode": dec, "prefill": prefill}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--model", default="llama8b", choices=["llama8b", "tinyllama", "qwen3", "moe"],
                    help="llama8b: the headline (config 3); tinyllama, qwen3: configs 1 and 4; "
                         "moe: config 5, the 40-layer MoE FFN stack at batch-1 decode")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-iters", type=int, default=64)
    ap.add_argument("--profile-steps", type=int, default=0,
                    help="after the timed decode, this many more steps with every launch timed by HIP events "
                         "under the reference's profile categories (its --metal-profile report)")
    ap.add_argument("--profile-out", default=None, help="file for the profile summary (default: stderr)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the other benchmark configurations the headline run also measures (other_configs)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported (batch-1 decode of this "
              f"model does not shard profitably: each GPU would stream its share of every layer's weights in "
              f"turn, with a collective per layer)", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    from zhip import hip, synth

    if args.model == "moe":
        return bench_moe(args)

    ctx_len = context_length(args.model, args.prompt, args.warmup, args.steps, args.profile_steps)
    spec = {"llama8b": synth.llama8b_spec, "tinyllama": synth.tinyllama_spec,
            "qwen3": synth.qwen3_8b_spec}[args.model](context=ctx_len)
    t0 = time.time()
    img = synth.build(spec, seed=args.seed)
    log(f"built {spec.name} ({img.buf.nbytes / 1e9:.2f} GB) in {time.time() - t0:.1f}s")

    ctx = hip.Context(0)
    t0 = time.time()
    sess = hip.Session(ctx, img, context=ctx_len)
    startup_s = time.time() - t0
    log(f"session on {ctx.info.name.decode()} ({ctx.info.arch.decode()}, {ctx.info.compute_units} CUs) "
        f"in {startup_s:.1f}s")

    prompt = synth.prompt_tokens(args.seed, args.prompt, spec.vocab)
    t0 = time.time()
    warm_tokens, wst = sess.generate(prompt, args.warmup)
    first_call_s = time.time() - t0
    # the batched passes cover every prompt row but the last (which runs through the decode step)
    pflops = spec.prompt_pass_flops(args.prompt - 1)
    ptflops = pflops / max(wst.prompt_ns, 1) / 1e3
    prefill = {"tokens": args.prompt, "ms": round(wst.prompt_ns / 1e6, 3),
               "tok_s": round(args.prompt / max(wst.prompt_ns, 1) * 1e9, 1),
               "tflops": round(ptflops, 2), "mfma_fraction_bf16": round(ptflops / MFMA_BF16_TFLOPS, 5),
               "path": "batched passes of up to 256 tokens (MFMA GEMMs, multi-query causal attention), "
                       "the last token through the decode step"}
    log(f"prefill {args.prompt} tokens in {wst.prompt_ns / 1e6:.1f} ms ({prefill['tok_s']} tok/s); with "
        f"{args.warmup} warm-up steps {time.time() - t0:.1f}s")

    # the cold run (runtime/bench_runner.zig:32-105 reports it beside the warm averages): session
    # creation (weight upload, buffers), the first generate call (step graph capture, the prompt
    # passes, the warm-up steps) and the warm-up steps' own decode rate
    cold = {"startup_ms": round(1e3 * startup_s, 1), "first_call_ms": round(1e3 * first_call_s, 1),
            "prompt_ms": round(wst.prompt_ns / 1e6, 3), "decode_steps": args.warmup,
            "decode_tok_s": round(args.warmup / max(wst.wall_ns, 1) * 1e9, 1) if args.warmup else None}
    toks, st = sess.generate(np.array([wst.next_token], np.uint32), args.steps)
    wall_s = st.wall_ns / 1e9
    tok_s = args.steps / wall_s
    ms_per_step = 1000.0 * wall_s / args.steps
    pos0 = args.prompt + args.warmup + 1
    mean_pos = pos0 + (args.steps - 1) / 2.0
    bytes_per_token = spec.weight_bytes_per_token() + spec.kv_bytes_per_token(int(round(mean_pos)))
    hbm_frac = bytes_per_token * tok_s / (HBM_PEAK_GBS * 1e9)
    log(f"decode: {tok_s:.1f} tok/s ({ms_per_step:.3f} ms/step, gpu events {st.gpu_elapsed_ns / 1e6 / args.steps:.3f}"
        f" ms/step), {bytes_per_token / 1e9:.3f} GB/token -> {100 * hbm_frac:.1f}% of HBM peak")
    next_tok = int(st.next_token)

    profile = None
    if args.profile_steps > 0:
        # the reference's decode profile (runtime/metal_profile.zig; printed as "metal_profile:" by
        # runtime/mod.zig:177-178): direct launches, so these steps are slower than the timed ones
        ptoks, recs = sess.profile_decode(next_tok, args.profile_steps)
        next_tok = int(ptoks[-1])
        text = hip.render_profile(recs)
        kv = hip.parse_profile(text)
        if args.profile_out:
            with open(args.profile_out, "w") as f:
                f.write(text)
        else:
            print("metal_profile:\n" + text, file=sys.stderr, end="", flush=True)
        profile = {"steps": args.profile_steps, "decode_ns": int(kv["profiled_decode_ns"]),
                   "commit_wait_gpu_ns": int(kv["profile.commit_wait.gpu_ns"]),
                   "share_pct": {c: float(kv[f"profile.{c}.share_pct"]) for c in hip.PROFILE_CATEGORIES},
                   "top_bottlenecks": [kv[f"profile.top_bottleneck_{i}"] for i in (1, 2, 3)],
                   "out": args.profile_out}
        log(f"profile: {args.profile_steps} steps, top {profile['top_bottlenecks']}")

    verify = None
    if args.model == "qwen3":
        verify = verify_passes(sess, next_tok, ms_per_step, spec)

    kernels = {}
    # each launch alone; qkv_attention is q/k/v and the attention in the one
    # launch a decode step runs them in (absent where the session keeps two)
    for name in ("qkv", "attention", "qkv_attention", "o_proj", "gate_up", "down", "output"):
        iters = args.kernel_iters if name != "output" else max(4, args.kernel_iters // 8)
        try:
            ns, nb = sess.time_kernel(name, iters)
        except hip.HipError:
            if name != "qkv_attention":
                raise
            continue
        kernels[name] = {"avg_us": round(ns / 1e3, 2), "bytes": nb, "gbs": round(nb / ns, 1) if ns else None}
        log(f"kernel {name}: {ns / 1e3:.2f} us, {nb / 1e6:.2f} MB -> {nb / max(ns, 1):.0f} GB/s")
    dom = kernels["gate_up"]
    traffic = None
    if args.model == "llama8b":
        from zhip import pmc
        traffic = pmc.read_traffic(os.path.join(REPO, "profiles", "decode_kernels_llama8b_4k_hbm_traffic.md"))
    gate_fmt = {"llama8b": "Q4_K", "tinyllama": "Q4_K", "qwen3": "Q8_0"}.get(args.model, "quantized")
    roofline = {"bound": "hbm", "kernel": f"gate_up (fused RMSNorm + {gate_fmt} gate/up + SwiGLU)",
                "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "bytes_per_launch": dom["bytes"], "avg_launch_us": dom["avg_us"]}
    sess.close()
    ctx.close()

    others = None
    if args.model == "llama8b" and not args.no_other_configs:
        others = other_configs(args)

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import zo
        ncpu = os.cpu_count() or 1
        threads = 1 + min(11, ncpu - 1)
        m = zo.Model(img.buf)
        o = zo.Session(m, context=ctx_len, kv_f16=False, threads=threads)
        o.fill_kv_pattern(pos0, seed=1)
        tok = int(toks[0])
        budget = cpu_step_budget(ctx_len, pos0)
        n, t_cpu = 0, 0.0
        while n < budget and (t_cpu < args.cpu_seconds or n < 2):
            t1 = time.perf_counter()
            tok = o.step_greedy(tok)
            t_cpu += time.perf_counter() - t1
            n += 1
        o.close()
        cpu = {"value": round(n / t_cpu, 4), "unit": "tok/s", "cores": threads, "host_cores": ncpu,
               "kind": "port",
               "sample": f"{n} greedy decode steps of the same {spec.name} model from position {pos0} "
                         f"(KV cache filled with a fixed pattern; decode cost does not depend on its values), "
                         f"C restatement of the reference CPU path, {threads} threads of {ncpu} host cores"}
        log(f"cpu baseline: {cpu['value']} tok/s over {n} steps ({t_cpu:.1f}s)")

    if args.model == "llama8b":
        metric = "decode tok/s + % of HBM roofline, Llama-3.1-8B-shaped Q4_K_M, batch 1, 4k ctx"
        weights = "Q4_K (Q6_K attn_v, 16/32 ffn_down, output), random N(0,0.02)"
    elif args.model == "qwen3":
        metric = "decode tok/s + % of HBM roofline, Qwen3-8B-shaped Q8_0, batch 1"
        weights = "Q8_0 throughout, per-head QK RMSNorm, random N(0,0.02)"
    else:
        metric = "decode tok/s + % of HBM roofline, TinyLlama-1.1B-shaped Q4_K_M, batch 1"
        weights = "Q4_K (Q6_K attn_v, 10/22 ffn_down, output), random N(0,0.02)"
    line = {
        "metric": metric,
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{spec.name} greedy decode, batch 1, positions {pos0}-{pos0 + args.steps - 1}"
                               f" after a {args.prompt}-token prompt",
                   "weights": weights,
                   "kv_cache": "binary16", "batch": 1, "context": pos0 + args.steps, "parallelism": "none"},
        "hbm_fraction": round(hbm_frac, 4),
        "bytes_per_token": bytes_per_token,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "verify": verify,
        "prefill": prefill,
        "cold": cold,
        "profile": profile,
        "tokens_head": [int(t) for t in toks[:8]],
        "other_configs": others,
    }
    print(json.dumps(line), flush=True)


def moe_measure(seed, steps, warmup):
    """Config 5: 40 Qwen3.5-MoE-style sparse FFN layers (hidden 2048, 256 IQ4_XS experts of FFN 512, top-8
    softmax routing, a Q3_K shared expert with a sigmoid gate) at batch-1 decode.  A step is one token's
    hidden state through the whole stack (one graph replay); weights resident in HBM.  Also the
    512-row prefill.  Returns the spec, the layers (host copies) and the decode and prefill figures."""
    import numpy as np

    from zhip import hip, synth

    spec = synth.moe_config5_spec(40)
    t0 = time.time()
    layers = synth.build_moe_stack(spec, seed=seed)
    log(f"built {spec.name}: {spec.n_layers} layers in {time.time() - t0:.1f}s")
    ctx = hip.Context(0)
    st = hip.MoeStack(ctx, synth.moe_desc(spec), layers)
    x = synth.normal_row(seed, 0, spec.hidden, 0.0, 1.0)
    for _ in range(max(1, warmup)):
        x, _, _ = st.forward(x)
    ns = st.time(steps)
    tok_s = 1e9 / ns
    bpt = spec.weight_bytes_per_token()
    frac = bpt * tok_s / (HBM_PEAK_GBS * 1e9)
    log(f"moe stack: {ns / 1e3:.1f} us per token, {tok_s:.1f} tok/s, {bpt / 1e6:.1f} MB/token -> "
        f"{100 * frac:.1f}% of HBM peak")
    # the 512-token prefill: rows grouped by routed expert per layer, expert GEMMs on the matrix cores
    ptok = 512
    xs = np.stack([synth.normal_row(seed + 1, t, spec.hidden, 0.0, 1.0) for t in range(ptok)])
    _, psel, _ = st.prefill(xs)
    pns = st.time_prefill(ptok, max(1, min(steps, 8)))
    touched = float(np.mean([len(np.unique(psel[:, l, :])) for l in range(spec.n_layers)]))
    pbytes = spec.weight_bytes_all()
    pflops = spec.flops_per_token() * ptok
    prefill = {"tokens": ptok, "ms": round(pns / 1e6, 3), "tok_s": round(ptok * 1e9 / pns, 1),
               "weight_bytes": pbytes, "experts_touched_per_layer": round(touched, 1),
               "hbm_fraction": round(pbytes / (pns * 1e-9) / (HBM_PEAK_GBS * 1e9), 4),
               "tflops": round(pflops / (pns * 1e-9) / 1e12, 2),
               "mfma_fraction_bf16": round(pflops / (pns * 1e-9) / (MFMA_BF16_TFLOPS * 1e12), 5)}
    log(f"moe prefill: {ptok} rows in {pns / 1e6:.2f} ms ({prefill['tok_s']} tok/s), "
        f"{pbytes / 1e9:.2f} GB of weights -> {100 * prefill['hbm_fraction']:.1f}% of HBM peak, "
        f"{prefill['tflops']} TFLOP/s")
    st.close()
    ctx.close()
    decode = {"tok_s": round(tok_s, 3), "ms_per_step": round(ns / 1e6, 4), "hbm_fraction": round(frac, 4),
              "bytes_per_token": bpt}
    return spec, layers, decode, prefill


def bench_moe(args):
    """Config 5 as the bench's own line (--model moe), with its CPU baseline."""
    import numpy as np

    from zhip import synth

    spec, layers, dec, prefill = moe_measure(args.seed, args.steps, args.warmup)
    tok_s, ns, bpt, frac = dec["tok_s"], dec["ms_per_step"] * 1e6, dec["bytes_per_token"], dec["hbm_fraction"]
    cpu = None
    if not args.no_cpu_baseline:
        # the oracle's MoE path (computeMoeFfn restated, zo_moe_ffn), layer by layer, with the
        # reference's matvec thread policy, on a bounded sample of tokens
        from oracle import zo
        ncpu = os.cpu_count() or 1
        threads = 1 + min(11, ncpu - 1)

        def ptr(lay, name):
            return lay[name][0].ctypes.data if name in lay else None

        descs = [zo.MoeDesc(spec.router_type, ptr(l, "router"), spec.expert_type, ptr(l, "gate_exps"),
                            ptr(l, "up_exps"), ptr(l, "down_exps"), spec.shared_type, ptr(l, "gate_shexp"),
                            ptr(l, "up_shexp"), ptr(l, "down_shexp"), spec.router_type, ptr(l, "gate_inp_shexp"),
                            spec.hidden, spec.expert_ff, spec.shared_ff, spec.n_experts, spec.top_k,
                            spec.gating_func, spec.weights_norm, spec.weights_scale) for l in layers]
        h = synth.normal_row(args.seed, 0, spec.hidden, 0.0, 1.0)
        n, t_cpu = 0, 0.0
        while (t_cpu < args.cpu_seconds or n < 2) and n < 64:
            t1 = time.perf_counter()
            for lay, d in zip(layers, descs):
                normed = zo.rms_norm(h, lay["ffn_norm"][0].view(np.float32), spec.eps)
                out, _, _ = zo.moe_ffn(d, normed, threads=threads)
                h = (h + out).astype(np.float32)
            t_cpu += time.perf_counter() - t1
            n += 1
        cpu = {"value": round(n / t_cpu, 4), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"{n} tokens through the same {spec.n_layers}-layer stack, C restatement of the "
                         f"reference's CPU MoE path, {threads} threads of {ncpu} host cores"}
        log(f"cpu baseline: {cpu['value']} tok/s over {n} tokens ({t_cpu:.1f}s)")
    line = {
        "metric": "MoE FFN stack decode tok/s + % of HBM roofline, 40 x (256 IQ4_XS experts top-8 + Q3_K shared)",
        "value": tok_s, "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ns / 1e6, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{spec.name}, {spec.n_layers} layers, batch 1", "batch": 1, "parallelism": "none"},
        "hbm_fraction": frac, "bytes_per_token": bpt, "cpu_baseline": cpu, "prefill": prefill,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
