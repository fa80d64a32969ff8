"""Writes tests/golden/headline_streams.json (and headline_long_logits.npz): the CPU oracle's greedy
streams on the headline shapes.

The Llama-3.1-8B-shaped Q4_K_M model (benchmark configuration 3) and the Qwen3-8B-shaped Q8_0 model (config 4),
each built by zhip.synth from seed 1, get three oracle runs (oracle/, the C restatement of the reference's
CPU decode path, fed token by token as runPrompt does, model/loader.zig:1016-1036):
  * `tokens`: an 8-token seeded prompt and 64 greedy tokens with the binary16 KV semantics of the
    reference's GPU path (Metal store_kv_half, runtime/metal/matvec.metal:246-255);
  * `f32_kv`: the same prompt and 64 tokens with an f32 KV cache, the reference CPU path proper
    (model/loader.zig:950-951), and the first step where it leaves the binary16 stream (null: none);
  * `long`: a 320-token seeded prompt (binary16 KV), the logits after it (in the .npz) and the next 64
    greedy tokens.  The HIP session runs such a prompt in batched passes of up to 256 rows, so this
    pins its two-token-tile GEMMs over full reductions (K = 4096 and 14336 / 12288).  The entry also
    records the oracle's own sensitivity there: the relative L2 change of its logits when one weight of
    layer 0's attention norm moves by one ulp.
The oracle needs minutes for these on host cores, so they are computed once here and the GPU tests
compare the HIP session with them; each entry carries a digest of the model image it was made from, so a
change of the synthetic weights is caught instead of compared against.  Entries already present are
kept (pass --force to recompute everything).

Run from the repository root:  python3 tests/golden/make_headline_streams.py [--force]
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
for p in (REPO, os.path.join(REPO, "ziggy-llm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import zo  # noqa: E402
from zhip import synth  # noqa: E402

OUT = os.path.join(HERE, "headline_streams.json")
LOGITS = os.path.join(HERE, "headline_long_logits.npz")
PROMPT_LEN, STEPS, SEED, CONTEXT = 8, 64, 1, 96
LONG_SEED, LONG_LEN, LONG_CONTEXT = 2, 320, 416
THREADS = os.cpu_count() or 1


def image_digest(buf) -> str:
    """blake2b over the image size and a 4 KiB sample of every MiB (the whole image would take long)."""
    h = hashlib.blake2b(digest_size=16)
    h.update(str(buf.nbytes).encode())
    mv = memoryview(buf)
    for off in range(0, buf.nbytes, 1 << 20):
        h.update(mv[off:off + 4096])
    h.update(mv[max(0, buf.nbytes - 4096):])
    return h.hexdigest()


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def say(*a):
    print(*a, flush=True)


def prompt_logits(zm, prompt, context):
    o = zo.Session(zm, context=context, kv_f16=True, threads=THREADS)
    for t in prompt[:-1]:
        o.step_no_output(int(t))
    logits = o.step(int(prompt[-1]))
    return o, logits


def first_divergence(a, b):
    for i, (x, y) in enumerate(zip(a, b)):
        if int(x) != int(y):
            return i
    return None


def model_entries(key, spec_fn, have, force, logits_out):
    spec = spec_fn(context=CONTEXT)
    say(f"{key}: building {spec.name}")
    img = synth.build(spec, seed=SEED)
    digest = image_digest(img.buf)
    if have is not None and have.get("image_digest") != digest:
        raise SystemExit(f"{key}: the synthetic weights changed; rerun with --force")
    e = dict(have or {}) if not force else {}
    prompt = synth.prompt_tokens(SEED, PROMPT_LEN, spec.vocab)
    zm = zo.Model(img.buf)
    e.update({"spec": spec.name, "seed": SEED, "context": CONTEXT, "prompt": [int(t) for t in prompt],
              "image_bytes": int(img.buf.nbytes), "image_digest": digest, "kv": "binary16"})
    if "tokens" not in e:
        say(f"{key}: binary16-KV stream")
        o = zo.Session(zm, context=CONTEXT, kv_f16=True, threads=THREADS)
        toks, _ = o.generate(prompt, STEPS)
        o.close()
        e["tokens"] = [int(t) for t in toks]
    if "f32_kv" not in e:
        say(f"{key}: f32-KV stream")
        o = zo.Session(zm, context=CONTEXT, kv_f16=False, threads=THREADS)
        toks, _ = o.generate(prompt, STEPS)
        o.close()
        toks = [int(t) for t in toks]
        e["f32_kv"] = {"tokens": toks, "first_divergence": first_divergence(toks, e["tokens"])}
    if "long" not in e or key not in logits_out:
        say(f"{key}: {LONG_LEN}-token prompt")
        lp = synth.prompt_tokens(LONG_SEED, LONG_LEN, spec.vocab)
        o, logits = prompt_logits(zm, lp, LONG_CONTEXT)
        want = [zo.argmax(logits)]
        for _ in range(STEPS - 1):
            want.append(o.step_greedy(want[-1]))
        o.close()
        say(f"{key}: one-ulp sensitivity")
        w = img.tensor_view("blk.0.attn_norm.weight").view(np.float32)
        keep = w[5]
        w[5] = np.nextafter(keep, np.float32(2))
        o2, logits_ulp = prompt_logits(zm, lp, LONG_CONTEXT)
        o2.close()
        w[5] = keep
        e["long"] = {"prompt_seed": LONG_SEED, "prompt_len": LONG_LEN, "context": LONG_CONTEXT,
                     "tokens": [int(t) for t in want], "logits_key": key,
                     "oracle_one_ulp_rel_l2": rel_l2(logits_ulp, logits)}
        logits_out[key] = logits.astype(np.float32)
    zm.close()
    return e


def main():
    force = "--force" in sys.argv[1:]
    have = {} if force or not os.path.exists(OUT) else json.load(open(OUT))
    logits = {} if force or not os.path.exists(LOGITS) else dict(np.load(LOGITS))
    out = {}
    for key, fn in (("llama8b", synth.llama8b_spec), ("qwen3_8b", synth.qwen3_8b_spec)):
        out[key] = model_entries(key, fn, have.get(key), force, logits)
        with open(OUT, "w") as f:  # after each model: a long run keeps what it finished
            json.dump({**have, **out}, f, indent=1)
            f.write("\n")
        np.savez_compressed(LOGITS, **logits)
    say(f"wrote {OUT} and {LOGITS}")


if __name__ == "__main__":
    main()
