"""Writes tests/golden/headline_streams.json: the CPU oracle's greedy streams on the headline shapes.

The Llama-3.1-8B-shaped Q4_K_M model and the Qwen3-8B-shaped Q8_0 model (config 4),
each built by zhip.synth from seed 1, take an 8-token seeded prompt and decode 64 greedy tokens in the
oracle (oracle/, the C restatement of the reference's CPU decode path) with the binary16 KV semantics of
the reference's GPU path.  The oracle needs minutes for these on host cores, so its streams are computed
once here and the GPU tests compare the HIP session with them; each entry carries a digest of the model
image it was made from, so a change of the synthetic weights is caught instead of compared against.

Run from the repository root:  python3 tests/golden/make_headline_streams.py
"""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
for p in (REPO, os.path.join(REPO, "ziggy-llm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import zo  # noqa: E402
from zhip import synth  # noqa: E402

OUT = os.path.join(HERE, "headline_streams.json")
PROMPT_LEN, STEPS, SEED, CONTEXT = 8, 64, 1, 96


def image_digest(buf) -> str:
    """blake2b over the image size and a 4 KiB sample of every MiB (the whole image would take long)."""
    h = hashlib.blake2b(digest_size=16)
    h.update(str(buf.nbytes).encode())
    mv = memoryview(buf)
    for off in range(0, buf.nbytes, 1 << 20):
        h.update(mv[off:off + 4096])
    h.update(mv[max(0, buf.nbytes - 4096):])
    return h.hexdigest()


def stream(spec_fn):
    spec = spec_fn(context=CONTEXT)
    img = synth.build(spec, seed=SEED)
    prompt = synth.prompt_tokens(SEED, PROMPT_LEN, spec.vocab)
    o = zo.Session(zo.Model(img.buf), context=CONTEXT, kv_f16=True, threads=os.cpu_count() or 1)
    toks, _ = o.generate(prompt, STEPS)
    return {"spec": spec.name, "seed": SEED, "context": CONTEXT, "prompt": [int(t) for t in prompt],
            "tokens": [int(t) for t in toks], "image_bytes": int(img.buf.nbytes), "image_digest": image_digest(img.buf),
            "kv": "binary16"}


def main():
    out = {"llama8b": stream(synth.llama8b_spec), "qwen3_8b": stream(synth.qwen3_8b_spec)}
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
