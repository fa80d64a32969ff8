"""Distance of the HIP path (binary16 KV cache, the reference GPU path's store_kv_half) from the reference
CPU path proper, whose KV cache is f32 (model/loader.zig:950-951, restated by the oracle with kv_f16=False).

Free-running: the HIP greedy stream must equal the f32 oracle's for 64 tokens (the reference CPU path's
own stream); the first diverging step is printed before the assertion.  Teacher-forced: both sides are fed
the same tokens (the f32 oracle's stream), so the logits of every step are compared at the same inputs:
within 2e-3 relative L2.  binary16 K/V carries up to 2^-11 relative rounding into every score and value;
the measured worst case is ~3e-4 on the small models and ~1.03e-3 on the TinyLlama shape (22 layers).
"""
import sys

import numpy as np
import pytest

from oracle import zo
from zhip import hip, synth
from zhip.gguf import Q8_0

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


MODELS = {
    "llama-q4km": (lambda: synth.small_spec(arch="llama", down_q6k_layers=[1]), 17, 8),
    "qwen3-q8": (lambda: synth.small_spec(arch="qwen3", qk_norm=True, default_type=Q8_0, attn_v_type=Q8_0,
                                          output_type=Q8_0, embd_type=Q8_0, rope_theta=1000000.0), 17, 8),
    "llama-hd128-g4": (lambda: synth.small_spec(arch="llama", hidden=512, ffn=1024, n_head=4, n_kv=1,
                                                head_dim=128, n_layers=3, context=160), 17, 8),
    "tinyllama": (lambda: synth.tinyllama_spec(context=128), 1, 32),
}


@pytest.mark.parametrize("name", list(MODELS))
def test_distance_from_the_f32_kv_cpu_path(hip_ctx, name):
    spec_fn, seed, plen = MODELS[name]
    spec = spec_fn()
    say(f"f32-KV distance {name}")
    img = synth.build(spec, seed=seed)
    prompt = synth.prompt_tokens(seed, plen, spec.vocab)
    steps = 64
    model = zo.Model(img.buf)
    want, _ = zo.Session(model, context=spec.context, kv_f16=False, threads=16).generate(prompt, steps)
    s = hip.Session(hip_ctx, img, context=spec.context)
    got, _ = s.generate(prompt, steps)
    diverge = next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), None)
    say(f"{name}: first divergence from the f32-KV stream: {diverge if diverge is not None else 'none in 64'}")
    assert diverge is None, f"{name}: the HIP stream leaves the f32-KV CPU stream at step {diverge}"
    # teacher-forced logits over the prompt and the f32 stream
    s.reset()
    o = zo.Session(model, context=spec.context, kv_f16=False, threads=16)
    feed = [int(t) for t in prompt] + [int(t) for t in want[:-1]]
    worst = 0.0
    for i, t in enumerate(feed):
        if i < len(prompt) - 1:
            s.step_no_output(t)
            o.step_no_output(t)
            continue
        s.step_greedy(t)
        ol = o.step(t)
        d = rel_l2(s.logits(), ol)
        worst = max(worst, d)
        assert d < 2e-3, (name, i, d)
    say(f"{name}: worst logits rel L2 against the f32-KV path over {len(feed) - len(prompt) + 1} steps: {worst:.2e}")
    s.close()
