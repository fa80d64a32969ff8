"""GPU parity of the output shortlist (the device top-k of the logits that the host
sampler draws from) and of stochastic decoding through it.

- The shortlist kernel against an exact top-k of the same values (numpy: value
  descending, then id ascending -- the tie rule of topk_f32, matvec.metal:1568-1651):
  ids and values bit-exact, across slice boundaries, ties, -inf and vocabulary sizes.
- session_step_shortlist against the session's own logits (the same step) and against
  the oracle's logits for that step.
- A sampled stream (temperature 0.8, top-k 40, top-p 0.9, repeat penalty 1.1): per step
  the session's shortlist through sample_shortlist, against the oracle's full logits
  through sample_logits with the same draws -- the reference's own equivalence of the two
  paths for an exact top-k shortlist (sampling.zig:278-300).
"""
import sys

import numpy as np
import pytest

from oracle import zo
from zhip import hip, synth
from zhip.hip import SamplingOptions

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def exact_topk(x, k):
    order = np.lexsort((np.arange(x.size), -x.astype(np.float64)))
    return order[:k]


@pytest.mark.parametrize("n,k", [(1, 1), (100, 17), (4095, 64), (4096, 64), (4097, 64), (128256, 40),
                                 (152064, 64), (262144, 64)])
def test_shortlist_kernel_matches_an_exact_top_k(hip_ctx, n, k):
    say(f"shortlist n {n} k {k}")
    rng = np.random.default_rng(n + k)
    x = rng.normal(0, 3, n).astype(np.float32)
    if n > 10:
        x[rng.integers(0, n, n // 10)] = -np.inf
        top = float(np.max(x))
        # ties at the top, across slices, and a tie band straddling the k-th place
        for i in rng.integers(0, n, min(12, n)):
            x[i] = top
        band = np.sort(x)[-k] if n >= k else top
        for i in rng.integers(0, n, min(20, n)):
            x[i] = band
    xb = hip_ctx.buffer(x)
    eb = hip_ctx.empty(k * 8)
    hip_ctx.topk(xb, eb, n, k)
    e = eb.read(np.uint32, 2 * k).reshape(k, 2)
    ids = e[:, 0]
    vals = e[:, 1].view(np.float32)
    want = exact_topk(x, k)
    assert ids.tolist() == want.tolist()
    assert np.array_equal(vals.view(np.uint32), x[want].view(np.uint32))


def test_shortlist_rejects_bad_lengths(hip_ctx):
    xb = hip_ctx.buffer(np.zeros(10, np.float32))
    eb = hip_ctx.empty(65 * 8)
    with pytest.raises(hip.HipError):
        hip_ctx.topk(xb, eb, 10, 65)
    with pytest.raises(hip.HipError):
        hip_ctx.topk(xb, eb, 10, 11)


def test_session_step_shortlist(hip_ctx):
    spec = synth.small_spec(vocab=5000)
    img = synth.build(spec, seed=41)
    prompt = synth.prompt_tokens(3, 12, spec.vocab)
    o = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True)
    for t in prompt[:-1]:
        o.step_no_output(int(t))
    want_logits = o.step(int(prompt[-1]))
    s = hip.Session(hip_ctx, img, context=spec.context)
    s.generate(prompt[:-1], 0)
    ids, lg = s.step_shortlist(int(prompt[-1]), 64)
    assert s.position == len(prompt)
    own = s.logits()
    want = exact_topk(own, 64)
    assert ids.tolist() == want.tolist()
    assert np.array_equal(lg.view(np.uint32), own[want].view(np.uint32))
    rel = np.linalg.norm(own.astype(np.float64) - want_logits) / np.linalg.norm(want_logits)
    assert rel < 1e-4
    with pytest.raises(hip.HipError):
        s.step_shortlist(1, 65)
    s.close()


@pytest.mark.parametrize("name,kw", [("llama-q4km", dict(arch="llama")),
                                     ("qwen3-q8", dict(arch="qwen3", qk_norm=True, default_type=8, attn_v_type=8,
                                                       output_type=8, embd_type=8, rope_theta=1000000.0))])
def test_sampled_stream_matches_the_oracle(hip_ctx, name, kw):
    say(f"sampled stream {name}")
    spec = synth.small_spec(**kw)
    img = synth.build(spec, seed=43)
    prompt = [int(t) for t in synth.prompt_tokens(4, 9, spec.vocab)]
    opts = SamplingOptions(temperature=0.8, top_k=40, top_p=0.9, repeat_penalty=1.1)
    k = hip.shortlist_len(opts, spec.vocab)
    draws = np.random.default_rng(2024).random(24)
    # oracle: full logits through sampleToken
    o = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True)
    for t in prompt[:-1]:
        o.step_no_output(t)
    hist, tok, want = list(prompt), prompt[-1], []
    for u in draws:
        tok = hip.sample_logits(o.step(tok), hist, opts, float(u))
        want.append(tok)
        hist.append(tok)
    # device: shortlist per step through sampleShortlist
    s = hip.Session(hip_ctx, img, context=spec.context)
    s.generate(np.array(prompt[:-1], np.uint32), 0)
    hist, tok, got = list(prompt), prompt[-1], []
    for u in draws:
        ids, lg = s.step_shortlist(tok, k)
        tok = hip.sample_shortlist(ids, lg, hist, opts, float(u))
        got.append(tok)
        hist.append(tok)
    s.close()
    assert got == want
