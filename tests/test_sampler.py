"""CPU checks of the host sampler (ziggy_hip_sample_shortlist / _sample_logits), the
reference's sampleShortlist / sampleToken policy (sampling.zig:11-110) that runs on the
host over the device shortlist.

Pins, none of which restates the sampler's code:
- the reference's own tests (sampling.zig:209-306), with this build's draws in place of
  DefaultPrng's (the sampler takes the uniform value random.float(f64) would give);
- inverse-CDF sampling as mathematics fixes it: with weights w_i = exp((l_i - max) / T),
  u lands on the first candidate whose running share of the total reaches u, so a grid of
  u values must reproduce the cumulative softmax computed independently by numpy, and many
  draws must reproduce the probabilities;
- top-p and min-p as set definitions (smallest most-probable prefix reaching p; weights at
  least min_p of the largest).
"""
import numpy as np
import pytest

from zhip import hip
from zhip.hip import SamplingOptions


def draws(seed, n=32):
    return np.random.default_rng(seed).random(n)


def cdf(logits, t):
    # the options carry binary32: the temperature the sampler divides by is float32(t)
    l = np.asarray(logits, np.float64)
    w = np.exp((l - l.max()) / float(np.float32(t)))
    return np.cumsum(w) / w.sum()


def test_non_positive_temperature_is_argmax():
    # sampling.zig:226-231
    assert hip.sample_logits([-1.0, 3.0, 0.5], [], SamplingOptions(temperature=0.0), 0.5) == 1


def test_seeded_draws_repeat():
    # sampling.zig:209-224: the same draw gives the same token; any draw a valid one
    logits = [2.0, 1.8, 1.7, 1.6]
    o = SamplingOptions(temperature=0.8)
    for u in draws(42):
        a, b = hip.sample_logits(logits, [], o, u), hip.sample_logits(logits, [], o, u)
        assert a == b and 0 <= a < len(logits)


def test_top_k_restricts_the_set():
    # sampling.zig:233-242
    o = SamplingOptions(temperature=1.0, top_k=2)
    assert {hip.sample_logits([10.0, 9.0, 1.0, 0.5], [], o, u) for u in draws(123)} <= {0, 1}


def test_top_p_trims_the_tail():
    # sampling.zig:244-253
    o = SamplingOptions(temperature=1.0, top_p=0.9)
    assert {hip.sample_logits([8.0, 7.5, 1.0, 0.2], [], o, u) for u in draws(321)} <= {0, 1}


def test_repeat_penalty_demotes():
    # sampling.zig:255-264 asserts that 32 draws of its own generator never give token 2,
    # which holds for those draws only (token 2 keeps ~1.3% of the mass).  Stated as the
    # demotion it checks: token 0 (recent) falls from ~52% to its penalised share, 4.0 / 1.5
    logits = [4.0, 3.9, 1.0]
    grid = (np.arange(4000) + 0.5) / 4000
    with_p = np.array([hip.sample_logits(logits, [0], SamplingOptions(temperature=0.7, repeat_penalty=1.5), u)
                       for u in grid])
    without = np.array([hip.sample_logits(logits, [0], SamplingOptions(temperature=0.7), u) for u in grid])
    want = np.diff(np.concatenate([[0.0], cdf([4.0 / 1.5, 3.9, 1.0], 0.7)]))
    assert abs((with_p == 0).mean() - want[0]) < 1e-3 and (without == 0).mean() > 0.5


def test_min_p_trims_the_tail():
    # sampling.zig:266-275
    o = SamplingOptions(temperature=1.0, min_p=0.5)
    assert {hip.sample_logits([6.0, 5.5, 0.5, 0.2], [], o, u) for u in draws(17)} <= {0, 1}


def test_shortlist_equals_full_top_k():
    # sampling.zig:278-300: sampling the exact top-k shortlist = sampling the full logits with that top-k
    logits = [4.0, 3.5, 2.0, 1.0, -1.0]
    o = SamplingOptions(temperature=0.9, top_k=3, top_p=0.85, min_p=0.0, repeat_penalty=1.2)
    for u in draws(1234, 256):
        assert hip.sample_logits(logits, [1], o, u) == hip.sample_shortlist([0, 1, 2], [4.0, 3.5, 2.0], [1], o, u)


def test_shortlist_len():
    # sampling.zig:302-306
    assert hip.shortlist_len(SamplingOptions(temperature=0.7), 32000) == 64
    assert hip.shortlist_len(SamplingOptions(temperature=0.7, top_k=12), 32000) == 12
    assert hip.shortlist_len(SamplingOptions(temperature=0.0), 32000) == 0
    assert hip.shortlist_len(SamplingOptions(temperature=0.7, top_k=100), 50) == 50


@pytest.mark.parametrize("t", [0.5, 1.0, 1.7])
def test_inverse_cdf(t):
    rng = np.random.default_rng(7)
    logits = rng.normal(0, 2, 40).astype(np.float32)
    c = cdf(logits, t)
    o = SamplingOptions(temperature=t)
    for u in np.concatenate([rng.random(200), c[:-1] - 1e-9, c[:-1] + 1e-9]):
        u = float(min(max(u, 0.0), 1.0 - 1e-12))
        want = int(np.searchsorted(c, u, side="left"))
        assert hip.sample_logits(logits, [], o, u) == want, u


def test_draw_frequencies_follow_the_softmax():
    logits = np.array([1.0, 0.5, 0.0, -0.5, -3.0], np.float32)
    o = SamplingOptions(temperature=0.8)
    n = 20000
    got = np.bincount([hip.sample_logits(logits, [], o, u) for u in draws(99, n)], minlength=5) / n
    p = np.exp((logits - logits.max()) / 0.8)
    p /= p.sum()
    assert np.abs(got - p).max() < 0.015


def test_top_p_and_min_p_as_sets():
    rng = np.random.default_rng(11)
    logits = rng.normal(0, 1.5, 30).astype(np.float32)
    p = np.exp(logits.astype(np.float64) - logits.max())
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    # top-p: the smallest most-probable prefix whose share reaches 0.7
    keep = order[: int(np.searchsorted(np.cumsum(p[order]), 0.7, side="left")) + 1]
    o = SamplingOptions(temperature=1.0, top_p=0.7)
    assert {hip.sample_logits(logits, [], o, u) for u in draws(3, 400)} <= set(keep.tolist())
    # min-p: weights at least 0.3 of the largest
    keep = np.nonzero(p >= 0.3 * p.max())[0]
    o = SamplingOptions(temperature=1.0, min_p=0.3)
    assert {hip.sample_logits(logits, [], o, u) for u in draws(4, 400)} <= set(keep.tolist())


def test_repeat_penalty_direction():
    # a repeated positive logit is divided by the penalty, a repeated negative one multiplied:
    # with penalty 2, logits [1.0, 0.6] and token 0 recent, token 1 (0.6 > 0.5) is the argmax of
    # the adjusted set; with [-1.0, -1.9] and token 0 recent, token 1 (-1.9 > -2.0) leads
    o = SamplingOptions(temperature=1e-6, repeat_penalty=2.0)
    assert hip.sample_shortlist([0, 1], [1.0, 0.6], [0], o, 0.5) == 1
    assert hip.sample_shortlist([0, 1], [-1.0, -1.9], [0], o, 0.5) == 1


def test_sampler_rejects_bad_draws():
    with pytest.raises(hip.HipError):
        hip.sample_logits([1.0, 2.0], [], SamplingOptions(temperature=1.0), 1.0)
    with pytest.raises(hip.HipError):
        hip.sample_shortlist([0], [1.0], [], SamplingOptions(temperature=1.0), -0.1)
