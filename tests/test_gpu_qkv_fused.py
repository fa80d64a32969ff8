"""The decode step's q/k/v projection and attention in one launch
(launch_qkv_attention: the projection workgroups store q, k and v with
device-scope stores; the attention workgroups of the same launch issue their K
loads first and read their head's q, k and v as they land) against the two
launches of ZIGGY_HIP_QKV_FUSE=0, and against the CPU oracle.

The two paths run the same arithmetic on the same values, so the greedy tokens
and the logits must be the same bits.  The q/k/v words rotate through 2, 3 and
4 sets (2, 3 and 7 layers); repeated generate calls replay the step graph,
which must leave the sets re-armed.  After a 6-token prompt each step's
attention is one split per kv head; after a 300-token prompt it is two, merged
by polling inside the fused launch.  ZIGGY_HIP_ATTN_V_NOW=1 forces the
variant long contexts use (the V tiles issued right after the q/k/v wait),
which must give the same bits.  The shapes are the smallest the fused
launch serves: hidden 1024 (teams of 64 lanes), head_dim 128 with four query
heads per kv head (Q4_K q/k with Q6_K v, or Q8_0 throughout), and head_dim 64
with eight (the TinyLlama shape's attention).
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


BASE = dict(arch="llama", hidden=1024, ffn=2048, n_head=8, n_kv=2, head_dim=128, vocab=512, context=160)
CASES = {
    "q4km-2-layers": dict(BASE, n_layers=2, down_q6k_layers=[1]),
    "q4km-3-layers": dict(BASE, n_layers=3, down_q6k_layers=[0, 2]),
    "q8-7-layers": dict(BASE, arch="qwen3", n_layers=7, qk_norm=True, default_type=Q8_0, attn_v_type=Q8_0,
                        output_type=Q8_0, embd_type=Q8_0, rope_theta=1000000.0),
    # head_dim 64 with eight query heads per kv head (the TinyLlama shape's attention)
    "q4km-hd64-g8": dict(BASE, n_layers=3, n_head=16, n_kv=2, head_dim=64, down_q6k_layers=[1]),
}


def run(hip_ctx, img, spec, prompt, steps):
    s = hip.Session(hip_ctx, img, context=spec.context)
    toks, _ = s.generate(prompt, steps)
    logits = s.logits()
    # a second call replays the step graph over the same prompt
    s.reset()
    toks2, _ = s.generate(prompt, steps)
    logits2 = s.logits()
    s.close()
    assert list(toks) == list(toks2) and np.array_equal(logits, logits2)
    return toks, logits


@pytest.mark.parametrize("name,prompt_len,v_now",
                         [(n, 6, "") for n in CASES] +
                         [("q4km-3-layers", 300, ""), ("q8-7-layers", 300, ""), ("q4km-hd64-g8", 300, "")] +
                         [("q8-7-layers", 6, "1"), ("q4km-3-layers", 300, "1"), ("q4km-hd64-g8", 300, "1")])
def test_fused_qkv_attention_equals_two_launches_and_oracle(hip_ctx, monkeypatch, name, prompt_len, v_now):
    # a 6-token prompt keeps every step's attention in one split; after 300
    # tokens each kv head has two splits and the launch merges them (polled)
    spec = synth.small_spec(**dict(CASES[name], context=prompt_len + 40))
    say(f"fused q/k/v + attention {name}: {spec.n_layers} layers, hidden {spec.hidden}, prompt {prompt_len}, "
        f"v_now {v_now or 'auto'}")
    if v_now:
        monkeypatch.setenv("ZIGGY_HIP_ATTN_V_NOW", v_now)
    img = synth.build(spec, seed=41)
    prompt = synth.prompt_tokens(7, prompt_len, spec.vocab)
    steps = 24
    monkeypatch.setenv("ZIGGY_HIP_QKV_FUSE", "0")
    want, want_logits = run(hip_ctx, img, spec, prompt, steps)
    monkeypatch.delenv("ZIGGY_HIP_QKV_FUSE")
    got, got_logits = run(hip_ctx, img, spec, prompt, steps)
    assert list(got) == list(want)
    assert np.array_equal(got_logits, want_logits)
    o = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True)
    ref, _ = o.generate(prompt, steps)
    assert list(got) == list(ref)


def test_fused_variant_switch_rebuilds_the_step_graph(hip_ctx, monkeypatch):
    # the session picks the fused launch's variant when generate builds the
    # step graph; asking for the other one on the same session rebuilds it
    spec = synth.small_spec(**dict(CASES["q4km-3-layers"], context=340))
    img = synth.build(spec, seed=53)
    prompt = synth.prompt_tokens(13, 300, spec.vocab)
    steps = 16
    monkeypatch.setenv("ZIGGY_HIP_ATTN_V_NOW", "0")
    s = hip.Session(hip_ctx, img, context=spec.context)
    want, _ = s.generate(prompt, steps)
    want_logits = s.logits()
    for flag in ("1", "0", "1"):
        monkeypatch.setenv("ZIGGY_HIP_ATTN_V_NOW", flag)
        s.reset()
        got, _ = s.generate(prompt, steps)
        assert list(got) == list(want), flag
        assert np.array_equal(s.logits(), want_logits), flag
    s.close()


def test_fused_qkv_attention_profile_records(hip_ctx):
    # the profiled decode runs the step's launches: four per layer, q/k/v and attention one record
    spec = synth.small_spec(**CASES["q4km-3-layers"])
    img = synth.build(spec, seed=43)
    prompt = synth.prompt_tokens(9, 5, spec.vocab)
    steps = 4
    s = hip.Session(hip_ctx, img, context=spec.context)
    want, _ = s.generate(prompt, steps + 1)
    s.reset()
    for t in prompt[:-1]:
        s.step_no_output(int(t))
    toks, recs = s.profile_decode(int(prompt[-1]), steps)
    s.close()
    assert list(toks) == [int(t) for t in want[:steps]]
    L = spec.n_layers
    assert len(recs) == (4 * L + 7) * steps
    K = hip.PROFILE_KINDS
    per = recs.reshape(steps, 4 * L + 7)
    for t in range(steps):
        body = np.array(list(per[t]["kind"][2:2 + 4 * L])).reshape(L, 4)
        assert (body == [K["attention"], K["projections"], K["projections"], K["projections"]]).all()
        att = per[t][2]
        assert att["rows"] == spec.n_head and att["extra"] == spec.n_kv


def test_time_kernel_between_steps_keeps_the_stream(hip_ctx, monkeypatch):
    # timing each launch of the step, the fused one included (whole passes
    # over the layers), between greedy steps leaves the stream as it was
    spec = synth.small_spec(**dict(CASES["q4km-3-layers"], context=80))
    img = synth.build(spec, seed=47)
    prompt = synth.prompt_tokens(11, 5, spec.vocab)
    s = hip.Session(hip_ctx, img, context=spec.context)
    want, _ = s.generate(prompt, 12)
    s.reset()
    for t in prompt[:-1]:
        s.step_no_output(int(t))
    got, tok = [], int(prompt[-1])
    for i in range(12):
        tok = s.step_greedy(tok)
        got.append(tok)
        if i == 5:
            sizes = {}
            for name in ("qkv", "attention", "qkv_attention", "o_proj", "gate_up", "down", "output"):
                ns, nb = s.time_kernel(name, 5)
                assert ns > 0 and nb > 0
                sizes[name] = nb
            assert sizes["qkv_attention"] == sizes["qkv"] + sizes["attention"]
    assert got == [int(t) for t in want[:12]]
    s.close()
    # a session that keeps q/k/v and the attention apart has no fused launch to time
    monkeypatch.setenv("ZIGGY_HIP_QKV_FUSE", "0")
    s = hip.Session(hip_ctx, img, context=spec.context)
    with pytest.raises(hip.HipError):
        s.time_kernel("qkv_attention", 5)
    s.close()
