"""GPU parity of the whole decode path (session) against the CPU oracle.

Greedy token streams must be identical to the oracle's for the first 64
tokens on the synthetic models; the oracle runs with the binary16 KV cache
semantics of the reference's GPU path (runtime/metal/matvec.metal:246-255) so
both sides round K/V identically.  Logits match within 1e-4 relative L2.
"""
import sys

import numpy as np
import pytest

from oracle import zo
from zhip import hip, synth
from zhip.gguf import F16, F32, Q4_K, Q6_K, Q8_0

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("ptype", [Q4_K, Q6_K])
def test_toy_fixture_text(hip_ctx, ptype):
    # runtime/llama_runtime.zig:237-326: the GPU path must reproduce the CPU text
    say(f"toy fixture {ptype}")
    img = synth.toy_llama_fixture(256, 256, ptype, ptype)
    s = hip.Session(hip_ctx, img)
    toks, _ = s.generate(np.array([3], np.uint32), 6)
    assert synth.toy_detokenize(toks) == " b c! a b c"
    s.close()


SMALL = {
    "llama-q4km": dict(arch="llama", down_q6k_layers=[1]),
    "qwen3-q8": dict(arch="qwen3", qk_norm=True, default_type=Q8_0, attn_v_type=Q8_0, output_type=Q8_0,
                     embd_type=Q8_0, rope_theta=1000000.0),
    "llama-hd128-g4": dict(arch="llama", hidden=512, ffn=1024, n_head=4, n_kv=1, head_dim=128, n_layers=3,
                           context=160),
    "llama-f16": dict(arch="llama", default_type=F16, attn_v_type=F16, output_type=F16, embd_type=F16),
    # an FFN longer than one matvec team (16384): the down rows run as two column windows
    "llama-ffn16640": dict(arch="llama", hidden=256, ffn=16640, n_layers=2, down_q6k_layers=[1]),
    # head_dim 96 (the reference's own attention test shape): the matrix-core kernel with 3 k-steps
    "llama-hd96-g4": dict(arch="llama", hidden=768, ffn=1024, n_head=8, n_kv=2, head_dim=96, n_layers=2,
                          context=160),
}


@pytest.mark.parametrize("name", list(SMALL))
def test_small_model_stream_and_logits(hip_ctx, name):
    say(f"small model {name}")
    spec = synth.small_spec(**SMALL[name])
    img = synth.build(spec, seed=17)
    prompt = synth.prompt_tokens(3, 8, spec.vocab)
    o = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True)
    want, _ = o.generate(prompt, 64)
    s = hip.Session(hip_ctx, img, context=spec.context)
    got, stats = s.generate(prompt, 64)
    assert list(got) == list(want)
    # logits and cache rows of a host-driven prompt replay
    s.reset()
    o2 = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True)
    for t in prompt[:-1]:
        o2.step_no_output(int(t))
        s.step_no_output(int(t))
    nxt = s.step_greedy(int(prompt[-1]))
    ol = o2.step(int(prompt[-1]))
    assert nxt == zo.argmax(ol)
    assert rel_l2(s.logits(), ol) < 1e-4
    # K/V rows of the cache match the oracle's binary16-rounded values
    for layer in range(spec.n_layers):
        k_g, v_g = s.kv(layer, len(prompt) - 1)
        k_o, v_o = o2.kv(layer, len(prompt) - 1)
        assert rel_l2(k_g, k_o) < 1e-3 and rel_l2(v_g, v_o) < 1e-3
    s.close()


def test_long_prompt_logits(hip_ctx):
    # 16 kv heads give 16 attention splits, so 1090 positions fold two 64-position
    # chunks into a split (online softmax inside a split, merge across splits)
    # in the session's fused attention (q/k RoPE + K/V store in-kernel)
    say("long prompt")
    spec = synth.small_spec(hidden=1024, ffn=1024, n_head=16, n_kv=16, head_dim=64, n_layers=2, context=1100)
    img = synth.build(spec, seed=37)
    prompt = synth.prompt_tokens(7, 1090, spec.vocab)
    o = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True)
    s = hip.Session(hip_ctx, img, context=spec.context)
    for t in prompt[:-1]:
        o.step_no_output(int(t))
        s.step_no_output(int(t))
    nxt = s.step_greedy(int(prompt[-1]))
    ol = o.step(int(prompt[-1]))
    assert nxt == zo.argmax(ol)
    assert rel_l2(s.logits(), ol) < 1e-4
    s.close()


def test_per_layer_contract_matches_step(hip_ctx):
    # the gpu.Session contract (begin_token / run_attention_block / run_ffn_block /
    # run_output_argmax, runtime/gpu/session.zig:258-651) gives the step's token
    spec = synth.small_spec()
    img = synth.build(spec, seed=23)
    o = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True)
    s = hip.Session(hip_ctx, img, context=spec.context)
    prompt = synth.prompt_tokens(4, 5, spec.vocab)
    for p, t in enumerate(prompt):
        want_next = o.step_greedy(int(t))
        hidden = zo.dequantize(img.tensors["token_embd.weight"].ttype,
                               img.tensor_view("token_embd.weight")[int(t) * (img.tensors["token_embd.weight"].nbytes // spec.vocab):],
                               1, spec.hidden)[0]
        s.begin_token(hidden)
        for layer in range(spec.n_layers):
            s.run_attention_block(layer, p)
            s.run_ffn_block(layer)
        assert s.run_output_argmax() == want_next
    s.close()


def test_generate_equals_stepwise(hip_ctx):
    spec = synth.small_spec(arch="qwen3", qk_norm=True)
    img = synth.build(spec, seed=29)
    prompt = synth.prompt_tokens(5, 6, spec.vocab)
    s = hip.Session(hip_ctx, img, context=spec.context)
    got, _ = s.generate(prompt, 20)
    s.reset()
    for t in prompt[:-1]:
        s.step_no_output(int(t))
    toks = [s.step_greedy(int(prompt[-1]))]
    for _ in range(19):
        toks.append(s.step_greedy(toks[-1]))
    assert list(got) == toks
    s.close()


def test_context_overflow_is_an_error(hip_ctx):
    spec = synth.small_spec(context=16)
    img = synth.build(spec, seed=31)
    s = hip.Session(hip_ctx, img, context=16)
    with pytest.raises(hip.HipError):
        s.generate(np.arange(3, 13, dtype=np.uint32), 10)
    with pytest.raises(hip.HipError):
        s.step_greedy(spec.vocab + 5)
    s.close()


@pytest.mark.slow
def test_tinyllama_stream_64(hip_ctx):
    # configuration 1: TinyLlama-shaped Q4_K_M, 32 seeded prompt ids, greedy
    say("tinyllama")
    spec = synth.tinyllama_spec(context=256)
    img = synth.build(spec, seed=1)
    prompt = synth.prompt_tokens(1, 32, spec.vocab)
    o = zo.Session(zo.Model(img.buf), context=256, kv_f16=True, threads=16)
    want, _ = o.generate(prompt, 64)
    s = hip.Session(hip_ctx, img, context=256)
    got, _ = s.generate(prompt, 64)
    assert list(got) == list(want)
    s.close()
