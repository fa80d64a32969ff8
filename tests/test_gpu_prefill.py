"""Batched prompt prefill on the matrix cores against the oracle's token-by-token prompt.

The reference feeds a prompt one token at a time (runPrompt, model/loader.zig:1016-1036); the session
runs every prompt token but the last in batched passes of up to 256 tokens (exact-code GEMMs, multi-query
causal attention over the rows the pass itself stores), then the last one through the decode step.  The
logits after the prompt must be within 1e-4 relative L2 of the oracle's, and the next 64 greedy tokens
equal its stream.  Prompts of 300 tokens take two passes, the last one ragged; the models cover query
heads per kv head 1, 2 and 8, head sizes 64 and 128, per-head QK norm and Q4_K_M / Q8_0 weights.
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
    "llama-q4km-g2": dict(arch="llama", down_q6k_layers=[1], context=512),
    "llama-g1-hd64": dict(arch="llama", n_head=4, n_kv=4, context=512),
    "qwen3-q8-g8-hd128": dict(arch="qwen3", qk_norm=True, hidden=512, ffn=1024, n_head=8, n_kv=1, head_dim=128,
                              default_type=Q8_0, attn_v_type=Q8_0, output_type=Q8_0, embd_type=Q8_0, context=512,
                              rope_theta=1000000.0),
    "llama-hd96-g4": dict(arch="llama", hidden=768, ffn=1024, n_head=8, n_kv=2, head_dim=96, context=512),
    # Q8_0 with odd chunk counts (768 and 1280 values): the two-tile product's one-chunk stages end on a
    # chunk whose pair partner is past the range
    "llama-q8-odd-chunks": dict(arch="llama", hidden=768, ffn=1280, n_head=6, n_kv=2, head_dim=128,
                                default_type=Q8_0, attn_v_type=Q8_0, output_type=Q8_0, embd_type=Q8_0, context=512),
}


@pytest.mark.parametrize("name", list(MODELS))
# 18: one pass of 17 rows (the two-token-tile products with a second tile of one row); 65 and 300: full
# and partial tiles over one or two passes
@pytest.mark.parametrize("plen", [2, 18, 65, 300])
def test_batched_prefill_matches_the_token_by_token_prompt(hip_ctx, name, plen):
    say(f"prefill {name} prompt {plen}")
    spec = synth.small_spec(**MODELS[name])
    img = synth.build(spec, seed=61)
    prompt = synth.prompt_tokens(62, plen, spec.vocab)
    o = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True)
    for t in prompt[:-1]:
        o.step_no_output(int(t))
    want_logits = o.step(int(prompt[-1]))
    want = [zo.argmax(want_logits)]
    for _ in range(63):
        want.append(o.step_greedy(want[-1]))
    s = hip.Session(hip_ctx, img, context=spec.context)
    got, st = s.generate(prompt, 64)
    assert st.prompt_ns > 0
    assert [int(t) for t in got] == want
    # logits after the prompt: a second session, prompt only (the last token runs the output head)
    s2 = hip.Session(hip_ctx, img, context=spec.context)
    _, st2 = s2.generate(prompt, 0)
    assert st2.next_token == want[0]
    assert rel_l2(s2.logits(), want_logits) < 1e-4
    # the cache rows the passes wrote
    for pos in (0, plen // 2, plen - 2):
        if pos < 0:
            continue
        for layer in range(spec.n_layers):
            k_g, v_g = s2.kv(layer, pos)
            k_o, v_o = o.kv(layer, pos)
            assert rel_l2(k_g, k_o) < 1e-3 and rel_l2(v_g, v_o) < 1e-3
    s.close()
    s2.close()
