"""Prompt-prefix KV reuse across turns (ziggy_hip_session_prefill_cached) against the reference's golden
and the CPU oracle.

The reference keeps one session across turns of its resident runtime and reuses the cached prompt prefix
(generateLoadedStreamingCached, model/loader.zig:2281-2336): its golden (runtime/resident_runtime.zig:
454-490) runs "a" for one token (" b"), then "a b" for two, which must reuse cached rows and produce
" c!".  The turn loop follows the reference's greedy loop (:2360-2446): each emitted token is stepped, so
after a turn the session holds the prompt and every emitted token.
"""
import sys

import numpy as np
import pytest

from oracle import zo
from zhip import hip, synth
from zhip.gguf import Q4_K, Q6_K

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def turn(s, prompt, max_tokens):
    """One resident-runtime turn: cached prefill, then emit / step max_tokens greedy tokens."""
    reused, nxt = s.prefill_cached(prompt)
    emitted = [nxt]
    if max_tokens > 1:
        out, st = s.generate(np.array([nxt], np.uint32), max_tokens - 1)
        emitted += [int(t) for t in out]
        last = st.next_token
    else:
        _, st = s.generate(np.array([nxt], np.uint32), 0)
        last = st.next_token
    return reused, emitted, last


@pytest.mark.parametrize("ptype", [Q4_K, Q6_K])
def test_prefix_reuse_golden_text(hip_ctx, ptype):
    # tokens of the toy vocabulary: 3 = "▁a", 4 = "▁b" ("a b" encodes to [3, 4], no BOS)
    say(f"prefix reuse golden {ptype}")
    img = synth.toy_llama_fixture(256, 256, ptype, ptype)
    s = hip.Session(hip_ctx, img)
    reused, emitted, _ = turn(s, [3], 1)
    assert reused == 0 and synth.toy_detokenize(emitted) == " b"
    reused, emitted, _ = turn(s, [3, 4], 2)
    assert reused > 0 and synth.toy_detokenize(emitted) == " c!"
    s.close()


def test_prefix_reuse_continues_the_oracle_stream(hip_ctx):
    # turn 2's prompt extends everything turn 1 left in the cache; its continuation must be the
    # oracle's greedy stream for that prompt run from an empty cache
    say("prefix reuse vs oracle")
    spec = synth.small_spec(arch="llama", down_q6k_layers=[1])
    img = synth.build(spec, seed=53)
    p1 = [int(t) for t in synth.prompt_tokens(21, 10, spec.vocab)]
    s = hip.Session(hip_ctx, img, context=spec.context)
    reused, emitted, _ = turn(s, p1, 5)
    assert reused == 0
    want1, _ = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True).generate(np.array(p1, np.uint32), 5)
    assert emitted == [int(t) for t in want1]
    p2 = p1 + emitted + [int(t) for t in synth.prompt_tokens(22, 3, spec.vocab)]
    reused, emitted2, _ = turn(s, p2, 12)
    assert reused == len(p1) + len(emitted)
    want2, _ = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True).generate(np.array(p2, np.uint32), 12)
    assert emitted2 == [int(t) for t in want2]
    s.close()
