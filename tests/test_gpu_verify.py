"""GPU parity of the batched speculative verify (ziggy_hip_session_verify).

The verify pass runs the current token and its drafts through the model in
one batch on the matrix cores.  Its predictions must be the oracle's greedy
stream (the reference's verifyDraftTokensSequential is numerically a plain
greedy stream, model/loader.zig:1131-1151), the emitted count must follow
the reference's acceptance rule, and decoding after the pass (over the K/V
rows the pass wrote) must continue the oracle's stream.
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


SMALL = {
    "llama-q4km": dict(arch="llama", down_q6k_layers=[1]),
    "qwen3-q8": dict(arch="qwen3", qk_norm=True, default_type=Q8_0, attn_v_type=Q8_0, output_type=Q8_0,
                     embd_type=Q8_0, rope_theta=1000000.0),
    "llama-hd128-g4": dict(arch="llama", hidden=512, ffn=1024, n_head=4, n_kv=1, head_dim=128, n_layers=3,
                           context=160),
}


@pytest.mark.parametrize("name", list(SMALL))
def test_verify_accepts_the_greedy_stream(hip_ctx, name):
    say(f"verify {name}")
    spec = synth.small_spec(**SMALL[name])
    img = synth.build(spec, seed=23)
    prompt = synth.prompt_tokens(5, 9, spec.vocab)
    want, _ = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True).generate(prompt, 40)
    want = [int(t) for t in want]
    s = hip.Session(hip_ctx, img, context=spec.context)
    _, st = s.generate(prompt, 0)
    assert st.next_token == want[0]
    # eight drafts, all right: nine predictions emitted (the last one the bonus)
    pred, n = s.verify(want[0], want[1:9])
    assert n == 9 and list(pred) == want[1:10]
    assert s.position == len(prompt) + 9
    # decoding continues the stream over the K/V rows the pass wrote
    got, _ = s.generate(np.array([want[9]], np.uint32), 8)
    assert [int(t) for t in got] == want[10:18]
    s.close()


LONG = {
    # query heads per kv head 1, 4 and 8: 8, 2 and 1 queries per attention workgroup
    "g1-hd64": dict(arch="llama", n_head=4, n_kv=4, context=512),
    "g4-hd128-qknorm": dict(arch="qwen3", qk_norm=True, hidden=512, ffn=1024, n_head=4, n_kv=1, head_dim=128,
                            default_type=Q8_0, attn_v_type=Q8_0, output_type=Q8_0, embd_type=Q8_0, context=512,
                            rope_theta=1000000.0),
    "g8-hd64": dict(arch="llama", hidden=512, n_head=8, n_kv=1, context=512),
}


@pytest.mark.parametrize("name", list(LONG))
def test_verify_over_a_long_context(hip_ctx, name):
    # 300 positions: several attention splits per query group, so the
    # multi-query launch merges partials; the rows it stores feed the decode after
    say(f"verify long {name}")
    spec = synth.small_spec(**LONG[name])
    img = synth.build(spec, seed=37)
    prompt = synth.prompt_tokens(9, 300, spec.vocab)
    want, _ = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True).generate(prompt, 30)
    want = [int(t) for t in want]
    s = hip.Session(hip_ctx, img, context=spec.context)
    _, st = s.generate(prompt, 0)
    assert st.next_token == want[0]
    pred, n = s.verify(want[0], want[1:12])
    assert n == 12 and list(pred) == want[1:13]
    got, _ = s.generate(np.array([want[12]], np.uint32), 8)
    assert [int(t) for t in got] == want[13:21]
    s.close()


MANY_SPLITS = {
    # 1500 positions, up to 32 splits per query group: more splits than one
    # round of the multi-query merge folds (16), so it folds in two rounds
    "g1-hd64": dict(arch="llama", n_head=4, n_kv=4, context=2048),
    "g8-hd64": dict(arch="llama", hidden=512, n_head=8, n_kv=1, context=2048),
}


@pytest.mark.parametrize("name", list(MANY_SPLITS))
def test_verify_merges_more_splits_than_one_round(hip_ctx, name):
    say(f"verify many splits {name}")
    spec = synth.small_spec(**MANY_SPLITS[name])
    img = synth.build(spec, seed=41)
    prompt = synth.prompt_tokens(11, 1500, spec.vocab)
    want, _ = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True).generate(prompt, 16)
    want = [int(t) for t in want]
    s = hip.Session(hip_ctx, img, context=spec.context)
    _, st = s.generate(prompt, 0)
    assert st.next_token == want[0]
    pred, n = s.verify(want[0], want[1:12])
    assert n == 12 and list(pred) == want[1:13]
    s.close()


def test_verify_rejects_at_the_first_wrong_draft(hip_ctx):
    spec = synth.small_spec(**SMALL["llama-q4km"])
    img = synth.build(spec, seed=29)
    prompt = synth.prompt_tokens(6, 7, spec.vocab)
    want, _ = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True).generate(prompt, 30)
    want = [int(t) for t in want]
    s = hip.Session(hip_ctx, img, context=spec.context)
    s.generate(prompt, 0)
    drafts = want[1:9]
    drafts[2] = (drafts[2] + 1) % spec.vocab  # the third draft is wrong
    pred, n = s.verify(want[0], drafts)
    assert n == 3 and list(pred[:3]) == want[1:4]
    assert s.position == len(prompt) + 3
    # the rejected rows are overwritten: the stream goes on from the emitted token
    got, _ = s.generate(np.array([want[3]], np.uint32), 10)
    assert [int(t) for t in got] == want[4:14]
    # no drafts: one greedy step (want[14] is the pending token after the generated ones)
    pred, n = s.verify(want[14], [])
    assert n == 1 and int(pred[0]) == want[15]
    s.close()


def test_verify_rejects_bad_arguments(hip_ctx):
    spec = synth.small_spec()
    img = synth.build(spec, seed=1)
    s = hip.Session(hip_ctx, img, context=spec.context)
    with pytest.raises(hip.HipError):
        s.verify(1, list(range(16)))  # 17 tokens > one 16-token pass
    with pytest.raises(hip.HipError):
        s.verify(spec.vocab, [1, 2])  # out-of-range id
    s.close()


def test_rewind_then_verify_accepts_the_decoded_drafts(hip_ctx):
    # drafts decoded by the session itself, the position moved back, then verified: all accepted
    spec = synth.small_spec(**SMALL["qwen3-q8"])
    img = synth.build(spec, seed=31)
    prompt = synth.prompt_tokens(8, 11, spec.vocab)
    s = hip.Session(hip_ctx, img, context=spec.context)
    _, st = s.generate(prompt, 0)
    p0 = s.position
    drafts, st2 = s.generate(np.array([st.next_token], np.uint32), 8)
    s.rewind(p0)
    assert s.position == p0
    pred, n = s.verify(st.next_token, [int(t) for t in drafts])
    assert n == 9 and [int(t) for t in pred[:8]] == [int(t) for t in drafts]
    assert int(pred[8]) == st2.next_token
    with pytest.raises(hip.HipError):
        s.rewind(s.position + 1)
    s.close()


def test_prefill_cached_reuses_the_common_prefix(hip_ctx):
    # the stream after a prompt fed through prefill_cached equals a fresh session's, and the
    # reused prefix is the common prefix of the rows the session holds and the prompt
    spec = synth.small_spec(**SMALL["qwen3-q8"])
    img = synth.build(spec, seed=47)
    first = [int(t) for t in synth.prompt_tokens(12, 20, spec.vocab)]
    s = hip.Session(hip_ctx, img, context=spec.context)
    reused, nxt = s.prefill_cached(first)
    assert reused == 0 and s.position == 20
    gen, _ = s.generate(np.array([nxt], np.uint32), 6)  # rows: first, nxt, the 6 generated
    held = first + [nxt] + [int(t) for t in gen]
    assert s.position == len(held)

    def fresh(prompt):
        f = hip.Session(hip_ctx, img, context=spec.context)
        _, st = f.generate(np.array(prompt, np.uint32), 0)
        out, _ = f.generate(np.array([st.next_token], np.uint32), 8)
        f.close()
        return st.next_token, [int(t) for t in out]

    cases = [
        held + [7, 8, 9],            # extends every cached row (the reference's reuse case)
        first[:11] + [3, 4, 5, 6],   # diverges inside the cache: rows up to 11 kept
        held,                        # the cached rows themselves: the last token fed again
        [5, 6] + first,              # nothing in common
    ]
    for prompt in cases:
        common = 0
        while common < min(len(held), len(prompt)) and held[common] == prompt[common]:
            common += 1
        reused, nxt = s.prefill_cached(prompt)
        assert reused == common  # commonPrefixLen (model/loader.zig:2310-2313)
        want_next, want_stream = fresh(prompt)
        assert nxt == want_next
        out, _ = s.generate(np.array([nxt], np.uint32), 8)
        assert [int(t) for t in out] == want_stream
        held = list(prompt) + [nxt] + [int(t) for t in out]
    s.close()
