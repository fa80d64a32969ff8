"""The profiled decode (ziggy_hip_session_profile_decode): the same greedy
tokens as unprofiled steps, one record per launch under the reference's
categories (runtime/gpu/session.zig's recordCategoryWithShape calls, fused
here), and device times that account for the step."""
import sys

import numpy as np
import pytest

from zhip import hip, synth

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_profile_decode_tokens_and_records(hip_ctx):
    say("profile_decode small qwen3")
    spec = synth.small_spec(arch="qwen3", qk_norm=True)
    img = synth.build(spec, seed=29)
    prompt = synth.prompt_tokens(5, 6, spec.vocab)
    steps = 6
    s = hip.Session(hip_ctx, img, context=spec.context)
    want, _ = s.generate(prompt, steps + 1)  # the prompt's next token, then `steps` more
    s.reset()
    for t in prompt[:-1]:
        s.step_no_output(int(t))
    toks, recs = s.profile_decode(int(prompt[-1]), steps)
    assert list(toks) == [int(t) for t in want[:steps]]
    assert s.position == len(prompt) - 1 + steps
    L = spec.n_layers
    assert len(recs) == (5 * L + 7) * steps
    K = hip.PROFILE_KINDS
    per = recs.reshape(steps, 5 * L + 7)
    for t in range(steps):
        r = per[t]
        assert r[0]["kind"] == K["token_begin"] and r[-1]["kind"] == K["token_end"]
        kinds = list(r["kind"][1:-1])
        launches = kinds[:5 * L + 2]
        assert launches[0] == K["elementwise_ops"] and launches[-1] == K["output_reduce"]
        body = np.array(launches[1:-1]).reshape(L, 5)
        assert (body == [K["projections"], K["attention"], K["projections"], K["projections"],
                         K["projections"]]).all()
        assert kinds[5 * L + 2:] == [K["commit_wait"], K["commit_wait_gpu"], K["host_readback"]]
        att = r[1 + 2]  # layer 0's attention: session.zig:445-450's shape
        assert att["rows"] == spec.n_head and att["extra"] == spec.n_kv
        assert att["depth"] == len(prompt) + t
        out = r[1 + 5 * L + 1]
        assert out["depth"] == spec.vocab
        # the launches' intervals tile the step's first-to-last event time
        # (each rounded down to whole nanoseconds)
        dev = int(r["ns"][1:1 + 5 * L + 2].sum())
        gpu = int(r[1 + 5 * L + 3]["ns"])
        assert gpu > 0 and abs(dev - gpu) <= 1e-4 * gpu + 2 * (5 * L + 2)
    kv = hip.parse_profile(hip.render_profile(recs))
    assert kv["profiled_decode_tokens"] == str(steps)
    assert int(kv["profile.projections.calls"]) == 4 * L * steps
    assert int(kv["profile.attention.calls"]) == L * steps
    assert int(kv["profile.output_reduce.calls"]) == steps
    assert int(kv["profile.commit_wait.calls"]) == steps
    say(hip.render_profile(recs).split("profile.token_0")[0])
    s.close()


def test_profile_decode_rejects_small_buffer_and_overflow(hip_ctx):
    spec = synth.small_spec(context=16)
    img = synth.build(spec, seed=31)
    s = hip.Session(hip_ctx, img, context=16)
    with pytest.raises(hip.HipError):
        s.profile_decode(3, 17)  # past the context
    assert s.position == 0
    s.close()
