"""The decode profiler's summary text against the reference's Profiler
(runtime/metal_profile.zig): its own unit test (:386-406), restated with the
same records and the same expected substrings, then figures worked out by hand
from the profiler's rules (shares of the category total, the top-three
insertion, shape order, token scoping).  Host code only: no GPU."""
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "ziggy-llm_amd"))
from zhip import hip  # noqa: E402


def recs(*rows):
    out = np.zeros(len(rows), hip.PROFILE_RECORD)
    for i, r in enumerate(rows):
        kind, ns = r[0], r[1]
        out[i]["kind"] = hip.PROFILE_KINDS[kind]
        out[i]["ns"] = ns
        if len(r) > 2:
            shape = r[2]
            out[i]["has_shape"] = 1
            for f in ("rows", "cols", "depth", "extra", "tensor_type"):
                out[i][f] = shape.get(f, 0)
    return out


def reference_case():
    # metal_profile.zig:388-396
    return recs(("token_begin", 0),
                ("projections", 200, dict(rows=64, cols=128, tensor_type=12)),
                ("attention", 90),
                ("kv_writes", 30, dict(rows=1, cols=128, depth=2)),
                ("cpu_sampling", 10),
                ("commit_wait", 50),
                ("commit_wait_gpu", 25),
                ("moon_quant", 150, dict(rows=64, cols=128, tensor_type=12)),
                ("token_end", 0))


def test_reference_unit_test_substrings():
    text = hip.render_profile(reference_case())
    for want in ("profile.top_bottleneck_1=projections:200ns",
                 "profile.shape_1=projections:rows=64:cols=128",
                 "profile.token_0.cpu_sampling.ns=10",
                 "profile.commit_wait.gpu_ns=25",
                 "profile.token_0.commit_wait.gpu_ns=25",
                 "moon_quant.profile.total_ns=150",
                 "moon_quant.profile.token_0.ns=150"):
        assert want in text, want


def test_reference_case_by_hand():
    text = hip.render_profile(reference_case())
    kv = hip.parse_profile(text)
    # the total is the sum over the nine categories: 200 + 90 + 30 + 10 + 50
    assert kv["profiled_decode_ns"] == "380"
    assert kv["profiled_decode_tokens"] == "1"
    assert kv["profile.projections.share_pct"] == "52.632"   # 200 / 380
    assert kv["profile.attention.calls"] == "1"
    assert kv["profile.normalization.ns"] == "0" and kv["profile.normalization.calls"] == "0"
    assert kv["moon_quant.profile.share_of_decode_pct"] == "39.474"  # 150 / 380, not part of the total
    assert kv["profile.commit_wait.gpu_share_of_decode_pct"] == "6.579"  # 25 / 380
    assert kv["profile.top_bottleneck_2"] == "attention:90ns:23.684pct"
    assert kv["profile.top_bottleneck_3"] == "commit_wait:50ns:13.158pct"
    # only recordWithShape calls make shapes; the larger total first
    assert kv["profile.shape_2"] == "kv_writes:rows=1:cols=128:depth=2:extra=0:tensor_type=0:calls=1:ns=30"
    assert "profile.shape_3" not in kv
    assert kv["moon_quant.profile.shape_1"] == "rows=64:cols=128:depth=0:extra=0:tensor_type=12:calls=1:ns=150"
    assert kv["profile.token_0.total_ns"] == "380"
    # key order of renderSummary
    keys = [line.split("=", 1)[0] for line in text.splitlines()]
    assert keys[:8] == ["metal_decode_profile_enabled", "profiled_decode_tokens", "profiled_decode_ns",
                        "moon_quant.profile.total_ns", "moon_quant.profile.calls",
                        "moon_quant.profile.share_of_decode_pct", "profile.commit_wait.gpu_ns",
                        "profile.commit_wait.gpu_share_of_decode_pct"]
    assert keys[8:11] == ["profile.projections.ns", "profile.projections.share_pct", "profile.projections.calls"]
    cats = [k.split(".")[1] for k in keys[8:8 + 27:3]]
    assert cats == hip.PROFILE_CATEGORIES
    tok = [k for k in keys if k.startswith(("profile.token_0", "moon_quant.profile.token_0"))]
    assert tok == (["profile.token_0.total_ns"] + [f"profile.token_0.{c}.ns" for c in hip.PROFILE_CATEGORIES]
                   + ["moon_quant.profile.token_0.ns", "profile.token_0.commit_wait.gpu_ns"])


def test_scoping_ties_and_aggregation():
    shp = dict(rows=4096, cols=4096, tensor_type=12)
    r = recs(("projections", 999, shp),            # before any token: ignored
             ("token_begin", 0),
             ("projections", 100, shp),
             ("attention", 100),                   # ties projections: the earlier category keeps slot 1
             ("projections", 5, shp),              # same shape: aggregated (2 calls, 105 ns)
             ("commit_wait_gpu", 0),               # zero GPU time: not counted
             ("output_reduce", 105, dict(rows=1, cols=1, depth=32000, tensor_type=14)),
             ("token_end", 0),
             ("attention", 7),                     # after the token: ignored
             ("token_begin", 0),
             ("normalization", 3),
             ("token_begin", 0),                   # a second begin drops the open breakdown
             ("elementwise_ops", 4),
             ("token_end", 0))
    kv = hip.parse_profile(hip.render_profile(r))
    assert kv["profiled_decode_tokens"] == "2"
    # categories keep what was recorded while a token was open, including the dropped breakdown
    assert kv["profile.projections.ns"] == "105" and kv["profile.projections.calls"] == "2"
    assert kv["profile.normalization.ns"] == "3"
    assert kv["profiled_decode_ns"] == str(105 + 100 + 105 + 3 + 4)
    assert kv["profile.top_bottleneck_1"].startswith("projections:105ns")
    assert kv["profile.top_bottleneck_2"].startswith("output_reduce:105ns")
    assert kv["profile.top_bottleneck_3"].startswith("attention:100ns")
    # equal totals: more calls first
    assert kv["profile.shape_1"] == "projections:rows=4096:cols=4096:depth=0:extra=0:tensor_type=12:calls=2:ns=105"
    assert kv["profile.shape_2"] == "output_reduce:rows=1:cols=1:depth=32000:extra=0:tensor_type=14:calls=1:ns=105"
    assert kv["profile.commit_wait.gpu_ns"] == "0"
    assert kv["profile.token_0.total_ns"] == "310" and kv["profile.token_1.total_ns"] == "4"
    assert kv["profile.token_1.normalization.ns"] == "0" and kv["profile.token_1.elementwise_ops.ns"] == "4"


def test_empty_and_errors():
    kv = hip.parse_profile(hip.render_profile(np.zeros(0, hip.PROFILE_RECORD)))
    assert kv["profiled_decode_tokens"] == "0"
    for i in (1, 2, 3):  # untouched slots: (projections, 0)
        assert kv[f"profile.top_bottleneck_{i}"] == "projections:0ns:0.000pct"
    bad = np.zeros(1, hip.PROFILE_RECORD)
    bad[0]["kind"] = 9
    with pytest.raises(hip.HipError):
        hip.render_profile(bad)


def test_shape_limit_is_eight():
    rows = [("token_begin", 0)] + [("projections", 100 + i, dict(rows=i + 1, cols=64)) for i in range(12)] + [
        ("token_end", 0)]
    kv = hip.parse_profile(hip.render_profile(recs(*rows)))
    assert "profile.shape_8" in kv and "profile.shape_9" not in kv
    assert kv["profile.shape_1"].startswith("projections:rows=12:")  # the largest total
