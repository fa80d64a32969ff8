"""The measurement probes behind the launch-structure figures run and report
sane values: the in-launch dependency latencies (no wait ran out of its
bound) and the input-row load patterns (every pattern timed, on two
workgroups per CU)."""
import math
import sys

import pytest

from zhip import hip

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_sync_probe(hip_ctx):
    say("probe_sync: 200 rounds")
    r = hip_ctx.probe_sync(200)
    assert not r.timed_out
    assert r.workgroups > 0
    for v in (r.handoff_relaxed_us, r.handoff_acqrel_us, r.barrier_flags_us, r.barrier_counter_us):
        assert math.isfinite(v) and 0 < v < 1000


def test_row_load_probe(hip_ctx):
    say("probe_row_load: 5 launches per pattern")
    r = hip_ctx.probe_row_load(5)
    assert r.values == 4096 and r.workgroups % 2 == 0 and r.workgroups > 0
    for arr in (r.slot_us, r.coalesced_us, r.lds_us):
        for v in arr:
            assert math.isfinite(v) and 0 < v < 1000
    with pytest.raises(hip.HipError):
        hip_ctx.probe_row_load(0)
