"""bench.py's KV sizing: every leg of a run fits the cache it allocates (CPU only, no GPU).

The driver runs `bench.py --gpus 1 --steps 20 --warmup 5`; the builder's own runs use 256 / 16.  A run
uses, in order: the prompt and warm-up steps (prompt + warmup rows), the timed decode (1 + steps rows),
one free row for the per-kernel timing, then the CPU baseline from pos0 = prompt + warmup + 1 for up to
CPU_MAX_STEPS steps on a cache filled to pos0, and for config 4 three verify passes of 9 rows.
"""
import pytest

import bench


@pytest.mark.parametrize("model", ["llama8b", "tinyllama", "qwen3"])
@pytest.mark.parametrize("steps,warmup,prompt", [(20, 5, 4096), (256, 16, 4096), (1, 0, 32), (128, 16, 16384)])
def test_every_leg_fits_the_cache(model, steps, warmup, prompt):
    ctx = bench.context_length(model, prompt, warmup, steps)
    gpu_rows = prompt + warmup + 1 + steps
    assert gpu_rows + 1 <= ctx  # time_kernel needs one free row
    if model == "qwen3":
        assert gpu_rows + 3 * 9 + 1 <= ctx
    pos0 = prompt + warmup + 1
    budget = bench.cpu_step_budget(ctx, pos0)
    # the CPU sample is never cut short by the cache, and its last step stays inside it
    assert budget == bench.CPU_MAX_STEPS
    assert pos0 + budget <= ctx


def test_cpu_budget_caps_at_the_cache():
    assert bench.cpu_step_budget(100, 90) == 10
    assert bench.cpu_step_budget(100, 100) == 0
    assert bench.cpu_step_budget(10_000, 0) == bench.CPU_MAX_STEPS
