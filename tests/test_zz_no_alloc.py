"""The allocation-free attention entry (ziggy_hip_attention_fused_f32_noalloc) against the context entry
(ziggy_hip_attention_fused_f32) through the C ABI.

Both run the same split-K kernels with the same split count, so their outputs must be bit-identical; the
no-alloc entry takes its partials and counters from a static per-device array that keeps the previous
call's contents, so two calls run back to back, the second at a smaller shape (fewer kv heads, fewer
splits), and both are also held to the oracle's attention at the matvec tolerance.
"""
import sys

import numpy as np
import pytest

from oracle import zo
from zhip import hip

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def run_both(ctx, heads, kvh, hd, pos, seed, window=0):
    rng = np.random.default_rng(seed)
    kv_dim = kvh * hd
    ctx_len = pos + 1
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = rng.standard_normal(ctx_len * kv_dim).astype(np.float16)
    v = rng.standard_normal(ctx_len * kv_dim).astype(np.float16)
    bq, bk, bv = ctx.buffer(q), ctx.buffer(k), ctx.buffer(v)
    out_ctx = ctx.empty(heads * hd * 4)
    out_na = ctx.empty(heads * hd * 4)
    ctx.attention(bq, bk, bv, out_ctx, heads, kvh, hd, kv_dim, ctx_len, pos, window_start=window)
    ctx.attention_noalloc(bq, bk, bv, out_na, heads, kvh, hd, kv_dim, ctx_len, pos, window_start=window)
    want = zo.attention(q, k.astype(np.float32), v.astype(np.float32), heads, kvh, hd, pos, window)
    return out_ctx.read(), out_na.read(), want


def test_noalloc_attention_matches_context_entry(hip_ctx):
    # first call: the Llama-3.1-8B shape at position 4095 (23 splits per kv head); second: a smaller
    # shape whose kv heads and splits cover only part of what the first call left in the array
    for heads, kvh, hd, pos, seed in [(32, 8, 128, 4095, 1), (8, 2, 64, 300, 2)]:
        say(f"noalloc attention {heads}/{kvh}x{hd} pos {pos}")
        got_ctx, got_na, want = run_both(hip_ctx, heads, kvh, hd, pos, seed)
        assert np.array_equal(got_na, got_ctx), (heads, kvh, hd, pos)
        assert rel_l2(got_na, want) < 1e-4


def test_noalloc_attention_sliding_window(hip_ctx):
    # window starts that are not a multiple of the 32-position tile (sliding-window layers,
    # model/loader.zig:1440-1444), the larger call first
    for heads, kvh, hd, pos, window, seed in [(32, 8, 128, 4095, 100, 3), (8, 2, 64, 300, 37, 4)]:
        say(f"noalloc attention {heads}/{kvh}x{hd} pos {pos} window {window}")
        got_ctx, got_na, want = run_both(hip_ctx, heads, kvh, hd, pos, seed, window)
        assert np.array_equal(got_na, got_ctx), (heads, kvh, hd, pos, window)
        assert rel_l2(got_na, want) < 1e-4


def test_noalloc_attention_rejects_partials_beyond_the_static_array(hip_ctx):
    # 512 kv heads of head_dim 256: one split each, 512 x 8 x 258 floats = 4.2 MB > the 4 MiB array.
    # Rejected on the host before any launch.
    heads = kvh = 512
    hd = 256
    say("noalloc attention oversize rejection")
    q = hip_ctx.empty(heads * hd * 4)
    kc = hip_ctx.empty(kvh * hd * 2)
    vc = hip_ctx.empty(kvh * hd * 2)
    out = hip_ctx.empty(heads * hd * 4)
    with pytest.raises(hip.HipError) as ei:
        hip_ctx.attention_noalloc(q, kc, vc, out, heads, kvh, hd, kvh * hd, 1, 0)
    assert "static scratch" in str(ei.value)
