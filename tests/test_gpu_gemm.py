"""GPU parity of the MFMA path for M >= 8 tokens (ziggy_hip_run_gemm) against
the CPU oracle's matvec, token by token.

Bar: each token's output within 1e-4 relative L2 of the oracle (the matvec
tolerance); the bf16 hi/lo operand split keeps ~2^-16 relative error per
product.  Ragged token counts (1, 9, 33, 47, 65, 100) and row counts (not multiples of the
16-row tile) exercise the clamped tails.
"""
import sys

import numpy as np
import pytest

from oracle import zo
from zhip import synth
from zhip.gguf import F16, F32, IQ4_XS, Q3_K, Q4_K, Q6_K, Q8_0, row_bytes

pytestmark = pytest.mark.gpu
REL_L2 = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


# token counts of several 16-token tiles, ragged past them, with one- and several-stage reductions
SHAPES = [(1, 16, 256), (8, 100, 256), (9, 64, 4096), (16, 4096, 4096), (33, 300, 512), (9, 1000, 14336),
          (47, 200, 4096), (64, 300, 4096), (65, 130, 1024), (100, 1000, 512)]


@pytest.mark.parametrize("ttype", [Q4_K, Q6_K, Q8_0, IQ4_XS, Q3_K, F16, F32])
@pytest.mark.parametrize("shape", SHAPES)
def test_gemm_matches_oracle_per_token(hip_ctx, ttype, shape):
    tokens, rows, cols = shape
    if ttype == F32 and rows * cols > 4096 * 4096:
        pytest.skip("f32 matrix larger than the case needs")
    say(f"gemm type {ttype} tokens {tokens} {rows}x{cols}")
    q = np.zeros(row_bytes(ttype, cols) * rows, np.uint8)
    synth.fill_tensor(q, ttype, rows, cols, seed=rows * 7 + cols + ttype)
    x = np.stack([synth.normal_row(tokens + t, t, cols, 0.0, 1.0) for t in range(tokens)])
    m, xb = hip_ctx.buffer(q), hip_ctx.buffer(x)
    y = hip_ctx.empty(tokens * rows * 4)
    hip_ctx.gemm(ttype, m, xb, y, tokens, rows, cols)
    got = y.read().reshape(tokens, rows)
    for t in range(tokens):
        want = zo.matvec(ttype, q, rows, cols, x[t], threads=8)
        assert rel_l2(got[t], want) < REL_L2, (t, rel_l2(got[t], want))


@pytest.mark.parametrize("tokens", [9, 64])
def test_gemm_add_accumulates(hip_ctx, tokens):
    rows, cols = 256, 2048
    q = np.zeros(row_bytes(Q4_K, cols) * rows, np.uint8)
    synth.fill_tensor(q, Q4_K, rows, cols, seed=5)
    x = np.stack([synth.normal_row(1, t, cols, 0.0, 1.0) for t in range(tokens)])
    base = np.stack([synth.normal_row(2, t, rows, 0.0, 1.0) for t in range(tokens)])
    y = hip_ctx.buffer(base)
    hip_ctx.gemm(Q4_K, hip_ctx.buffer(q), hip_ctx.buffer(x), y, tokens, rows, cols, add=True)
    got = y.read().reshape(tokens, rows)
    for t in range(tokens):
        want = base[t] + zo.matvec(Q4_K, q, rows, cols, x[t], threads=8)
        assert rel_l2(got[t], want) < REL_L2
