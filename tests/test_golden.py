"""Golden vectors (tests/golden/blocks.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every committed vector bit for bit (dequant)
and exactly (its deterministic matvec), so a change to the oracle that moves
any value fails here.  GPU: the HIP dequant reproduces the committed dequant
bits, and the HIP matvec is within 1e-4 relative L2 of the committed outputs
(and of a float64 dot of the committed dequant rows).
"""
import os

import numpy as np
import pytest

from oracle import zo

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GOLD = np.load(os.path.join(HERE, "blocks.npz"), allow_pickle=False)
CASES = {"fill_q4k": (12, 3), "q4_k": (12, 4), "q6_k": (14, 4), "q8_0": (8, 4), "q3_k": (11, 4), "iq4_xs": (23, 4)}
COLS = 512


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_reproduces_golden(name):
    ttype, rows = CASES[name]
    q = GOLD[f"{name}/bytes"]
    deq = zo.dequantize(ttype, q, rows, COLS)
    assert np.array_equal(deq.view(np.uint32), GOLD[f"{name}/dequant_bits"])
    y = zo.matvec(ttype, q, rows, COLS, GOLD[f"{name}/x"])
    assert np.array_equal(y, GOLD[f"{name}/y"])
    # the committed outputs are dot products of the committed dequant rows
    want = GOLD[f"{name}/dequant_bits"].view(np.float32).astype(np.float64) @ GOLD[f"{name}/x"].astype(np.float64)
    assert rel_l2(GOLD[f"{name}/y"], want) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_hip_matches_golden(hip_ctx, name):
    ttype, rows = CASES[name]
    q = GOLD[f"{name}/bytes"]
    out = hip_ctx.empty(rows * COLS * 4)
    mb = hip_ctx.buffer(q)
    hip_ctx.dequantize(ttype, mb, out, rows, COLS)
    assert np.array_equal(out.read(np.float32).view(np.uint32).reshape(rows, COLS), GOLD[f"{name}/dequant_bits"])
    y = hip_ctx.empty(rows * 4)
    hip_ctx.matvec(ttype, mb, hip_ctx.buffer(GOLD[f"{name}/x"]), y, rows, COLS)
    assert rel_l2(y.read(), GOLD[f"{name}/y"]) < 1e-4
