"""Writes tests/golden/blocks.npz: golden dequant and dot vectors.

Generated in the build container by the C oracle (oracle/, a restatement of
the reference's CPU decoders), from the deterministic inputs of vectors.py:
  * fillQ4KMatrix (3 x 512) and the reference Q4_K matvec ramp;
  * per format (Q4_K, Q6_K, Q8_0, Q3_K, IQ4_XS): 4 x 512 special blocks
    (binary16 scale fields forced to special values) and the format's
    reference test ramp (Q3_K / IQ4_XS reuse the Q4_K one);
for each: the raw bytes, the dequantized f32 rows (bit patterns) and the
oracle's matvec output on the ramp.

Run from the repository root:  python3 tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, HERE)

from oracle import zo  # noqa: E402
from vectors import (IQ4_XS, Q3_K, Q4_K, Q6_K, Q8_0, RAMPS, fill_q4k_matrix, ramp,  # noqa: E402
                     special_blocks)


def main():
    out = {}
    rows, cols = 3, 512
    m = fill_q4k_matrix(rows, cols)
    x = ramp(cols, *RAMPS["q4k_matvec"])
    out["fill_q4k/bytes"] = m
    out["fill_q4k/dequant_bits"] = zo.dequantize(Q4_K, m, rows, cols).view(np.uint32)
    out["fill_q4k/x"] = x
    out["fill_q4k/y"] = zo.matvec(Q4_K, m, rows, cols, x)
    ramp_of = {Q4_K: "q4k_model", Q6_K: "q6k", Q8_0: "q8_0", Q3_K: "q4k_matvec", IQ4_XS: "q4k_matvec"}
    for t, name in ((Q4_K, "q4_k"), (Q6_K, "q6_k"), (Q8_0, "q8_0"), (Q3_K, "q3_k"), (IQ4_XS, "iq4_xs")):
        r, c = 4, 512
        q = special_blocks(t, r, c, seed=100 + t)
        xr = ramp(c, *RAMPS[ramp_of[t]])
        out[f"{name}/bytes"] = q
        out[f"{name}/dequant_bits"] = zo.dequantize(t, q, r, c).view(np.uint32)
        out[f"{name}/x"] = xr
        out[f"{name}/y"] = zo.matvec(t, q, r, c, xr)
    np.savez_compressed(os.path.join(HERE, "blocks.npz"), **out)
    print("wrote", os.path.join(HERE, "blocks.npz"), {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
