"""Deterministic inputs of the golden fixtures (pure numpy; no oracle).

fill_q4k_matrix restates the reference test generator fillQ4KMatrix
(runtime/metal_backend_test.zig:894-924); the input ramps restate the inputs
of the reference's matvec tests (runtime/metal_backend_test.zig:18-20 for
Q4_K, :125-127 for the Q4_K model test, :311-313 for Q6_K, :533-535 for
Q8_0); special_blocks are random block bytes with the binary16 scale fields
forced to special values (subnormal, max normal, negative zero, one, the
smallest normal, negative max).
"""
import numpy as np

# GGUF type ids (model/loader.zig:119-153)
Q8_0, Q3_K, Q4_K, Q6_K, IQ4_XS = 8, 11, 12, 14, 23
BLOCK = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_0: (32, 34), Q3_K: (256, 110), IQ4_XS: (256, 136)}
SCALE_FIELDS = {Q4_K: [0, 2], Q6_K: [208], Q8_0: [0], Q3_K: [108], IQ4_XS: [0]}
SPECIAL_F16 = [0x0001, 0x03FF, 0x7BFF, 0x8000, 0x3C00, 0x0400, 0xFBFF]


def row_bytes(ttype, cols):
    v, b = BLOCK[ttype]
    return cols // v * b


def fill_q4k_matrix(rows, cols):
    rs = cols // 256 * 144
    buf = np.zeros(rows * rs, np.uint8)
    for r in range(rows):
        for b in range(cols // 256):
            base = r * rs + b * 144
            buf[base:base + 2] = np.frombuffer(np.float16(0.125 * (r + b + 1)).tobytes(), np.uint8)
            buf[base + 2:base + 4] = np.frombuffer(np.float16(0.0625 * (b + 1)).tobytes(), np.uint8)
            for i in range(4):
                buf[base + 4 + i] = (1 + r + b + i) & 63
                buf[base + 8 + i] = (i + b) & 63
                buf[base + 12 + i] = ((1 + r + i) & 0x0F) | (((2 + b + i) & 0x0F) << 4)
            for i in range(128):
                lo, hi = (i + r + b) % 16, (i * 3 + r + b + 5) % 16
                buf[base + 16 + i] = lo | (hi << 4)
    return buf


def special_blocks(ttype, rows, cols, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, row_bytes(ttype, cols) * rows, dtype=np.uint8)
    nb = BLOCK[ttype][1]
    for i in range(len(q) // nb):
        for o in SCALE_FIELDS[ttype]:
            v = SPECIAL_F16[(i + o) % len(SPECIAL_F16)]
            q[i * nb + o] = v & 0xFF
            q[i * nb + o + 1] = v >> 8
    return q


def ramp(n, mod, shift, step, offset):
    """((i % mod) - shift) * step + offset, in binary32 as the reference computes it."""
    i = np.arange(n)
    return ((i % mod - shift).astype(np.float32) * np.float32(step) + np.float32(offset)).astype(np.float32)


RAMPS = {
    "q4k_matvec": (17, 8, 0.125, 0.1),      # metal_backend_test.zig:18-20
    "q4k_model": (31, 15, 0.03125, 0.02),   # :125-127
    "q6k": (19, 9, 0.0625, 0.05),           # :311-313
    "q8_0": (13, 6, 0.125, 0.05),           # :533-535
}
