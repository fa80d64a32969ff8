"""Pins the oracle's binary16 K/V rounding (zo_round_f16) against numpy.

The binary16 KV mode of the oracle rounds every stored K/V value as Metal's
store_kv_half does, `half(src[i])` (runtime/metal/matvec.metal:246-255): IEEE
round-to-nearest-even with gradual underflow, overflow to infinity from 65520.
numpy's float32 -> float16 cast is an independent implementation of the same
IEEE conversion, so it is the yardstick here.  The value set covers every
binary32 exponent, the mantissas at, just below and just above each rounding
tie (even and odd halves), every binary16 subnormal with its two neighbouring
ties, the subnormal/normal boundary, the 65504 / 65520 overflow boundary,
signed zeros, infinities and NaN, plus random bit patterns.  Two planted
misreadings of the conversion (truncation, ties away from zero) are shown to
differ from numpy on this set, so the set can tell them apart.
"""
import numpy as np
import pytest

from oracle import zo


def _bits(u):
    return np.array(u, np.uint32).view(np.float32)


def _value_set():
    vals = []
    # every binary32 exponent; mantissas around the binary16 rounding point of
    # a normal result (13 dropped bits: tie at 0x1000), with an even and an odd
    # kept bit, and the ends of the mantissa range
    mants = []
    for hm in (0, 1, 2, 3, 0x3FE, 0x3FF):
        base = hm << 13
        for off in (0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF):
            mants.append(base + off)
    mants += [0x7FFFFF, 0x400000, 0x3FFFFF]
    rng = np.random.default_rng(7)
    for e in range(256):
        ms = mants + list(rng.integers(0, 1 << 23, 16))
        for m in ms:
            for sgn in (0, 1):
                vals.append((sgn << 31) | (e << 23) | (int(m) & 0x7FFFFF))
    out = [_bits(vals)]
    # every binary16 subnormal k * 2^-24, the ties (k + 1/2) * 2^-24 and one
    # binary32 ulp either side of each tie
    k = np.arange(0, 1025, dtype=np.float64)
    for x in (k * 2.0 ** -24, (k + 0.5) * 2.0 ** -24):
        x32 = x.astype(np.float32)
        out += [x32, -x32, np.nextafter(x32, np.float32(np.inf)), np.nextafter(x32, np.float32(0))]
    # the smallest normal half and its neighbourhood
    tn = np.float32(2.0 ** -14)
    out.append(np.array([tn, np.nextafter(tn, np.float32(0)), np.nextafter(tn, np.float32(1)),
                         np.float32(2.0 ** -14 - 2.0 ** -25), np.float32(2.0 ** -25), np.float32(2.0 ** -26),
                         np.nextafter(np.float32(2.0 ** -25), np.float32(1))], np.float32))
    # overflow boundary: 65504 is the largest half; 65520 is the tie to 2^16 (inf)
    ov = np.array([65504.0, 65505.0, 65519.0, 65520.0, 65536.0, 1e30], np.float32)
    ov = np.concatenate([ov, np.nextafter(ov, np.float32(0)), np.nextafter(ov, np.float32(np.inf))])
    out += [ov, -ov]
    out.append(np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan], np.float32))
    out.append(_bits(np.random.default_rng(11).integers(0, 1 << 32, 20000, dtype=np.uint64).astype(np.uint32)))
    return np.concatenate(out).astype(np.float32)


def _numpy_round(v):
    with np.errstate(over="ignore"):
        return v.astype(np.float16).astype(np.float32)


def _same(a, b):
    # bit-identical, NaN == NaN (payloads differ between implementations)
    nan = np.isnan(a) & np.isnan(b)
    return nan | (a.view(np.uint32) == b.view(np.uint32))


def _truncating(v):
    """A planted misreading: binary16 by truncation (round toward zero)."""
    out = np.empty_like(v)
    with np.errstate(over="ignore"):
        for i, x in enumerate(v):
            h = np.float16(x)
            if np.isfinite(x) and np.isfinite(h) and abs(float(h)) > abs(float(x)):
                h = np.nextafter(h, np.float16(0))
            elif np.isfinite(x) and not np.isfinite(h):
                h = np.float16(np.copysign(65504.0, x))
            out[i] = np.float32(h)
    return out


def _ties_away(v):
    """A planted misreading: ties rounded away from zero instead of to even."""
    out = _numpy_round(v)
    with np.errstate(over="ignore"):
        for i, x in enumerate(v):
            _tie_away_one(out, i, x)
    return out


def _tie_away_one(out, i, x):
    if not np.isfinite(x) or abs(x) >= 65520:
        return
    h = np.float16(x)
    lo = np.nextafter(h, np.float16(-np.inf)) if float(h) > float(x) else h
    hi = np.nextafter(lo, np.float16(np.inf))
    if float(x) - float(lo) == float(hi) - float(x):  # an exact tie
        out[i] = np.float32(hi if x > 0 else lo)


VALUES = _value_set()


def test_round_f16_matches_numpy_ieee_conversion():
    got = zo.round_f16(VALUES)
    want = _numpy_round(VALUES)
    bad = ~_same(got, want)
    assert not bad.any(), (VALUES[bad][:8], got[bad][:8], want[bad][:8])


def test_round_f16_special_values():
    got = zo.round_f16(np.array([65504.0, 65519.996, 65520.0, -65520.0, 2.0 ** -25, 3 * 2.0 ** -25,
                                 2.0 ** -24, -0.0, np.inf, -np.inf], np.float32))
    assert got[0] == 65504.0 and got[1] == 65504.0
    assert got[2] == np.inf and got[3] == -np.inf
    assert got[4] == 0.0                # tie between 0 and 2^-24: to even (0)
    assert got[5] == 2.0 ** -23         # tie between 2^-24 and 2^-23: to even (2^-23)
    assert got[6] == 2.0 ** -24
    assert got[7] == 0.0 and np.signbit(got[7])
    assert got[8] == np.inf and got[9] == -np.inf
    assert np.isnan(zo.round_f16(np.array([np.nan], np.float32))[0])


@pytest.mark.parametrize("planted", [_truncating, _ties_away])
def test_value_set_rejects_planted_misreadings(planted):
    sub = VALUES[np.isfinite(VALUES)]
    assert (~_same(planted(sub), _numpy_round(sub))).sum() > 100
