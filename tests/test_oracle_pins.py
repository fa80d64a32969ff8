"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Every check here is independent of the oracle's own formula: known-answer
tests and golden outputs the reference's tests hold, closed forms of the
reference's fixture encoders, brute-force bit-layout probes, f64 invariants,
and the reference's own test references restated from its test files.
"""
import numpy as np
import pytest

from oracle import zo
from zhip import synth
from zhip.gguf import F16, F32, IQ4_XS, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0

HALF_ONE = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)


def f16(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


# ---------------- known answers held by the reference ----------------

def test_scale_min_k4_known_answer():
    # moon_quant.zig:401-434: raw scale bytes -> scales {1..8}, mins {9..15, 1}
    raw = bytes([1, 2, 3, 4, 9, 10, 11, 12, 5 | (13 << 4), 6 | (14 << 4), 7 | (15 << 4), 8 | (1 << 4)])
    got = [zo.scale_min_k4(j, raw) for j in range(8)]
    assert [g[0] for g in got] == [1, 2, 3, 4, 5, 6, 7, 8]
    assert [g[1] for g in got] == [9, 10, 11, 12, 13, 14, 15, 1]


@pytest.mark.parametrize("ttype,nbytes", [(Q3_K, 110), (IQ4_XS, 136)])
def test_zero_blocks_decode_to_zero(ttype, nbytes):
    # model/quant_extra.zig:299-318
    out = zo.dequantize(ttype, np.zeros(nbytes, np.uint8), 1, 256)
    assert np.all(out == 0)


def test_q5k_known_answer_block_reference_quirk():
    # model/loader.zig:4599-4620 asserts 16.0 everywhere and dot 4096 for this
    # block, but the bytes it sets (scale bytes 0-7) only give sub-blocks 0-3 a
    # scale of 1 under getScaleMinK4 (:3814-3825, pinned by the known answer
    # above): sub-blocks 4-7 take their scale from bytes 8-11, which stay 0.
    # The oracle follows the decoder; this records the discrepancy.
    row = np.zeros(176, np.uint8)
    row[0:2] = HALF_ONE
    row[4:8] = 1
    row[8:12] = 1
    row[16:48] = 0xFF
    d = zo.dequantize(Q5_K, row, 1, 256)[0]
    assert np.all(d[:128] == 16.0) and np.all(d[128:] == 0.0)
    assert zo.dot_row(Q5_K, row, np.ones(256, np.float32)) == 2048.0


def test_topk_known_answer():
    # runtime/metal_backend_test.zig:47-71: k=3 -> {4, 1, 6}, ties to the lower index
    idx, w = zo.select_topk(np.array([0.2, 1.5, -2.0, 1.0, 3.0, 0.4, 1.5, -1.0], np.float32), 3)
    assert list(idx) == [4, 1, 6]
    assert list(w) == [3.0, 1.5, 1.5]


def test_argmax_known_answer_and_ties():
    # runtime/metal_backend_test.zig:872-892 and sampling.zig:196-206 (first maximum wins)
    assert zo.argmax(np.array([-1.0, 4.0, 2.5, 4.5, 3.0], np.float32)) == 3
    assert zo.argmax(np.array([1.0, 7.0, 7.0, 2.0], np.float32)) == 1


def test_toy_fixture_golden_text():
    # runtime/llama_runtime.zig:212-235: greedy from "a" (token 3) -> " b c!"
    img = synth.toy_llama_fixture()
    s = zo.Session(zo.Model(img.buf))
    toks, _ = s.generate([3], 3)
    assert list(toks) == [4, 5, 6]
    assert synth.toy_detokenize(toks) == " b c!"


@pytest.mark.parametrize("ptype", [Q4_K, Q6_K])
def test_toy_quant_fixtures_golden_text(ptype):
    # runtime/llama_runtime.zig:274-326 (Q4_K fixture, 6 tokens); Q6_K from makeLlamaQ6KFixture
    img = synth.toy_llama_fixture(256, 256, ptype, ptype)
    s = zo.Session(zo.Model(img.buf))
    toks, _ = s.generate([3], 6)
    assert synth.toy_detokenize(toks) == " b c! a b c"


# ---------------- closed forms of the reference's fixture encoders ----------------

@pytest.mark.parametrize("ttype", [Q4_K, Q6_K])
def test_binary_fixture_blocks_decode_exactly(ttype):
    # appendQ4KBlock / appendQ6KBlock (runtime/llama_fixture.zig:342-425) encode
    # 0/1 values whose decode is the input itself.
    rng = np.random.default_rng(1)
    v = rng.integers(0, 2, size=(3, 512)).astype(np.float32)
    blocks = synth._binary_blocks(v, ttype, 512)
    assert np.array_equal(zo.dequantize(ttype, blocks, 3, 512), v)
    x = rng.standard_normal(512).astype(np.float32)
    for r in range(3):
        exact = float(np.dot(v[r].astype(np.float64), x.astype(np.float64)))
        rb = zo.row_bytes(ttype, 512)
        assert abs(zo.dot_row(ttype, blocks[r * rb:(r + 1) * rb], x) - exact) <= 1e-5 * max(1.0, abs(exact))


def test_q8_0_fixture_encodes_zero_as_plus_one():
    # appendQ8_0Block (runtime/llama_fixture.zig:379-386): q = +1 if v >= 0 else -1
    v = np.array([0, 1, 0, 1] * 8, np.float32)[None, :]
    out = zo.dequantize(Q8_0, synth._binary_blocks(v, Q8_0, 32), 1, 32)
    assert np.all(out == 1.0)


# ---------------- brute-force bit-layout probes ----------------

def q4k_unit_block():
    # d = 1, dmin = 0, every sub-block scale 1, min 0: s[0..3] = 1, s[8..11] = 1
    b = np.zeros(144, np.uint8)
    b[0:2] = HALF_ONE
    b[4:8] = 1
    b[12:16] = 1
    return b


def test_q4k_nibble_layout_brute_force():
    # byte l of group g: low nibble -> value 64g + l, high nibble -> 64g + 32 + l
    for g in range(4):
        for l in range(32):
            for hi in (0, 1):
                b = q4k_unit_block()
                b[16 + 32 * g + l] = 0xF0 if hi else 0x0F
                out = zo.dequantize(Q4_K, b, 1, 256)[0]
                want = np.zeros(256, np.float32)
                want[64 * g + 32 * hi + l] = 15.0
                assert np.array_equal(out, want)


def test_q4k_scale_and_min_index_mapping():
    # sub-block j (values 32j..32j+31) uses scale/min index j of getScaleMinK4
    for j in range(8):
        b = q4k_unit_block()
        b[2:4] = HALF_ONE  # dmin = 1
        raw = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
        # give sub-block j scale 3 and min 2, using the 6-bit packing of getScaleMinK4
        sc, mn = 3, 2
        if j < 4:
            raw[j], raw[j + 4] = sc, mn
        else:
            raw[j + 4] = sc | (mn << 4)
        b[4:16] = raw
        b[16:144] = 0x11  # every nibble 1
        out = zo.dequantize(Q4_K, b, 1, 256)[0]
        want = np.ones(256, np.float32)
        want[32 * j:32 * j + 32] = 3.0 - 2.0
        assert np.array_equal(out, want), j


def test_q6k_bit_layout_brute_force():
    # d = 1, all scales 1, qh = 0xAA (high bits 2 -> +32 cancels -32)
    def base():
        b = np.zeros(210, np.uint8)
        b[128:192] = 0xAA
        b[192:208] = 1
        b[208:210] = HALF_ONE
        return b
    for h in range(2):
        for l in range(32):
            for off, nib_hi, idx in ((0, 0, l), (32, 0, 32 + l), (0, 1, 64 + l), (32, 1, 96 + l)):
                b = base()
                b[64 * h + off + l] = 0x50 if nib_hi else 0x05
                out = zo.dequantize(Q6_K, b, 1, 256)[0]
                want = np.zeros(256, np.float32)
                want[128 * h + idx] = 5.0
                assert np.array_equal(out, want), (h, l, off, nib_hi)
            for k in range(4):  # qh[32h + l] bits 2k..2k+1 -> value 128h + 32k + l
                b = base()
                b[128 + 32 * h + l] = (0xAA & ~(3 << (2 * k))) | (3 << (2 * k))  # field 3 -> +16
                out = zo.dequantize(Q6_K, b, 1, 256)[0]
                want = np.zeros(256, np.float32)
                want[128 * h + 32 * k + l] = 16.0
                assert np.array_equal(out, want), (h, l, k)


def test_q6k_signed_scale_per_16_values():
    for i in range(16):
        b = np.zeros(210, np.uint8)
        b[128:192] = 0xAA
        b[0:128] = 0x11  # every value 1
        b[192:208] = 1
        b[192 + i] = 0xFD  # -3
        b[208:210] = HALF_ONE
        out = zo.dequantize(Q6_K, b, 1, 256)[0]
        want = np.ones(256, np.float32)
        want[16 * i:16 * i + 16] = -3.0
        assert np.array_equal(out, want)


def test_iq4xs_table_and_scale_codes():
    # dl = d * (ls - 32), value = dl * kvalues_iq4nl[n] (model/quant_extra.zig:8, 205-212)
    kv = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    for ib in range(8):
        for code in (0, 31, 33, 63):
            for n in range(16):
                b = np.zeros(136, np.uint8)
                b[0:2] = HALF_ONE
                b[4 + ib // 2] = (code & 0xF) << (4 * (ib % 2))
                sh = ((code >> 4) & 3) << (2 * ib)
                b[2], b[3] = sh & 0xFF, sh >> 8
                b[8 + 16 * ib + 3] = n | (n << 4)
                out = zo.dequantize(IQ4_XS, b, 1, 256)[0]
                dl = code - 32
                assert out[32 * ib + 3] == dl * kv[n] and out[32 * ib + 19] == dl * kv[n]
                other = np.delete(out[32 * ib:32 * ib + 32], [3, 19])
                assert np.all(other == dl * kv[0])


def test_q3k_values_and_scale_codes():
    # value = d * (scale_code - 32) * ((2-bit q) - (hmask bit ? 0 : 4))
    rng = np.random.default_rng(7)
    for trial in range(20):
        codes = rng.integers(0, 64, 16)
        raw = np.zeros(12, np.uint8)
        for k in range(4):  # the 6-bit packing expandQ3KScales undoes (model/quant_extra.zig:248-279)
            raw[k] = (codes[k] & 0xF) | ((codes[8 + k] & 0xF) << 4)
            raw[4 + k] = (codes[4 + k] & 0xF) | ((codes[12 + k] & 0xF) << 4)
            raw[8 + k] = (codes[k] >> 4) | ((codes[4 + k] >> 4) << 2) | ((codes[8 + k] >> 4) << 4) | \
                         ((codes[12 + k] >> 4) << 6)
        v = rng.integers(0, 256)
        h, r = v // 128, v % 128
        j, s, l = r // 32, (r % 32) // 16, r % 16
        q2, hb = rng.integers(0, 4), rng.integers(0, 2)
        b = np.zeros(110, np.uint8)
        b[96:108] = raw
        b[108:110] = HALF_ONE
        b[32 + 32 * h + 16 * s + l] = q2 << (2 * j)
        if hb:
            b[16 * s + l] = 1 << (4 * h + j)
        out = zo.dequantize(Q3_K, b, 1, 256)[0]
        sc = codes[v // 16] - 32
        assert out[v] == sc * (q2 - (0 if hb else 4))
        mask = np.ones(256, bool)
        mask[v] = False
        assert np.all(out[mask] == (codes[np.arange(256)[mask] // 16] - 32) * -4.0)


# ---------------- dot vs dequant (f64 ground truth) ----------------

@pytest.mark.parametrize("ttype", [Q4_K, Q6_K, Q8_0, Q3_K, IQ4_XS, F16, F32])
def test_dot_matches_f64_dot_of_dequant(ttype):
    rng = np.random.default_rng(ttype)
    cols, rows = 1024, 8
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    q = synth.quantize_rows(w, ttype)
    deq = zo.dequantize(ttype, q, rows, cols).astype(np.float64)
    x = rng.standard_normal(cols).astype(np.float32)
    y = zo.matvec(ttype, q, rows, cols, x)
    ref = deq @ x.astype(np.float64)
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 1e-5, rel


# ---------------- elementwise closed forms ----------------

def test_rms_norm_closed_form():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(4096).astype(np.float32) * 3
    w = rng.standard_normal(4096).astype(np.float32)
    out = zo.rms_norm(x, w, 1e-5)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt(np.mean(xd * xd) + 1e-5) * w
    assert np.max(np.abs(out - ref)) < 1e-5 * np.max(np.abs(ref))


def test_softmax_invariants():
    v = np.array([1.0, 2.0, 3.0, -1.0], np.float32)
    s = zo.softmax(v)
    assert abs(s.sum() - 1) < 1e-6
    assert np.allclose(s, zo.softmax(v + 100.0), atol=1e-7)
    e = np.exp(v.astype(np.float64) - 3)
    assert np.allclose(s, e / e.sum(), rtol=1e-6)


@pytest.mark.parametrize("style", [0, 1])
def test_rope_invariants(style):
    rng = np.random.default_rng(5)
    v = rng.standard_normal(2 * 128).astype(np.float32)
    assert np.array_equal(zo.rope(v, 2, 128, 128, 0, 10000.0, style), v)  # pos 0 is the identity
    r = zo.rope(v, 2, 128, 128, 37, 10000.0, style)
    pairs = (lambda a: a.reshape(2, 64, 2).transpose(2, 0, 1)) if style == 0 else (lambda a: a.reshape(2, 2, 64).transpose(1, 0, 2))
    n0 = np.hypot(*pairs(v.astype(np.float64)))
    n1 = np.hypot(*pairs(r.astype(np.float64)))
    assert np.allclose(n0, n1, rtol=1e-5)  # each rotated pair keeps its norm
    r2 = zo.rope(zo.rope(v, 2, 128, 128, 10, 500000.0, style), 2, 128, 128, 27, 500000.0, style)
    assert np.allclose(r2, zo.rope(v, 2, 128, 128, 37, 500000.0, style), atol=2e-5)  # rotations compose
    # partial rotary dims leave the tail untouched (metal_backend_test.zig:768-870 uses 6 of 8)
    p = zo.rope(v[:16], 2, 8, 6, 3, 10000.0, style)
    assert np.array_equal(p.reshape(2, 8)[:, 6:], v[:16].reshape(2, 8)[:, 6:])


def test_rope_reference_test_case():
    # applyRoPEReference (runtime/metal_backend_test.zig:978-1010): 2 heads, hd 8,
    # rope_dim 6, position 3, base 10000, interleaved; src = (i - 7) * 0.125 + 0.05
    src = (np.arange(16, dtype=np.float64) - 7) * 0.125 + 0.05
    want = src.copy()
    for h in range(2):
        for pair in range(0, 6, 2):
            th = 3.0 / 10000.0 ** (pair / 6)
            x0, x1 = src[8 * h + pair], src[8 * h + pair + 1]
            want[8 * h + pair] = x0 * np.cos(th) - x1 * np.sin(th)
            want[8 * h + pair + 1] = x0 * np.sin(th) + x1 * np.cos(th)
    got = zo.rope(src.astype(np.float32), 2, 8, 6, 3, 10000.0, 0)
    assert np.max(np.abs(got - want)) < 5e-6


def attention_f64(q, kc, vc, heads, kv_heads, hd, pos, scale):
    # attentionReference (runtime/metal_backend_test.zig:932-976) in float64
    kv_dim = kv_heads * hd
    out = np.zeros(heads * hd)
    for h in range(heads):
        kvh = h // (heads // kv_heads)
        qh = q[h * hd:(h + 1) * hd].astype(np.float64)
        k = kc.reshape(-1, kv_dim)[:pos + 1, kvh * hd:(kvh + 1) * hd].astype(np.float64)
        v = vc.reshape(-1, kv_dim)[:pos + 1, kvh * hd:(kvh + 1) * hd].astype(np.float64)
        s = k @ qh * scale
        p = np.exp(s - s.max())
        out[h * hd:(h + 1) * hd] = (p / p.sum()) @ v
    return out


def test_attention_reference_test_case():
    # the reference's own case (runtime/metal_backend_test.zig:691-766): 3 heads, 1 kv head, hd 96, pos 4
    heads, kvh, hd, pos = 3, 1, 96, 4
    q = ((np.arange(heads * hd) % 19 - 9) * 0.07 + 0.02).astype(np.float32)
    kc = ((np.arange(5 * hd) % 17 - 8) * 0.06 - 0.01).astype(np.float32)
    vc = ((np.arange(5 * hd) % 13 - 6) * 0.08 + 0.03).astype(np.float32)
    got = zo.attention(q, kc, vc, heads, kvh, hd, pos)
    want = attention_f64(q, kc, vc, heads, kvh, hd, pos, 1 / np.sqrt(hd))
    assert np.max(np.abs(got - want)) < 1e-5


def test_attention_invariants():
    rng = np.random.default_rng(9)
    heads, kvh, hd, pos = 8, 2, 64, 40
    kc = rng.standard_normal((pos + 1) * kvh * hd).astype(np.float32)
    vc = rng.standard_normal((pos + 1) * kvh * hd).astype(np.float32)
    # q = 0: uniform weights -> mean of v
    out = zo.attention(np.zeros(heads * hd, np.float32), kc, vc, heads, kvh, hd, pos)
    vm = vc.reshape(pos + 1, kvh, hd).mean(axis=0)
    for h in range(heads):
        assert np.allclose(out[h * hd:(h + 1) * hd], vm[h // (heads // kvh)], atol=1e-5)
    # position 0: output is v_0
    q = rng.standard_normal(heads * hd).astype(np.float32)
    out0 = zo.attention(q, kc, vc, heads, kvh, hd, 0)
    for h in range(heads):
        kv = h // (heads // kvh)
        assert np.allclose(out0[h * hd:(h + 1) * hd], vc[kv * hd:(kv + 1) * hd], atol=1e-6)
    # general position vs the float64 reference
    got = zo.attention(q, kc, vc, heads, kvh, hd, pos)
    want = attention_f64(q, kc, vc, heads, kvh, hd, pos, 1 / np.sqrt(hd))
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-6


def test_moe_routing_closed_form():
    # softmax over all experts, top-k, renormalise == softmax over the top-k logits
    rng = np.random.default_rng(11)
    logits = rng.standard_normal(256).astype(np.float32)
    p = zo.softmax(logits)
    idx, w = zo.select_topk(p, 8)
    w = zo.normalize_positive(w)
    top = np.argsort(-logits.astype(np.float64), kind="stable")[:8]
    assert list(idx) == list(top)
    e = np.exp(logits[top].astype(np.float64) - logits[top].max())
    assert np.allclose(w, e / e.sum(), rtol=1e-5)


def test_f16_to_f32_matches_numpy_for_every_bit_pattern():
    # readF16AsF32 (model/loader.zig:4484-4488) is an exact widening, subnormals,
    # infinities and NaN payload class included: numpy's binary16 is the pin
    bits = np.arange(1 << 16, dtype=np.uint32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([zo.lib().zo_f16_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_silu_and_sigmoid_closed_forms():
    # siluInPlace / sigmoidScalar (model/loader.zig:4004-4029) against float64
    x = np.concatenate([np.linspace(-30, 30, 601), [0.0, -0.0, 1e-30, -88.0, 88.0]]).astype(np.float32)
    got = zo.silu(x)
    xd = x.astype(np.float64)
    want = xd / (1.0 + np.exp(-xd))
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 4e-7
    for v in (-20.0, -1.5, 0.0, 0.25, 3.0, 20.0):
        s = zo.lib().zo_sigmoid(float(np.float32(v)))
        assert abs(s - 1.0 / (1.0 + np.exp(-v))) < 1e-7


def test_rms_norm_per_head_closed_form():
    # rmsNormPerHeadWithOffset (model/loader.zig:1777-1812): each head slice is
    # normalised on its own (its own mean square) with the shared weights
    rng = np.random.default_rng(13)
    heads, hd = 5, 64
    x = rng.standard_normal(heads * hd).astype(np.float32)
    w = rng.standard_normal(hd).astype(np.float32)
    got = zo.rms_norm_per_head(x, w, heads, hd, 1e-6)
    # heads are independent: a head computed alone gives the same bits
    for h in range(heads):
        alone = zo.rms_norm_per_head(x[h * hd:(h + 1) * hd].copy(), w, 1, hd, 1e-6)
        assert np.array_equal(got[h * hd:(h + 1) * hd], alone)
    xd = x.reshape(heads, hd).astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(got.reshape(heads, hd) - want)) < 1e-5


def test_attention_window_is_the_truncated_cache():
    # computeAttention attends to [window_start, position] (model/loader.zig:1397-1438): with a window
    # it equals the attention over the cache rows from window_start on, at position - window_start
    rng = np.random.default_rng(3)
    heads, kvh, hd, pos = 8, 2, 64, 90
    kv_dim = kvh * hd
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = rng.standard_normal((pos + 1) * kv_dim).astype(np.float32)
    v = rng.standard_normal((pos + 1) * kv_dim).astype(np.float32)
    for w in (0, 1, 37, 64, 90):
        got = zo.attention(q, k, v, heads, kvh, hd, pos, w)
        want = zo.attention(q, k[w * kv_dim:], v[w * kv_dim:], heads, kvh, hd, pos - w)
        assert np.array_equal(got, want), w
    # a one-position window is that position's value row, per kv head
    got = zo.attention(q, k, v, heads, kvh, hd, pos, pos).reshape(heads, hd)
    vr = v[pos * kv_dim:(pos + 1) * kv_dim].reshape(kvh, hd)
    for h in range(heads):
        assert np.allclose(got[h], vr[h // (heads // kvh)], rtol=0, atol=1e-6)
