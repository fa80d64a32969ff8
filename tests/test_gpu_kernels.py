"""GPU parity of the primitive kernels against the CPU oracle, through the C ABI.

Bars: dequantised weights bit-exact; matvec and attention outputs within
1e-4 relative L2 of the oracle (the tolerance the north star sets for
floating point); argmax/top-k indices exact.
"""
import sys

import numpy as np
import pytest

from oracle import zo
from zhip import hip, synth
from zhip.gguf import F16, F32, IQ4_XS, Q3_K, Q4_K, Q6_K, Q8_0, row_bytes

pytestmark = pytest.mark.gpu
REL_L2 = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def random_weights(ttype, rows, cols, seed):
    q = np.zeros(row_bytes(ttype, cols) * rows, np.uint8)
    synth.fill_tensor(q, ttype, rows, cols, seed=seed)
    return q


def special_blocks(ttype, rows, cols, seed):
    """Random bytes with the d/dmin fields forced to special binary16 values
    (subnormal, max normal, negative zero) and max 6-bit scales."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, row_bytes(ttype, cols) * rows, dtype=np.uint8)
    specials = [0x0001, 0x03FF, 0x7BFF, 0x8000, 0x3C00, 0x0400, 0xFBFF]
    nb = {Q4_K: 144, Q6_K: 210, Q8_0: 34, Q3_K: 110, IQ4_XS: 136}[ttype]
    doff = {Q4_K: [0, 2], Q6_K: [208], Q8_0: [0], Q3_K: [108], IQ4_XS: [0]}[ttype]
    for i in range(len(q) // nb):
        for o in doff:
            v = specials[(i + o) % len(specials)]
            q[i * nb + o] = v & 0xFF
            q[i * nb + o + 1] = v >> 8
    return q


@pytest.mark.parametrize("ttype", [Q4_K, Q6_K, Q8_0, Q3_K, IQ4_XS, F16])
@pytest.mark.parametrize("kind", ["quantized", "special"])
def test_dequant_bit_exact(hip_ctx, ttype, kind):
    rows, cols = 24, 1024
    say(f"dequant {ttype} {kind}")
    q = random_weights(ttype, rows, cols, 3) if kind == "quantized" or ttype == F16 else special_blocks(ttype, rows, cols, 4)
    want = zo.dequantize(ttype, q, rows, cols)
    mb = hip_ctx.buffer(q)
    out = hip_ctx.empty(rows * cols * 4)
    hip_ctx.dequantize(ttype, mb, out, rows, cols)
    got = out.read(np.float32).reshape(rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def fill_q4k_matrix(rows, cols):
    """fillQ4KMatrix (runtime/metal_backend_test.zig:894-924)."""
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


def test_q4k_reference_matrix(hip_ctx):
    # the reference's Q4_K matvec test (runtime/metal_backend_test.zig:7-45)
    rows, cols = 3, 512
    m = fill_q4k_matrix(rows, cols)
    x = ((np.arange(cols) % 17 - 8) * 0.125 + 0.1).astype(np.float32)
    want = zo.matvec(Q4_K, m, rows, cols, x)
    y = hip_ctx.empty(rows * 4)
    hip_ctx.matvec(Q4_K, hip_ctx.buffer(m), hip_ctx.buffer(x), y, rows, cols)
    assert rel_l2(y.read(), want) < REL_L2
    deq = hip_ctx.empty(rows * cols * 4)
    hip_ctx.dequantize(Q4_K, hip_ctx.buffer(m), deq, rows, cols)
    assert np.array_equal(deq.read().view(np.uint32), zo.dequantize(Q4_K, m, rows, cols).ravel().view(np.uint32))


# cols 64..16384 cover every team width (1..256 lanes) and both partial
# (slots < team) and exact teams; rows cover ragged workgroup tails.
# Rows longer than one team (16384 values) run as column windows, the first
# stored or added as asked and the rest added: 16640 (a window of 256 after
# a full one), 28672 (Llama-70B-sized down rows) and 40960 (three windows).
SHAPES = [(7, 64), (33, 128), (96, 256), (50, 512), (300, 1024), (4096, 4096), (14336, 4096), (4096, 14336),
          (1024, 2048), (4096, 12288), (129, 8192), (65, 16384), (128256, 4096), (70, 16640), (300, 28672),
          (33, 40960)]
BLOCK_VALUES = {Q4_K: 256, Q6_K: 256, Q3_K: 256, IQ4_XS: 256, Q8_0: 32, F16: 1, F32: 1}


@pytest.mark.parametrize("ttype", [Q4_K, Q6_K, Q8_0, Q3_K, IQ4_XS, F16, F32])
@pytest.mark.parametrize("shape", SHAPES)
def test_matvec_parity(hip_ctx, ttype, shape):
    rows, cols = shape
    if ttype in (F16, F32, Q3_K, IQ4_XS) and rows * cols > 4096 * 4096:
        pytest.skip("large dense/extra-format shapes are covered by the smaller cases")
    if cols % BLOCK_VALUES[ttype]:
        pytest.skip("row length is not a whole number of blocks of this format")
    say(f"matvec {ttype} {rows}x{cols}")
    q = random_weights(ttype, rows, cols, rows + cols)
    x = synth.normal_row(77, 0, cols, 0.0, 1.0)
    want = zo.matvec(ttype, q, rows, cols, x, threads=8)
    mb, xb, yb = hip_ctx.buffer(q), hip_ctx.buffer(x), hip_ctx.empty(rows * 4)
    hip_ctx.matvec(ttype, mb, xb, yb, rows, cols)
    assert rel_l2(yb.read(), want) < REL_L2
    # _add variant and output offset (to_dst)
    base = synth.normal_row(78, 0, rows + 3, 0.0, 1.0)
    yb2 = hip_ctx.buffer(base)
    hip_ctx.matvec(ttype, mb, xb, yb2, rows, cols, add=True, y_off=12)
    got = yb2.read()
    assert np.array_equal(got[:3], base[:3])
    assert rel_l2(got[3:], base[3:] + want) < REL_L2


def test_silu_down_add_long_rows(hip_ctx):
    # the SiLU prologue over column windows: silu(gate) * up, both inputs offset per window
    rows, cols = 100, 20480
    q = random_weights(Q4_K, rows, cols, 5)
    g = synth.normal_row(3, 0, cols, 0.0, 1.0)
    u = synth.normal_row(4, 0, cols, 0.0, 1.0)
    base = synth.normal_row(5, 0, rows, 0.0, 1.0)
    act = zo.silu(g) * u
    want = base + zo.matvec(Q4_K, q, rows, cols, act.astype(np.float32), threads=8)
    out = hip_ctx.buffer(base)
    hip_ctx.matvec_silu_down_add(Q4_K, hip_ctx.buffer(q), hip_ctx.buffer(g), hip_ctx.buffer(u), out, rows, cols)
    assert rel_l2(out.read(), want) < REL_L2


def test_q6k_output_head_argmax(hip_ctx):
    # runtime/metal_backend_test.zig:448-507: argmax over a 32000-row Q6_K head
    rows, cols = 32000, 2048
    say("argmax head")
    q = random_weights(Q6_K, rows, cols, 5)
    x = ((np.arange(cols) % 41 - 20) * 0.015625 + 0.02).astype(np.float32)
    want = zo.matvec(Q6_K, q, rows, cols, x, threads=8)
    state = hip_ctx.buffer(np.array([0, 0xFFFFFFFF], np.uint32))
    hip_ctx.matvec_argmax(Q6_K, hip_ctx.buffer(q), hip_ctx.buffer(x), state, rows, cols)
    tok = int(state.read(np.uint32)[1])
    best = int(np.argmax(want))
    assert tok == best or want[tok] >= want[best] - 1e-4 * abs(want[best])


def test_silu_down_add(hip_ctx):
    rows, cols = 2048, 5632
    say("silu_down_add")
    q = random_weights(Q4_K, rows, cols, 11)
    g = synth.normal_row(1, 0, cols, 0.0, 1.0)
    u = synth.normal_row(2, 0, cols, 0.0, 1.0)
    act = zo.silu(g) * u
    base = synth.normal_row(3, 0, rows, 0.0, 1.0)
    want = base + zo.matvec(Q4_K, q, rows, cols, act.astype(np.float32))
    y = hip_ctx.buffer(base)
    hip_ctx.matvec_silu_down_add(Q4_K, hip_ctx.buffer(q), hip_ctx.buffer(g), hip_ctx.buffer(u), y, rows, cols)
    assert rel_l2(y.read(), want) < REL_L2


# Splits hold one or more 64-position chunks: with 256 / kv_heads splits at
# most, (16, 16, 128) and (64, 64, 64) fold several chunks per split (online
# softmax across chunks) from positions 1024 and 256 on.
@pytest.mark.parametrize("heads,kv_heads,hd", [(32, 8, 128), (32, 4, 64), (3, 1, 128), (1, 1, 256), (16, 16, 128),
                                               (64, 64, 64), (3, 1, 96), (24, 8, 96)])
@pytest.mark.parametrize("pos", [0, 1, 63, 64, 65, 200, 1000, 4095])
def test_attention_parity(hip_ctx, heads, kv_heads, hd, pos):
    say(f"attention {heads}/{kv_heads}x{hd} pos {pos}")
    rng = np.random.default_rng(pos * 7 + hd)
    kv_dim = kv_heads * hd
    ctx_len = pos + 1
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = rng.standard_normal(ctx_len * kv_dim).astype(np.float16)
    v = rng.standard_normal(ctx_len * kv_dim).astype(np.float16)
    want = zo.attention(q, k.astype(np.float32), v.astype(np.float32), heads, kv_heads, hd, pos)
    out = hip_ctx.empty(heads * hd * 4)
    hip_ctx.attention(hip_ctx.buffer(q), hip_ctx.buffer(k), hip_ctx.buffer(v), out, heads, kv_heads, hd, kv_dim,
                      ctx_len, pos)
    assert rel_l2(out.read(), want) < REL_L2


# Sliding windows: the reference passes window_start = position + 1 - sliding_window
# (model/loader.zig:1440-1444), any value up to the position; tiles of the
# matrix-core kernel start on a 32-position boundary at or below it and mask
# the positions before it.
@pytest.mark.parametrize("heads,kv_heads,hd", [(32, 8, 128), (32, 4, 64), (3, 1, 96), (1, 1, 256)])
@pytest.mark.parametrize("pos,window", [(300, 37), (300, 100), (4095, 4000), (1000, 1000), (64, 63), (4095, 31)])
def test_attention_window_parity(hip_ctx, heads, kv_heads, hd, pos, window):
    say(f"attention {heads}/{kv_heads}x{hd} pos {pos} window {window}")
    rng = np.random.default_rng(pos * 5 + window)
    kv_dim = kv_heads * hd
    ctx_len = pos + 1
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = rng.standard_normal(ctx_len * kv_dim).astype(np.float16)
    v = rng.standard_normal(ctx_len * kv_dim).astype(np.float16)
    want = zo.attention(q, k.astype(np.float32), v.astype(np.float32), heads, kv_heads, hd, pos, window)
    out = hip_ctx.empty(heads * hd * 4)
    hip_ctx.attention(hip_ctx.buffer(q), hip_ctx.buffer(k), hip_ctx.buffer(v), out, heads, kv_heads, hd, kv_dim,
                      ctx_len, pos, window_start=window)
    assert rel_l2(out.read(), want) < REL_L2


def test_attention_reference_case_head_dim_96(hip_ctx):
    # runtime/metal_backend_test.zig:691-766: 3 query heads on 1 kv head of 96, 5 positions, query at 4, scale
    # 0.125; the reference's expected values come from f32 caches, its kernel reads binary16 ones (tolerance
    # 0.005 absolute); against the binary16 cache the result is held to the kernel bar
    heads, kvh, hd, ctx_len, pos, scale = 3, 1, 96, 5, 4, 0.125
    kv_dim = kvh * hd
    i = np.arange(heads * hd)
    q = (((i % 19) - 9) * 0.07 + 0.02).astype(np.float32)
    j = np.arange(ctx_len * kv_dim)
    k32 = (((j % 17) - 8) * 0.06 - 0.01).astype(np.float32)
    v32 = (((j % 13) - 6) * 0.08 + 0.03).astype(np.float32)
    k16, v16 = k32.astype(np.float16), v32.astype(np.float16)

    def reference(kc, vc):
        kc = kc.astype(np.float64).reshape(ctx_len, hd)[:pos + 1]
        vc = vc.astype(np.float64).reshape(ctx_len, hd)[:pos + 1]
        out = []
        for h in range(heads):
            s = kc @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
            w = np.exp(s - s.max())
            out.append((w / w.sum()) @ vc)
        return np.concatenate(out)

    o = hip_ctx.empty(heads * hd * 4)
    hip_ctx.attention(hip_ctx.buffer(q), hip_ctx.buffer(k16), hip_ctx.buffer(v16), o, heads, kvh, hd, kv_dim, ctx_len,
                      pos, scale=scale)
    got = o.read()
    assert np.max(np.abs(got - reference(k32, v32))) <= 0.005
    assert rel_l2(got, reference(k16, v16)) < REL_L2


def test_attention_layer_base(hip_ctx):
    # the cache of layer 1 starts at layer_base = 1 * ctx * kv_dim (gpu/session.zig:382-383)
    heads, kvh, hd, ctx_len, pos = 8, 2, 64, 100, 70
    kv_dim = kvh * hd
    rng = np.random.default_rng(1)
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = rng.standard_normal(2 * ctx_len * kv_dim).astype(np.float16)
    v = rng.standard_normal(2 * ctx_len * kv_dim).astype(np.float16)
    lb = ctx_len * kv_dim
    want = zo.attention(q, k[lb:].astype(np.float32), v[lb:].astype(np.float32), heads, kvh, hd, pos)
    out = hip_ctx.empty(heads * hd * 4)
    hip_ctx.attention(hip_ctx.buffer(q), hip_ctx.buffer(k), hip_ctx.buffer(v), out, heads, kvh, hd, kv_dim, ctx_len,
                      pos, layer_base=lb)
    assert rel_l2(out.read(), want) < REL_L2


@pytest.mark.parametrize("style", [0, 1])
def test_rope_and_store(hip_ctx, style):
    say(f"rope {style}")
    rng = np.random.default_rng(2)
    v = rng.standard_normal(8 * 128).astype(np.float32)
    for pos in (0, 5, 4095, 16000):
        want = zo.rope(v, 8, 128, 128, pos, 500000.0, style)
        b = hip_ctx.buffer(v)
        hip_ctx.rope(b, 8, 128, 128, pos, 500000.0, style)
        assert rel_l2(b.read(), want) < REL_L2
    # partial rotary and rope-to-dst (runtime/metal_backend_test.zig:768-870)
    src = ((np.arange(16) - 7) * 0.125 + 0.05).astype(np.float32)
    want = zo.rope(src, 2, 8, 6, 3, 10000.0, style)
    dst = hip_ctx.buffer(np.full(24, -9.0, np.float32))
    hip_ctx.rope_to_dst(hip_ctx.buffer(src), dst, 20, 2, 8, 6, 3, 10000.0, style)
    got = dst.read()
    assert np.all(got[:5] == -9.0) and np.all(got[21:] == -9.0)
    assert np.max(np.abs(got[5:21] - want)) < 5e-4
    kvh = hip_ctx.empty(64 * 2)
    hip_ctx.store_kv_half(hip_ctx.buffer(v[:32]), kvh, 32, 32)
    assert np.array_equal(kvh.read(np.float16)[32:], v[:32].astype(np.float16))


def test_norms_and_elementwise(hip_ctx):
    rng = np.random.default_rng(4)
    x = rng.standard_normal(4096).astype(np.float32) * 2
    w = rng.standard_normal(4096).astype(np.float32)
    out = hip_ctx.empty(4096 * 4)
    hip_ctx.rms_norm(hip_ctx.buffer(x), hip_ctx.buffer(w), out, 4096, 1e-5)
    assert rel_l2(out.read(), zo.rms_norm(x, w, 1e-5)) < REL_L2
    qk = rng.standard_normal(32 * 128).astype(np.float32)
    wn = rng.standard_normal(128).astype(np.float32)
    out2 = hip_ctx.empty(32 * 128 * 4)
    hip_ctx.rms_norm_per_head(hip_ctx.buffer(qk), hip_ctx.buffer(wn), out2, 32, 128, 1e-6)
    assert rel_l2(out2.read(), zo.rms_norm_per_head(qk, wn, 32, 128, 1e-6)) < REL_L2
    g, u = rng.standard_normal(5000).astype(np.float32), rng.standard_normal(5000).astype(np.float32)
    gb = hip_ctx.buffer(g)
    hip_ctx.silu_mul(gb, hip_ctx.buffer(u), 5000)
    assert rel_l2(gb.read(), zo.silu(g) * u) < REL_L2
    tok = hip_ctx.empty(4)
    hip_ctx.argmax(hip_ctx.buffer(np.array([-1.0, 4.0, 2.5, 4.5, 3.0], np.float32)), tok, 5)
    assert tok.read(np.uint32)[0] == 3
    hip_ctx.argmax(hip_ctx.buffer(np.array([1.0, 7.0, 7.0, 2.0], np.float32)), tok, 4)
    assert tok.read(np.uint32)[0] == 1


def test_topk_and_routing(hip_ctx):
    # runtime/metal_backend_test.zig:47-71
    ent = hip_ctx.empty(3 * 8)
    hip_ctx.topk(hip_ctx.buffer(np.array([0.2, 1.5, -2.0, 1.0, 3.0, 0.4, 1.5, -1.0], np.float32)), ent, 8, 3)
    e = ent.read(np.uint32).reshape(3, 2)
    assert list(e[:, 0]) == [4, 1, 6]
    assert list(e[:, 1].view(np.float32)) == [3.0, 1.5, 1.5]
    rng = np.random.default_rng(6)
    logits = rng.standard_normal(256).astype(np.float32)
    ent8 = hip_ctx.empty(8 * 8)
    hip_ctx.topk(hip_ctx.buffer(logits), ent8, 256, 8)
    hip_ctx.normalize_topk(ent8, 8, True, True, 1.0)
    got = ent8.read(np.uint32).reshape(8, 2)
    idx, w = zo.select_topk(zo.softmax(logits), 8)
    assert list(got[:, 0]) == list(idx)
    assert rel_l2(got[:, 1].view(np.float32), zo.normalize_positive(w)) < REL_L2


@pytest.mark.parametrize("ttype", [IQ4_XS, Q3_K])
def test_indexed_expert_matvec(hip_ctx, ttype):
    # expert rows are offset by expert_id * rows_per_expert (matvec.metal:2566-2660)
    n_exp, rpe, cols = 16, 512, 2048
    say(f"indexed {ttype}")
    q = random_weights(ttype, n_exp * rpe, cols, 21)
    x = synth.normal_row(5, 0, cols, 0.0, 1.0)
    rb = row_bytes(ttype, cols)
    entries = np.array([[11, 0], [3, 0]], np.uint32)
    entries[:, 1] = np.array([0.75, -1.5], np.float32).view(np.uint32)
    eb, mb, xb = hip_ctx.buffer(entries), hip_ctx.buffer(q), hip_ctx.buffer(x)
    y = hip_ctx.empty(rpe * 4)
    hip_ctx.indexed_matvec(ttype, mb, xb, y, rpe, cols, eb, 0, rpe)
    want = zo.matvec(ttype, q[11 * rpe * rb:12 * rpe * rb], rpe, cols, x)
    assert rel_l2(y.read(), want) < REL_L2
    base = synth.normal_row(6, 0, rpe, 0.0, 1.0)
    y2 = hip_ctx.buffer(base)
    hip_ctx.indexed_matvec(ttype, mb, xb, y2, rpe, cols, eb, 1, rpe, add_weighted=True)
    want2 = base + np.float32(-1.5) * zo.matvec(ttype, q[3 * rpe * rb:4 * rpe * rb], rpe, cols, x)
    assert rel_l2(y2.read(), want2) < REL_L2
    # an expert id past the matrix reads nothing and leaves the output alone
    bad = hip_ctx.buffer(np.array([[n_exp, 0]], np.uint32))
    y3 = hip_ctx.buffer(base)
    hip_ctx.indexed_matvec(ttype, mb, xb, y3, rpe, cols, bad, 0, rpe, add_weighted=True)
    assert np.array_equal(y3.read(), base)


def test_invalid_arguments_are_rejected(hip_ctx):
    x = hip_ctx.empty(4096 * 4)
    m = hip_ctx.empty(144)  # one block only
    y = hip_ctx.empty(4)
    with pytest.raises(hip.HipError) as e:
        hip_ctx.matvec(Q4_K, m, x, y, 16, 4096)
    assert e.value.status == 6
    with pytest.raises(hip.HipError):
        hip_ctx.matvec(Q4_K, m, x, y, 1, 300)  # not a block multiple
    with pytest.raises(hip.HipError):
        hip_ctx.attention(x, m, m, y, 32, 8, 80, 640, 10, 3)  # head_dim 80 unsupported
