// zh_quant.h -- device-side GGUF block decoders for gfx950.
//
// Every format is processed in "slots" of 64 weights of one row.  A lane owns
// one slot for every row it visits, so its 64 activation values stay in VGPRs
// across rows.  The 64 values of a slot always come as 4 runs of 16
// contiguous activations: run w starts at x_base(slot) + w * x_stride.
//
// Block layouts and value formulas follow the reference decoders:
//   Q4_K  model/loader.zig:3647-3726, getScaleMinK4 :3814-3825
//   Q6_K  model/loader.zig:3728-3812
//   Q8_0  model/loader.zig:3589-3617
//   Q3_K  model/quant_extra.zig:45-126, expandQ3KScales :248-279
//   IQ4_XS model/quant_extra.zig:191-246, kvalues_iq4nl :8
// The matvec dots factor the per-block scales out of the 16/32-value sums
// (as the reference's own dotQ4KRow / dotQ6KRow do) and form those sums with
// integer dot products against a fixed-point copy of the activations (XDig);
// unsigned-offset codes (Q6_K q+32, Q3_K q+4) are corrected with per-run
// activation sums.
// The dequant_* functions reproduce the reference's exact binary32 operation
// order (no contraction) and are bit-exact with the CPU decoder.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zh {

enum Fmt : int { F32 = 0, F16 = 1, Q8_0 = 8, Q3_K = 11, Q4_K = 12, Q6_K = 14, IQ4_XS = 23 };

__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
__device__ __forceinline__ uint2 ld8(const uint8_t *p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
__device__ __forceinline__ uint32_t ld4(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
__device__ __forceinline__ uint32_t ld2(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}
// binary16 bits -> f32 (exact, subnormals included)
__device__ __forceinline__ float h2f(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)(bits & 0xFFFFu))); }
// unsigned byte k of w as f32 (v_cvt_f32_ubyteK)
__device__ __forceinline__ float ub(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }
__device__ __forceinline__ float sb(uint32_t w, int k) { return (float)(int8_t)((w >> (8 * k)) & 0xFFu); }
__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t width) {
    return __builtin_amdgcn_ubfe(v, off, width);
}
// Hides the known bits of v from the optimiser so byte extracts of a masked
// word select v_cvt_f32_ubyte{1,2,3} directly instead of v_bfe + ubyte0.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

template <int F> struct Geom;
template <> struct Geom<Q4_K> {
    static constexpr int kValues = 256, kBytes = 144, kSlotsPerBlock = 4;
    __device__ static int x_base(int s) { return (s >> 2) * 256 + (s & 3) * 64; }
    static constexpr int kXStride = 16;
    // slot s and run w of the 16-value run R (x[16R .. 16R + 15])
    __device__ static void run_slot(int R, int &s, int &w) { s = (R >> 4) * 4 + ((R >> 2) & 3), w = R & 3; }
};
template <> struct Geom<Q6_K> {
    static constexpr int kValues = 256, kBytes = 210, kSlotsPerBlock = 4;
    __device__ static int x_base(int s) { return (s >> 2) * 256 + ((s >> 1) & 1) * 128 + (s & 1) * 16; }
    static constexpr int kXStride = 32;
    __device__ static void run_slot(int R, int &s, int &w) {
        s = (R >> 4) * 4 + ((R >> 3) & 1) * 2 + (R & 1), w = (R & 7) >> 1;
    }
};
template <> struct Geom<Q3_K> {
    static constexpr int kValues = 256, kBytes = 110, kSlotsPerBlock = 4;
    __device__ static int x_base(int s) { return (s >> 2) * 256 + ((s >> 1) & 1) * 128 + (s & 1) * 16; }
    static constexpr int kXStride = 32;
    __device__ static void run_slot(int R, int &s, int &w) {
        s = (R >> 4) * 4 + ((R >> 3) & 1) * 2 + (R & 1), w = (R & 7) >> 1;
    }
};
template <> struct Geom<IQ4_XS> {
    static constexpr int kValues = 256, kBytes = 136, kSlotsPerBlock = 4;
    __device__ static int x_base(int s) { return (s >> 2) * 256 + (s & 3) * 64; }
    static constexpr int kXStride = 16;
    __device__ static void run_slot(int R, int &s, int &w) { s = (R >> 4) * 4 + ((R >> 2) & 3), w = R & 3; }
};
template <> struct Geom<Q8_0> {
    static constexpr int kValues = 32, kBytes = 34, kSlotsPerBlock = 1;  // a slot spans 2 blocks
    __device__ static int x_base(int s) { return s * 64; }
    static constexpr int kXStride = 16;
    __device__ static void run_slot(int R, int &s, int &w) { s = R >> 2, w = R & 3; }
};
template <> struct Geom<F16> {
    static constexpr int kValues = 1, kBytes = 2, kSlotsPerBlock = 1;
    __device__ static int x_base(int s) { return s * 64; }
    static constexpr int kXStride = 16;
};
template <> struct Geom<F32> {
    static constexpr int kValues = 1, kBytes = 4, kSlotsPerBlock = 1;
    __device__ static int x_base(int s) { return s * 64; }
    static constexpr int kXStride = 16;
};

// ---------------- activation slots ----------------
//
// The float formats (F16, F32) keep a lane's 64 activations as f32 (XSlot).
// The quantized formats use XDig: the lane's activations as 22-bit fixed
// point, x_i ~= scale * (65536 * d2 + 256 * d1 + d0), with a per-lane
// power-of-two scale chosen from max|x| and balanced base-256 digits
// d0, d1 in [-128, 127], d2 in [-64, 64].  A quant block's integer codes
// then meet the digits in v_dot4_i32_i8 (four products per instruction,
// exact int32 sums), and each sub-block's three digit sums are recombined in
// f32.  The only approximation is the fixed-point rounding of x, at most
// 2^-22 * max|x| per value (the size of binary32 rounding of the largest
// term); sums of products are exact before the recombination.

struct XSlot {
    float v[64];
    float sum[4];
};

struct XDig {
    uint32_t d[3][16];  // digit j of slot values 4c..4c+3, one signed byte each, in d[j][c]
    float scale;        // 2^-k (non-finite when an activation is)
    float sum[4];       // per-run f32 sums of the activations
};

template <int F> struct XOf { using type = XDig; };
template <> struct XOf<F16> { using type = XSlot; };
template <> struct XOf<F32> { using type = XSlot; };
template <int F> using XOf_t = typename XOf<F>::type;

__device__ __forceinline__ void run_sums(const float (&v)[64], float (&sum)[4]) {
#pragma unroll
    for (int w = 0; w < 4; w++) {
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < 16; k++) t += v[16 * w + k];
        sum[w] = t;
    }
}

__device__ __forceinline__ void to_slot(const float (&v)[64], XSlot &xs) {
#pragma unroll
    for (int i = 0; i < 64; i++) xs.v[i] = v[i];
    run_sums(v, xs.sum);
}

// The three balanced base-256 digit words of four activations scaled by 2^k.
__device__ __forceinline__ void digits4(float v0, float v1, float v2, float v3, int k, uint32_t &d0, uint32_t &d1,
                                        uint32_t &d2) {
    // u = xi + 0x808080 has the balanced digits + 128 as its bytes 0..2
    const uint32_t u0 = (uint32_t)(int)ldexpf(v0, k) + 0x808080u, u1 = (uint32_t)(int)ldexpf(v1, k) + 0x808080u;
    const uint32_t u2 = (uint32_t)(int)ldexpf(v2, k) + 0x808080u, u3 = (uint32_t)(int)ldexpf(v3, k) + 0x808080u;
    const uint32_t a = __builtin_amdgcn_perm(u1, u0, 0x05010400u);   // u0.b0 u1.b0 u0.b1 u1.b1
    const uint32_t b = __builtin_amdgcn_perm(u3, u2, 0x05010400u);   // u2.b0 u3.b0 u2.b1 u3.b1
    const uint32_t c2 = __builtin_amdgcn_perm(u1, u0, 0x07030602u);  // u0.b2 u1.b2 u0.b3 u1.b3
    const uint32_t e2 = __builtin_amdgcn_perm(u3, u2, 0x07030602u);
    d0 = __builtin_amdgcn_perm(b, a, 0x05040100u) ^ 0x80808080u;
    d1 = __builtin_amdgcn_perm(b, a, 0x07060302u) ^ 0x80808080u;
    d2 = __builtin_amdgcn_perm(e2, c2, 0x05040100u) ^ 0x80808080u;
}

// Scale exponent k of a slot: |v * 2^k| < 2^22 for max|v| = m; and the scale
// 2^-k, or NaN when an activation (m, or the slot total tot) is not finite
// (the digits cannot carry it, so every dot is NaN).
__device__ __forceinline__ int slot_exponent(float m) { return 22 - __builtin_amdgcn_frexp_expf(m); }
__device__ __forceinline__ float slot_scale(float m, float tot, int k) {
    return (m <= 3.4028235e38f && fabsf(tot) <= 3.4028235e38f) ? ldexpf(1.0f, -k) : __builtin_nanf("");
}

__device__ __forceinline__ void to_slot(const float (&v)[64], XDig &xd) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 64; i++) m = fmaxf(m, fabsf(v[i]));
    // m = f * 2^e with f in [0.5, 1): |v * 2^(22 - e)| < 2^22
    const int k = slot_exponent(m);
    run_sums(v, xd.sum);
    const float tot = (xd.sum[0] + xd.sum[1]) + (xd.sum[2] + xd.sum[3]);
    xd.scale = slot_scale(m, tot, k);
#pragma unroll
    for (int c = 0; c < 16; c++) digits4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3], k, xd.d[0][c], xd.d[1][c], xd.d[2][c]);
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Three-digit integer dot of 4 code words with slot words c0..c0+3 of xd,
// recombined to f32 (without the scale).
struct Dig3 {
    int a0 = 0, a1 = 0, a2 = 0;
    __device__ __forceinline__ void add(uint32_t q, const XDig &xd, int c) {
        a0 = sdot4(q, xd.d[0][c], a0);
        a1 = sdot4(q, xd.d[1][c], a1);
        a2 = sdot4(q, xd.d[2][c], a2);
    }
    __device__ __forceinline__ float value() const {
        return fmaf((float)a2, 65536.f, fmaf((float)a1, 256.f, (float)a0));
    }
};

// ---------------- slots: raw load (registers) + dot ----------------
//
// slot_load<F>(row, s) issues the 16-byte loads of slot s of `row` and
// returns the raw words; slot_dot<F>(raw, s, xs) decodes them and returns
// dot(64 weights, x).  Splitting the two lets a kernel keep the next rows'
// loads in flight while it computes the current one.

template <int F> struct Raw;
template <> struct Raw<Q4_K> { uint4 hd, qa, qb; };
template <> struct Raw<Q6_K> { uint4 qa, qb, qh; uint2 sc; uint32_t d; };
template <> struct Raw<Q8_0> { uint4 a, b, c, e; uint32_t f; };
template <> struct Raw<Q3_K> { uint4 hm, qs; uint32_t r0, r1, r2, d; };
template <> struct Raw<IQ4_XS> { uint4 q0, q1; uint32_t dsh, sl; };
template <> struct Raw<F16> { uint4 w[8]; };
template <> struct Raw<F32> { uint4 w[16]; };

template <int F> __device__ __forceinline__ Raw<F> slot_load(const uint8_t *__restrict__ row, int s);
template <int F> __device__ __forceinline__ float slot_dot(const Raw<F> &r, int s, const XOf_t<F> &xs);

// Q4_K: slot = (block b, group g): 32 qs bytes -> sub-block 2g (low nibbles) and 2g+1 (high).
template <> __device__ __forceinline__ Raw<Q4_K> slot_load<Q4_K>(const uint8_t *__restrict__ row, int s) {
    const uint8_t *blk = row + (s >> 2) * 144;
    const int g = s & 3;
    return {ld16(blk), ld16(blk + 16 + 32 * g), ld16(blk + 32 + 32 * g)};
}
template <> __device__ __forceinline__ float slot_dot<Q4_K>(const Raw<Q4_K> &r, int s, const XDig &xs) {
    const int g = s & 3;
    const uint4 hd = r.hd;
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    // getScaleMinK4 for j = 2g, 2g+1 with lane-uniform formulas
    const bool lo = g < 2;
    const uint32_t a_sc = lo ? hd.y : hd.w, a_m = lo ? hd.z : hd.w;
    const uint32_t o0 = lo ? 16u * g : 16u * (g - 2), o1 = o0 + 8u;
    const uint32_t wa = lo ? 6u : 4u, wb = lo ? 0u : 2u, om = lo ? 0u : 4u;
    const uint32_t sc0 = bfe(a_sc, o0, wa) | (bfe(hd.y, o0 + 6, wb) << 4);
    const uint32_t m0 = bfe(a_m, o0 + om, wa) | (bfe(hd.z, o0 + 6, wb) << 4);
    const uint32_t sc1 = bfe(a_sc, o1, wa) | (bfe(hd.y, o1 + 6, wb) << 4);
    const uint32_t m1 = bfe(a_m, o1 + om, wa) | (bfe(hd.z, o1 + 6, wb) << 4);
    const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
    Dig3 lo_acc, hi_acc;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        lo_acc.add(q[k] & 0x0F0F0F0Fu, xs, k);
        hi_acc.add((q[k] >> 4) & 0x0F0F0F0Fu, xs, 8 + k);
    }
    const float d1 = d * (float)sc0, mm1 = dmin * (float)m0, d2 = d * (float)sc1, mm2 = dmin * (float)m1;
    float res = fmaf(d1, lo_acc.value(), d2 * hi_acc.value()) * xs.scale;
    res = fmaf(-mm1, xs.sum[0] + xs.sum[1], res);
    res = fmaf(-mm2, xs.sum[2] + xs.sum[3], res);
    return res;
}

// Q6_K: slot = (block b, half h, l0 in {0,16}): ql[64h+l0..], ql[64h+32+l0..], qh[32h+l0..].
template <> __device__ __forceinline__ Raw<Q6_K> slot_load<Q6_K>(const uint8_t *__restrict__ row, int s) {
    const uint8_t *blk = row + (s >> 2) * 210;
    const int h = (s >> 1) & 1, l0 = (s & 1) * 16;
    return {ld16(blk + 64 * h + l0), ld16(blk + 64 * h + 32 + l0), ld16(blk + 128 + 32 * h + l0),
            ld8(blk + 192 + 8 * h), ld2(blk + 208)};
}
template <> __device__ __forceinline__ float slot_dot<Q6_K>(const Raw<Q6_K> &r, int s, const XDig &xs) {
    const float d = h2f(r.d);
    const int sb0 = s & 1;
    const uint32_t a[4] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w}, bq[4] = {r.qb.x, r.qb.y, r.qb.z, r.qb.w};
    const uint32_t hh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    Dig3 acc[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        // codes q + 32 in 0..63, one run (sub-block of 16) per word group
        acc[0].add((a[k] & 0x0F0F0F0Fu) | ((hh[k] & 0x03030303u) << 4), xs, k);
        acc[1].add((bq[k] & 0x0F0F0F0Fu) | ((hh[k] & 0x0C0C0C0Cu) << 2), xs, 4 + k);
        acc[2].add(((a[k] >> 4) & 0x0F0F0F0Fu) | (hh[k] & 0x30303030u), xs, 8 + k);
        acc[3].add(((bq[k] >> 4) & 0x0F0F0F0Fu) | ((hh[k] >> 2) & 0x30303030u), xs, 12 + k);
    }
    // sc[8h + l0/16 + 2w]: byte sb0 (+2) of sc.x (w = 0, 1) and sc.y (w = 2, 3)
    const float s0 = d * sb(r.sc.x, sb0), s1 = d * sb(r.sc.x, sb0 + 2);
    const float s2 = d * sb(r.sc.y, sb0), s3 = d * sb(r.sc.y, sb0 + 2);
    float res = s0 * fmaf(acc[0].value(), xs.scale, -32.f * xs.sum[0]);
    res = fmaf(s1, fmaf(acc[1].value(), xs.scale, -32.f * xs.sum[1]), res);
    res = fmaf(s2, fmaf(acc[2].value(), xs.scale, -32.f * xs.sum[2]), res);
    res = fmaf(s3, fmaf(acc[3].value(), xs.scale, -32.f * xs.sum[3]), res);
    return res;
}

// Q8_0: slot = 2 consecutive 34-byte blocks (68 bytes, 4-byte aligned within a row).
template <> __device__ __forceinline__ Raw<Q8_0> slot_load<Q8_0>(const uint8_t *__restrict__ row, int s) {
    const uint8_t *p = row + 68 * s;
    return {ld16(p), ld16(p + 16), ld16(p + 32), ld16(p + 48), ld4(p + 64)};
}
template <> __device__ __forceinline__ float slot_dot<Q8_0>(const Raw<Q8_0> &r, int s, const XDig &xs) {
    const uint32_t w[17] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c.x,
                            r.c.y, r.c.z, r.c.w, r.e.x, r.e.y, r.e.z, r.e.w, r.f};
    const float d0 = h2f(w[0]), d1 = h2f(w[8] >> 16);
    Dig3 b0, b1;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        b0.add(__builtin_amdgcn_alignbyte(w[m + 1], w[m], 2), xs, m);  // block 0 quants: bytes 2..33
        b1.add(w[9 + m], xs, 8 + m);                                    // block 1 quants: bytes 36..67
    }
    return fmaf(d1, b1.value(), d0 * b0.value()) * xs.scale;
}

// Q3_K: slot = (block b, half h, 16-group sh): qs[32h+16sh..], hmask[16sh..], 4 shifts.
template <> __device__ __forceinline__ Raw<Q3_K> slot_load<Q3_K>(const uint8_t *__restrict__ row, int s) {
    const uint8_t *blk = row + (s >> 2) * 110;
    const int h = (s >> 1) & 1, sh = s & 1;
    return {ld16(blk + 16 * sh), ld16(blk + 32 + 32 * h + 16 * sh), ld4(blk + 96), ld4(blk + 100), ld4(blk + 104),
            ld2(blk + 108)};
}
template <> __device__ __forceinline__ float slot_dot<Q3_K>(const Raw<Q3_K> &r, int s, const XDig &xs) {
    const int h = (s >> 1) & 1, sh = s & 1;
    const float dall = h2f(r.d);
    const uint32_t hmw[4] = {r.hm.x, r.hm.y, r.hm.z, r.hm.w}, qw[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
    Dig3 acc[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // (q + 4) = low 2 bits | high-mask bit << 2, per byte
            acc[j].add(((qw[k] >> (2 * j)) & 0x03030303u) | (((hmw[k] >> (4 * h + j)) & 0x01010101u) << 2), xs,
                       4 * j + k);
        }
    }
    float res = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        // scale index i = 8h + 2j + sh (expandQ3KScales)
        const int i = 8 * h + 2 * j + sh, qd = i & 3, grp = i >> 2;
        const uint32_t lowsrc = (grp & 1) ? r.r1 : r.r0;
        const uint32_t low4 = bfe(lowsrc, 8 * qd + 4 * (grp >> 1), 4);
        const uint32_t hi2 = bfe(r.r2, 8 * qd + 2 * grp, 2);
        const float sc = (float)((int)(low4 | (hi2 << 4)) - 32);
        res = fmaf(dall * sc, fmaf(acc[j].value(), xs.scale, -4.f * xs.sum[j]), res);
    }
    return res;
}

__device__ __constant__ static const float kIq4nl[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                                                         1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};

// kvalues_iq4nl as integers (the same table as kIq4nl)
constexpr int kIq4Int[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// kvalues_iq4nl as signed bytes, 4 entries per word, for register table lookups with v_perm
#define ZH_IQ4_B(v, i) (((uint32_t)(uint8_t)(int8_t)(v)) << (8 * (i)))
#define ZH_IQ4_W(w) \
    (ZH_IQ4_B(kIq4Int[4 * (w)], 0) | ZH_IQ4_B(kIq4Int[4 * (w) + 1], 1) | ZH_IQ4_B(kIq4Int[4 * (w) + 2], 2) | \
     ZH_IQ4_B(kIq4Int[4 * (w) + 3], 3))
#define ZH_IQ4_T0 ZH_IQ4_W(0)
#define ZH_IQ4_T1 ZH_IQ4_W(1)
#define ZH_IQ4_T2 ZH_IQ4_W(2)
#define ZH_IQ4_T3 ZH_IQ4_W(3)

// Looks up 4 nibbles (one per byte of n, each 0..15) in kvalues_iq4nl (signed bytes).
__device__ __forceinline__ uint32_t iq4_lookup4(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(ZH_IQ4_T1, ZH_IQ4_T0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(ZH_IQ4_T3, ZH_IQ4_T2, sel);
    // byte i of the result: lo.byte[i] (selector i) or hi.byte[i] (selector 4 + i) by bit 3 of the nibble
    const uint32_t pick = 0x03020100u + ((n & 0x08080808u) >> 1);
    return __builtin_amdgcn_perm(hi, lo, pick);
}

// IQ4_XS: slot = (block b, sub-block pair k): sub-blocks 2k, 2k+1.
template <> __device__ __forceinline__ Raw<IQ4_XS> slot_load<IQ4_XS>(const uint8_t *__restrict__ row, int s) {
    const uint8_t *blk = row + (s >> 2) * 136;
    const int k = s & 3;
    return {ld16(blk + 8 + 32 * k), ld16(blk + 24 + 32 * k), ld4(blk), ld4(blk + 4)};
}
template <> __device__ __forceinline__ float slot_dot<IQ4_XS>(const Raw<IQ4_XS> &r, int s, const XDig &xs) {
    const int k = s & 3;
    const float d = h2f(r.dsh);
    const uint32_t sh = r.dsh >> 16, sl = bfe(r.sl, 8 * k, 8);
    const uint32_t ls0 = (sl & 0xF) | (bfe(sh, 4 * k, 2) << 4), ls1 = (sl >> 4) | (bfe(sh, 4 * k + 2, 2) << 4);
    const uint32_t w0[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w}, w1[4] = {r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    Dig3 a0, a1;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        a0.add(iq4_lookup4(w0[c] & 0x0F0F0F0Fu), xs, c);
        a0.add(iq4_lookup4((w0[c] >> 4) & 0x0F0F0F0Fu), xs, 4 + c);
        a1.add(iq4_lookup4(w1[c] & 0x0F0F0F0Fu), xs, 8 + c);
        a1.add(iq4_lookup4((w1[c] >> 4) & 0x0F0F0F0Fu), xs, 12 + c);
    }
    return fmaf(d * (float)((int)ls1 - 32), a1.value(), (d * (float)((int)ls0 - 32)) * a0.value()) * xs.scale;
}

template <> __device__ __forceinline__ Raw<F16> slot_load<F16>(const uint8_t *__restrict__ row, int s) {
    Raw<F16> r;
    const uint8_t *p = row + 128 * s;
#pragma unroll
    for (int c = 0; c < 8; c++) r.w[c] = ld16(p + 16 * c);
    return r;
}
template <> __device__ __forceinline__ float slot_dot<F16>(const Raw<F16> &r, int s, const XSlot &xs) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const uint32_t w[4] = {r.w[c].x, r.w[c].y, r.w[c].z, r.w[c].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            acc = fmaf(h2f(w[k]), xs.v[8 * c + 2 * k], acc);
            acc = fmaf(h2f(w[k] >> 16), xs.v[8 * c + 2 * k + 1], acc);
        }
    }
    return acc;
}

template <> __device__ __forceinline__ Raw<F32> slot_load<F32>(const uint8_t *__restrict__ row, int s) {
    Raw<F32> r;
    const uint8_t *p = row + 256 * s;
#pragma unroll
    for (int c = 0; c < 16; c++) r.w[c] = ld16(p + 16 * c);
    return r;
}
template <> __device__ __forceinline__ float slot_dot<F32>(const Raw<F32> &r, int s, const XSlot &xs) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 16; c++) {
        acc = fmaf(__uint_as_float(r.w[c].x), xs.v[4 * c + 0], acc);
        acc = fmaf(__uint_as_float(r.w[c].y), xs.v[4 * c + 1], acc);
        acc = fmaf(__uint_as_float(r.w[c].z), xs.v[4 * c + 2], acc);
        acc = fmaf(__uint_as_float(r.w[c].w), xs.v[4 * c + 3], acc);
    }
    return acc;
}

// ---------------- bit-exact block decode (reference operation order) ----------------

#pragma clang fp contract(off)

__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *s, int &sc, int &m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// Decodes the 256 (or 32 for Q8_0) values of one block into out[].
template <int F> __device__ void dequant_block(const uint8_t *blk, float *out);

template <> __device__ void dequant_block<Q4_K>(const uint8_t *blk, float *out) {
    const float d = h2f(ld2(blk)), dmin = h2f(ld2(blk + 2));
    const uint8_t *sc = blk + 4, *q = blk + 16;
    for (int g = 0; g < 4; g++) {
        int s0, m0, s1, m1;
        scale_min_k4(2 * g, sc, s0, m0);
        scale_min_k4(2 * g + 1, sc, s1, m1);
        const float d1 = __fmul_rn(d, (float)s0), mm1 = __fmul_rn(dmin, (float)m0);
        const float d2 = __fmul_rn(d, (float)s1), mm2 = __fmul_rn(dmin, (float)m1);
        for (int l = 0; l < 32; l++) {
            out[64 * g + l] = __fsub_rn(__fmul_rn(d1, (float)(q[l] & 0x0F)), mm1);
            out[64 * g + 32 + l] = __fsub_rn(__fmul_rn(d2, (float)(q[l] >> 4)), mm2);
        }
        q += 32;
    }
}

template <> __device__ void dequant_block<Q6_K>(const uint8_t *blk, float *out) {
    const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
    const float d = h2f(ld2(blk + 208));
    for (int half = 0; half < 2; half++) {
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            const float a = d * (float)(int8_t)sc[is + 0], b = d * (float)(int8_t)sc[is + 2];
            const float c = d * (float)(int8_t)sc[is + 4], e = d * (float)(int8_t)sc[is + 6];
            out[l + 0] = a * (float)q1;
            out[l + 32] = b * (float)q2;
            out[l + 64] = c * (float)q3;
            out[l + 96] = e * (float)q4;
        }
        out += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

template <> __device__ void dequant_block<Q8_0>(const uint8_t *blk, float *out) {
    const float d = h2f(ld2(blk));
    for (int i = 0; i < 32; i++) out[i] = d * (float)(int8_t)blk[2 + i];
}

template <> __device__ void dequant_block<Q3_K>(const uint8_t *blk, float *out) {
    const uint8_t *hm = blk, *qs = blk + 32, *raw = blk + 96;
    const float dall = h2f(ld2(blk + 108));
    int scv[16];
    for (int i = 0; i < 16; i++) {
        const int qd = i & 3, grp = i >> 2;
        const int low4 = (raw[(grp & 1) * 4 + qd] >> (4 * (grp >> 1))) & 0xF;
        const int hi2 = (raw[8 + qd] >> (2 * grp)) & 3;
        scv[i] = (low4 | (hi2 << 4)) - 32;
    }
    int o = 0, si = 0;
    uint8_t mask = 1;
    for (int h = 0; h < 2; h++) {
        int shift = 0;
        for (int j = 0; j < 4; j++) {
            for (int half16 = 0; half16 < 2; half16++) {
                const float dl = dall * (float)scv[si++];
                for (int l = 0; l < 16; l++) {
                    const int idx = 32 * h + 16 * half16 + l;
                    const int v = (int)((qs[idx] >> shift) & 3) - ((hm[16 * half16 + l] & mask) ? 0 : 4);
                    out[o++] = dl * (float)v;
                }
            }
            shift += 2;
            mask = (uint8_t)(mask << 1);
        }
    }
}

template <> __device__ void dequant_block<IQ4_XS>(const uint8_t *blk, float *out) {
    const float d = h2f(ld2(blk));
    const uint32_t sh = ld2(blk + 2);
    const uint8_t *qs = blk + 8;
    for (int ib = 0; ib < 8; ib++) {
        const int low = (blk[4 + ib / 2] >> (4 * (ib % 2))) & 0x0f;
        const int high = (sh >> (2 * ib)) & 0x03;
        const float dl = d * (float)((low | (high << 4)) - 32);
        for (int j = 0; j < 16; j++) {
            out[32 * ib + j] = dl * kIq4nl[qs[j] & 0x0f];
            out[32 * ib + j + 16] = dl * kIq4nl[qs[j] >> 4];
        }
        qs += 16;
    }
}

// Value i of one block, with the same operation order as dequant_block
// (bit-exact with it); lets one thread decode one value.
template <int F> __device__ float dequant_value(const uint8_t *blk, int i);

template <> __device__ __forceinline__ float dequant_value<Q4_K>(const uint8_t *blk, int i) {
    const int g = i >> 6, hi = (i >> 5) & 1, l = i & 31;
    int sc, m;
    scale_min_k4(2 * g + hi, blk + 4, sc, m);
    const float d1 = __fmul_rn(h2f(ld2(blk)), (float)sc), mm = __fmul_rn(h2f(ld2(blk + 2)), (float)m);
    const uint8_t q = blk[16 + 32 * g + l];
    return __fsub_rn(__fmul_rn(d1, (float)(hi ? q >> 4 : q & 0x0F)), mm);
}

template <> __device__ __forceinline__ float dequant_value<Q6_K>(const uint8_t *blk, int i) {
    const int half = i >> 7, quarter = (i >> 5) & 3, l = i & 31;
    const uint8_t *ql = blk + 64 * half, *qh = blk + 128 + 32 * half, *sc = blk + 192 + 8 * half;
    const uint8_t lq = ql[l + ((quarter & 1) ? 32 : 0)];
    const int nib = (quarter & 2) ? lq >> 4 : lq & 0x0F;
    const int q = (nib | (((qh[l] >> (2 * quarter)) & 3) << 4)) - 32;
    const float sd = __fmul_rn(h2f(ld2(blk + 208)), (float)(int8_t)sc[l / 16 + 2 * quarter]);
    return __fmul_rn(sd, (float)q);
}

template <> __device__ __forceinline__ float dequant_value<Q8_0>(const uint8_t *blk, int i) {
    return __fmul_rn(h2f(ld2(blk)), (float)(int8_t)blk[2 + i]);
}

template <> __device__ __forceinline__ float dequant_value<Q3_K>(const uint8_t *blk, int i) {
    const int h = i >> 7, j = (i >> 5) & 3, half16 = (i >> 4) & 1, l = i & 15;
    const int si = 8 * h + 2 * j + half16, qd = si & 3, grp = si >> 2;
    const uint8_t *raw = blk + 96;
    const int low4 = (raw[(grp & 1) * 4 + qd] >> (4 * (grp >> 1))) & 0xF;
    const int hi2 = (raw[8 + qd] >> (2 * grp)) & 3;
    const int scv = (low4 | (hi2 << 4)) - 32;
    const int idx = 32 * h + 16 * half16 + l;
    const int v = (int)((blk[32 + idx] >> (2 * j)) & 3) - ((blk[16 * half16 + l] & (1 << (4 * h + j))) ? 0 : 4);
    return __fmul_rn(__fmul_rn(h2f(ld2(blk + 108)), (float)scv), (float)v);
}

template <> __device__ __forceinline__ float dequant_value<IQ4_XS>(const uint8_t *blk, int i) {
    const int ib = i >> 5, j = i & 31;
    const int low = (blk[4 + ib / 2] >> (4 * (ib % 2))) & 0x0f;
    const int high = (ld2(blk + 2) >> (2 * ib)) & 0x03;
    const float dl = __fmul_rn(h2f(ld2(blk)), (float)((low | (high << 4)) - 32));
    const uint8_t qb = blk[8 + 16 * ib + (j & 15)];
    return __fmul_rn(dl, kIq4nl[j < 16 ? qb & 0x0f : qb >> 4]);
}

#pragma clang fp contract(on)

}  // namespace zh
