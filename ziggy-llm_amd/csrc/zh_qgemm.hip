// zh_qgemm.hip -- M >= 8 tokens on the matrix cores with exact weight codes
// (Q4_K, Q6_K, Q8_0, IQ4_XS, Q3_K; reduction length a multiple of 256).
//
//   Y[m][n] (=, +=) sum_k W[n][k] X[m][k]
//
// A quantized weight is w = s_b * q (+ an offset for Q4_K), with q a small
// integer code and s_b the scale of its 16- or 32-value sub-block.  The codes
// enter the matrix cores exactly (bf16 represents integers up to 256
// exactly); the scales are applied per sub-block in f32 to the product's
// result:
//     Y[m][n] += s_{n,b} * D_b[m][n]  (- min_{n,b} * sum_{k in b} X[m][k])
// where D_b = sum_{k in b} X[m][k] q[n][k] is one MFMA (two: the activation
// enters as bf16 hi + lo, x = hi + lo to 2^-17 relative).  So a weight is
// never rounded, only the activations are, at 2^-17 -- well inside the
// 1e-4 relative-L2 bar.  Q4_K codes enter as 128 + c, built from their bits
// without a conversion; each product starts from -128 times the sub-block's
// activation sum, which cancels that excess inside the product, and the
// minimum terms of a chunk's eight sub-blocks are two f32 matrix products
// (min / 128 against the same staged sums).
//
// Product layout (v_mfma_f32_16x16x32_bf16 / 16x16x16_bf16, wave64):
// A = activations (row i = token), B = codes (column j = weight row),
// D[token][row]: lane (li = l % 16, lg = l / 16) holds A[li][8 lg .. +7]
// (4 lg .. +3 for 16-value steps), B[8 lg .. +7][li] and D[4 lg + r][li].
// The lane that decodes weight row li's codes therefore also holds row li's
// results and applies row li's scales itself: no scale exchange.
//
// A workgroup (4 wavefronts) takes 64 weight rows (16 per wavefront) of one
// token tile (16 tokens) over its reduction range.  The activations go
// through LDS in stages of up to 2048 values (128 KB of bf16 pieces for 16
// tokens), split once per workgroup.  Each wavefront streams its 16 rows'
// codes chunk by chunk (256 values): the chunk bytes of a row are loaded as
// whole 16-byte windows (consecutive lanes, consecutive windows: every load
// instruction reads a few rows' bytes contiguously) into a ring of R chunks in
// registers, then copied into the wavefront's own LDS image of the 16 rows,
// from which each lane reads the fields of its row in the product layout.  No
// workgroup barrier inside a stage; the ring runs across stages.
#include <cstdlib>

#include "zh_internal.h"
#include "zh_quant.h"

namespace zh {

typedef __bf16 bf8v __attribute__((ext_vector_type(8)));
typedef short s4v __attribute__((ext_vector_type(4)));
typedef float qf4v __attribute__((ext_vector_type(4)));
typedef uint32_t qu4v __attribute__((ext_vector_type(4)));

constexpr int kQRows = 64;    // weight rows per workgroup (16 per wavefront)
constexpr int kQChunk = 256;  // reduction values per staged chunk
constexpr int kNrmStage = 512;  // the longest stage of the deferred-norm (NRM) kernels

struct QGemmParams {
    const uint8_t *w, *w2;  // W row 0 (w2: the up matrix of SWIGLU)
    uint64_t stride;        // bytes per W row
    const float *x;
    float *y;
    int M, N, K, ldx, ldy;
    unsigned long long *argmax;
    // grouped: token tile blockIdx.y is tiles[3 t] = {expert, first, count} of list
    const int *tiles, *list, *ntiles;
    int x_div;
    uint64_t expert_stride;
    int ksplit;  // blockIdx.z takes reduction values [z K / ksplit, (z + 1) K / ksplit); results add atomically
    // Up to three matrices of one format and reduction length in one launch
    // (one input): matrix 0 is w / N / y / ldy, matrices 1 and 2 start at row
    // groups gs[0], gs[1] of the launch's `groups` row groups.
    int groups, nseg;
    const uint8_t *ws[2];
    float *ys[2];
    int Ns[2], ldys[2], gs[2];
    // the input already split (XPlanes; the XP kernels): row r's pieces at
    // xh / xl + r ldxs, its 32-value sums at xsum + r ldxs / 32
    const uint16_t *xh, *xl;
    const float *xsum;
    int ldxs;
    // NRM kernels: the deferred RMSNorm of the input rows -- the products take
    // x * norm_w (per reduction index), and the row's sum of squares of x
    // over this reduction range adds to row_ss[row] (one workgroup per range)
    const float *norm_w;
    float *row_ss;
};

// bf16 bits of two small integers held as f32 (exact: the high halves)
__device__ __forceinline__ uint32_t pack_bf(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}
__device__ __forceinline__ bf8v as_bf8(uint4 v) {
    bf8v r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}
__device__ __forceinline__ s4v as_s4(uint2 v) {
    s4v r;
    __builtin_memcpy(&r, &v, 8);
    return r;
}
// four unsigned byte codes minus an offset -> bf16 x 4
__device__ __forceinline__ uint2 codes_u4(uint32_t a, float off) {
    return {pack_bf(ub(a, 0) - off, ub(a, 1) - off), pack_bf(ub(a, 2) - off, ub(a, 3) - off)};
}
__device__ __forceinline__ uint4 codes_s8(uint32_t a, uint32_t b) {
    return {pack_bf(sb(a, 0), sb(a, 1)), pack_bf(sb(a, 2), sb(a, 3)), pack_bf(sb(b, 0), sb(b, 1)),
            pack_bf(sb(b, 2), sb(b, 3))};
}
// Four byte codes c < 128 -> bf16 of 128 + c, by bits: 0x43 above a byte c
// is the bf16 with exponent 2^7 and mantissa c, i.e. exactly 128 + c.  The
// products then carry 128 x (the sub-block's activation sum) plus the
// format's own offset, which the scale step takes off again (kOff).
constexpr uint32_t kMagic43 = 0x43434343u;
__device__ __forceinline__ uint2 codes_m4(uint32_t c) {
    return {__builtin_amdgcn_perm(kMagic43, c, 0x04010400u), __builtin_amdgcn_perm(kMagic43, c, 0x04030402u)};
}
__device__ __forceinline__ uint4 codes_m8(uint32_t a, uint32_t b) {
    const uint2 x = codes_m4(a), y = codes_m4(b);
    return {x.x, x.y, y.x, y.y};
}

// bf16 bits of a small integer (|v| < 256, exact in bf16)
constexpr uint32_t bf16_of_int(int v) {
    if (v == 0) return 0u;
    const uint32_t a = (uint32_t)(v < 0 ? -v : v);
    int e = 0;
    while ((a >> (e + 1)) != 0u) e++;  // the leading one
    return (v < 0 ? 0x8000u : 0u) | (uint32_t)(e + 127) << 7 | (((a << 7) >> e) & 0x7Fu);
}
// byte `hi` (0 low, 1 high) of the bf16 of kvalues_iq4nl entries 4 w .. 4 w + 3
constexpr uint32_t iq4_bf16_word(int w, int hi) {
    uint32_t r = 0;
    for (int i = 0; i < 4; i++) r |= ((bf16_of_int(kIq4Int[4 * w + i]) >> (8 * hi)) & 0xFFu) << (8 * i);
    return r;
}
// Four IQ4_XS nibbles (one per byte of n) -> the bf16 of their kvalues_iq4nl
// entries, two per word: the low and the high bytes of the bf16 values are
// looked up as in iq4_lookup4 and interleaved.
__device__ __forceinline__ uint2 iq4_bf16_lookup4(uint32_t n) {
    constexpr uint32_t L0 = iq4_bf16_word(0, 0), L1 = iq4_bf16_word(1, 0), L2 = iq4_bf16_word(2, 0),
                       L3 = iq4_bf16_word(3, 0), H0 = iq4_bf16_word(0, 1), H1 = iq4_bf16_word(1, 1),
                       H2 = iq4_bf16_word(2, 1), H3 = iq4_bf16_word(3, 1);
    const uint32_t sel = n & 0x07070707u, pick = 0x03020100u + ((n & 0x08080808u) >> 1);
    const uint32_t lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(L3, L2, sel), __builtin_amdgcn_perm(L1, L0, sel), pick);
    const uint32_t hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(H3, H2, sel), __builtin_amdgcn_perm(H1, H0, sel), pick);
    return {__builtin_amdgcn_perm(hi, lo, 0x05010400u), __builtin_amdgcn_perm(hi, lo, 0x07030602u)};
}
static_assert(bf16_of_int(1) == 0x3F80u && bf16_of_int(113) == 0x42E2u && bf16_of_int(-127) == 0xC2FEu,
              "bf16 bits of small integers");

// ---- per-format chunk (256 values of one row): fields and sub-block steps ----
//
// kCB: bytes of a chunk row; kShm: the bits its address can have below 16
// when the matrix starts 16-byte aligned (row and chunk sizes are multiples of
// 16, 8 or 2).  A staged chunk row sits in LDS at byte offset sh (its address
// mod 16): load(r, sh, lg) reads the words lane group lg needs from the row
// image r.  Steps: kSteps sub-blocks of kSub values; step(j) gives the lane's
// codes for values kSub/4 * lg .. of sub-block j and the sub-block's scale
// (Q4_K's minimums: min_coef).

// bytes o .. o + 3 of a staged row image (o even)
template <int SHM> __device__ __forceinline__ uint32_t rw4(const uint32_t *r, int o) {
    const uint32_t lo = r[o >> 2];
    if constexpr ((SHM & 3) == 0) {
        // sh has no bits below 4: o & 3 is a compile-time constant here
        return (o & 3) ? __builtin_amdgcn_alignbyte(r[(o >> 2) + 1], lo, o & 3) : lo;
    } else {
        return __builtin_amdgcn_alignbyte(r[(o >> 2) + 1], lo, o & 3);
    }
}
// bytes o, o + 1 (o even)
__device__ __forceinline__ uint32_t rw2(const uint32_t *r, int o) { return (r[o >> 2] >> (8 * (o & 2))) & 0xFFFFu; }

template <int F> struct QChunk;

// kOff: what the step's bf16 codes add to every weight of a sub-block (the
// products' excess is kOff x the activation sum; 0: codes are the values).
template <> struct QChunk<Q4_K> {
    static constexpr int kSub = 32, kSteps = 8, kCB = 144, kShm = 0;
    static constexpr float kOff = 128.f;
    uint4 hd;     // d, dmin, 12 scale bytes
    uint2 q[4];   // qs[32 g + 8 lg .. + 7] of group g
    __device__ __forceinline__ void load(const uint32_t *r, int sh, int lg) {
        hd = {rw4<kShm>(r, sh), rw4<kShm>(r, sh + 4), rw4<kShm>(r, sh + 8), rw4<kShm>(r, sh + 12)};
#pragma unroll
        for (int g = 0; g < 4; g++)
            q[g] = {rw4<kShm>(r, sh + 16 + 32 * g + 8 * lg), rw4<kShm>(r, sh + 20 + 32 * g + 8 * lg)};
    }
    __device__ __forceinline__ uint32_t sbyte(int k) const {
        const uint32_t w = k < 4 ? hd.y : k < 8 ? hd.z : hd.w;
        return (w >> (8 * (k & 3))) & 0xFFu;
    }
    // getScaleMinK4 (model/loader.zig:3814-3825): the scale here, the
    // minimum in min_coef
    __device__ __forceinline__ uint4 step(int j, float &s) const {
        const uint32_t sc = j < 4 ? sbyte(j) & 63 : (sbyte(j + 4) & 0x0F) | ((sbyte(j - 4) >> 6) << 4);
        s = h2f(hd.x) * (float)sc;
        const uint2 w = q[j >> 1];
        const int sh = (j & 1) ? 4 : 0;
        return codes_m8((w.x >> sh) & 0x0F0F0F0Fu, (w.y >> sh) & 0x0F0F0F0Fu);
    }
    // min_j / kOff of sub-blocks j = lg and j = 4 + lg (a runtime lane
    // group; the same minimums as step's), the minimum term's coefficients
    // against the staged sums -kOff X
    __device__ __forceinline__ void min_coef(int lg, float &c0, float &c1) const {
        const int o = 8 * lg;
        const uint32_t bz = (hd.z >> o) & 0xFFu, bw = (hd.w >> o) & 0xFFu;
        const float dm = h2f(hd.x >> 16);
        c0 = dm * (float)(bz & 63) * (1.f / kOff);
        c1 = dm * (float)((bw >> 4) | ((bz >> 6) << 4)) * (1.f / kOff);
    }
};

template <> struct QChunk<Q8_0> {
    static constexpr int kSub = 32, kSteps = 8, kCB = 272, kShm = 0;
    static constexpr float kOff = 0.f;
    uint2 q[8];
    uint32_t d[8];
    __device__ __forceinline__ void load(const uint32_t *r, int sh, int lg) {
#pragma unroll
        for (int b = 0; b < 8; b++) {
            q[b] = {rw4<kShm>(r, sh + 34 * b + 2 + 8 * lg), rw4<kShm>(r, sh + 34 * b + 6 + 8 * lg)};
            d[b] = rw2(r, sh + 34 * b);
        }
    }
    __device__ __forceinline__ uint4 step(int j, float &s) const {
        s = h2f(d[j]);
        return codes_s8(q[j].x, q[j].y);
    }
};

template <> struct QChunk<IQ4_XS> {
    static constexpr int kSub = 32, kSteps = 8, kCB = 136, kShm = 8;
    static constexpr float kOff = 0.f;
    uint2 hd;     // d, scales_h, scales_l[4]
    uint2 q[8];   // qs[16 ib + 8 (lg & 1) ..]
    int hi;       // lane groups 2, 3 take the high nibbles (values 16..31)
    __device__ __forceinline__ void load(const uint32_t *r, int sh, int lg) {
        hd = {rw4<kShm>(r, sh), rw4<kShm>(r, sh + 4)};
#pragma unroll
        for (int ib = 0; ib < 8; ib++) {
            const int o = sh + 8 + 16 * ib + 8 * (lg & 1);
            q[ib] = {rw4<kShm>(r, o), rw4<kShm>(r, o + 4)};
        }
        hi = lg >> 1;
    }
    // dequantizeRowIQ4XS (model/quant_extra.zig:191-246): dl = d * (ls - 32)
    __device__ __forceinline__ uint4 step(int j, float &s) const {
        const uint32_t low = (hd.y >> (8 * (j >> 1) + 4 * (j & 1))) & 0x0F;
        const uint32_t high = (hd.x >> (16 + 2 * j)) & 3;
        s = h2f(hd.x) * (float)((int)(low | (high << 4)) - 32);
        const int sh = hi ? 4 : 0;
        const uint2 a = iq4_bf16_lookup4((q[j].x >> sh) & 0x0F0F0F0Fu), b = iq4_bf16_lookup4((q[j].y >> sh) & 0x0F0F0F0Fu);
        return {a.x, a.y, b.x, b.y};
    }
};

// 16-value sub-blocks: a step is one 16x16x16 product (four codes per lane)
template <> struct QChunk<Q6_K> {
    static constexpr int kSub = 16, kSteps = 16, kCB = 210, kShm = 14;
    static constexpr float kOff = 0.f;
    uint32_t ql[2][2][2];  // [half][16-run][ql offset 0 / 32]
    uint32_t qh[2][2];     // [half][16-run]
    uint4 sc;              // 16 int8 scales
    uint32_t d;
    __device__ __forceinline__ void load(const uint32_t *rw, int sh, int lg) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int r = 0; r < 2; r++) {
                ql[h][r][0] = rw4<kShm>(rw, sh + 64 * h + 16 * r + 4 * lg);
                ql[h][r][1] = rw4<kShm>(rw, sh + 64 * h + 32 + 16 * r + 4 * lg);
                qh[h][r] = rw4<kShm>(rw, sh + 128 + 32 * h + 16 * r + 4 * lg);
            }
        sc = {rw4<kShm>(rw, sh + 192), rw4<kShm>(rw, sh + 196), rw4<kShm>(rw, sh + 200), rw4<kShm>(rw, sh + 204)};
        d = rw2(rw, sh + 208);
    }
    // dequantizeRowQ6K (model/loader.zig:3728-3761): sub-block j = (half, quarter, 16-run)
    __device__ __forceinline__ uint2 step(int j, float &s) const {
        const int h = j >> 3, qt = (j >> 1) & 3, r = j & 1;
        const uint32_t w = ql[h][r][qt & 1];
        const uint32_t nib = ((qt & 2) ? (w >> 4) : w) & 0x0F0F0F0Fu;
        const uint32_t code = nib | (((qh[h][r] >> (2 * qt)) & 0x03030303u) << 4);
        const int si = 8 * h + r + 2 * qt;
        const uint32_t sw = si < 4 ? sc.x : si < 8 ? sc.y : si < 12 ? sc.z : sc.w;
        s = h2f(d) * sb(sw, si & 3);
        return codes_u4(code, 32.f);
    }
};

template <> struct QChunk<Q3_K> {
    static constexpr int kSub = 16, kSteps = 16, kCB = 110, kShm = 14;
    static constexpr float kOff = 0.f;
    uint32_t qs[2][2];  // [half h][16-run]: qs[32 h + 16 r + 4 lg ..]
    uint32_t hm[2];     // [16-run]: hmask[16 r + 4 lg ..]
    uint32_t raw[3];    // 12 packed scale bytes
    uint32_t d;
    __device__ __forceinline__ void load(const uint32_t *rw, int sh, int lg) {
#pragma unroll
        for (int r = 0; r < 2; r++) {
            hm[r] = rw4<kShm>(rw, sh + 16 * r + 4 * lg);
#pragma unroll
            for (int h = 0; h < 2; h++) qs[h][r] = rw4<kShm>(rw, sh + 32 + 32 * h + 16 * r + 4 * lg);
        }
        raw[0] = rw4<kShm>(rw, sh + 96);
        raw[1] = rw4<kShm>(rw, sh + 100);
        raw[2] = rw4<kShm>(rw, sh + 104);
        d = rw2(rw, sh + 108);
    }
    // dequantizeRowQ3K / expandQ3KScales (model/quant_extra.zig:45-126, 248-279):
    // sub-block si = 8 h + 2 j + half16; q = low 2 bits - (hmask bit ? 0 : 4)
    __device__ __forceinline__ uint2 step(int si, float &s) const {
        const int h = si >> 3, j = (si >> 1) & 3, r = si & 1;
        const uint32_t code = ((qs[h][r] >> (2 * j)) & 0x03030303u) | (((hm[r] >> (4 * h + j)) & 0x01010101u) << 2);
        const int qd = si & 3, grp = si >> 2;
        const uint32_t lw = raw[grp & 1], hw = raw[2];
        const uint32_t low4 = (lw >> (8 * qd + 4 * (grp >> 1))) & 0xF;
        const uint32_t hi2 = (hw >> (8 * qd + 2 * grp)) & 3;
        s = h2f(d) * (float)((int)(low4 | (hi2 << 4)) - 32);
        return codes_u4(code, 4.f);
    }
};

// Geometry of the kernel for format F (two matrices for SWIGLU).  A chunk row
// at any offset kShm allows lies in kWin 16-byte windows; its LDS image has
// one spare window (a word read past the last byte) and an odd window count,
// so the 16 rows' words fall in distinct banks.  The activation stage (TT
// token tiles of 16) is as long as LDS allows next to the code images (2048,
// 1024 or 512 values).
template <int F, bool kPair, int TT = 1, int OCC = 1> struct QGeom {
    static constexpr int kMats = kPair ? 2 : 1;
    static constexpr int kWin = (QChunk<F>::kCB + QChunk<F>::kShm + 15) / 16;
    static constexpr int kRowW = 4 * ((kWin + 1) | 1);
    static constexpr int kPieces = 16 * kWin, kP = (kPieces + 63) / 64;  // windows per wavefront chunk, per lane
    // activation sums per sub-block: the Q4_K minimums and the code offsets
    static constexpr bool kXsum = QChunk<F>::kOff != 0.f || F == Q4_K;
    static constexpr int kCodeBytes = 4 * kMats * 16 * kRowW * 4;
    // activation rows of st + 8 values (the last without its padding), the
    // sums, the code images
    static constexpr int lds_bytes(int st) {
        return 2 * ((2 * 16 * TT - 1) * (st + 8) + st) + (kXsum ? st / QChunk<F>::kSub * 16 * TT * 4 : 4) + kCodeBytes;
    }
    // OCC > 1: the longest stage that leaves LDS for OCC workgroups per CU
    // (one stages or waits while another computes), where one fits
    static constexpr int kPart = 160 * 1024 / OCC, kAll = 160 * 1024;
    static constexpr int kStage = OCC > 1 && lds_bytes(2048) <= kPart   ? 2048
                                  : OCC > 1 && lds_bytes(1024) <= kPart ? 1024
                                  : OCC > 1 && lds_bytes(512) <= kPart  ? 512
                                  : OCC > 1 && lds_bytes(256) <= kPart  ? 256
                                  : lds_bytes(2048) <= kAll             ? 2048
                                  : lds_bytes(1024) <= kAll             ? 1024
                                                                        : 512;
    static constexpr int kStageChunks = kStage / kQChunk;
};

__device__ __forceinline__ uint32_t ordered_bits_q(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// XP: the input comes split (XPlanes) and a workgroup takes two token tiles
// (32 tokens): every decoded code serves both tiles' products.
template <int F, int OUT, bool GROUPED, int R, bool XP, bool NRM = false>
__global__ void __launch_bounds__(256, OUT != OUT_SWIGLU ? 2 : 1) qgemm_kernel(QGemmParams p) {
    static_assert(!NRM || (!XP && !GROUPED), "the deferred norm stages plain rows");
    constexpr bool kPair = OUT == OUT_SWIGLU;
    constexpr int TT = XP ? 2 : 1;  // token tiles of 16 per workgroup
    // LDS for two workgroups per CU (three for the grouped single products,
    // whose registers allow it; one for the dense SWIGLU pair)
    constexpr int OCC = GROUPED && !kPair ? 3 : XP || GROUPED || !kPair ? 2 : 1;
    using QC = QChunk<F>;
    using G = QGeom<F, kPair, TT, OCC>;
    constexpr int kSub = QC::kSub, kCB = QC::kCB, kShm = QC::kShm;
    constexpr int kMats = G::kMats, kWin = G::kWin, kRowW = G::kRowW, kPieces = G::kPieces, kP = G::kP;
    constexpr bool kXsum = G::kXsum;
    // NRM: stages of at most two chunks (the norm weights are staged beside
    // the activations; a longer stage's registers spill)
    constexpr int kStage = NRM && G::kStage > kNrmStage ? kNrmStage : G::kStage, kStageChunks = kStage / kQChunk;
    static_assert((kStageChunks % R == 0 || (kStageChunks == 1 && R == 2)) && R % 2 == 0,
                  "stages hold whole rings of an even depth, or one chunk at depth 2");

    touch_params(p);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
    int m0 = blockIdx.y * 16 * TT, M = p.M;
    const int *ids = nullptr;
    const uint8_t *w = p.w, *w2 = p.w2;
    if (GROUPED) {
        if ((int)blockIdx.y >= *p.ntiles) return;
        const int *gt = p.tiles + 3 * blockIdx.y;
        w += (uint64_t)gt[0] * p.expert_stride;
        if (kPair) w2 += (uint64_t)gt[0] * p.expert_stride;
        ids = p.list + gt[1];
        m0 = 0;
        M = gt[2];
    }
    // Row groups of 64 rows (16 per wavefront): this workgroup takes groups
    // blockIdx.x, blockIdx.x + gridDim.x, ... -- several only when its
    // reduction range is one stage, whose activations then serve them all.
    // Work items (group, chunk) run group by group; the code ring runs across
    // groups.  Group g belongs to matrix seg(g) (the last whose first group
    // is at most g).
    struct Seg {
        const uint8_t *w;
        float *y;
        int N, ldy, g0;
    };
    auto seg_of = [&](int g) {
        Seg r{w, p.y, p.N, p.ldy, 0};
        if (p.nseg > 1 && g >= p.gs[0]) r = Seg{p.ws[0], p.ys[0], p.Ns[0], p.ldys[0], p.gs[0]};
        if (p.nseg > 2 && g >= p.gs[1]) r = Seg{p.ws[1], p.ys[1], p.Ns[1], p.ldys[1], p.gs[1]};
        return r;
    };
    const int ng = (p.groups - 1 - (int)blockIdx.x) / (int)gridDim.x + 1;
    const int kspan = p.K / p.ksplit, kbeg = blockIdx.z * kspan;
    const int nspan = kspan / kQChunk, cb = kbeg / kQChunk;
    const int nitems = ng * nspan;
    // item t (clamped): its matrices, their rows, the first row of this
    // wavefront, the chunk
    auto item = [&](int t, const uint8_t *(&wm)[kMats], int &nrows, int &row0, int &ca) {
        const int tc = min(t, nitems - 1), gi = tc / nspan, g = (int)blockIdx.x + gi * (int)gridDim.x;
        const Seg sg = seg_of(g);
        wm[0] = sg.w;
        if (kPair) wm[kMats - 1] = w2;
        nrows = sg.N;
        row0 = (g - sg.g0) * kQRows + 16 * wave;
        ca = cb + tc - gi * nspan;
    };

    // The activations of a stage (up to kStage values of all 16 TT tokens)
    // sit in LDS as bf16 hi / lo pieces; thread (token tt, part) stages values
    // 16 part + 256 i of tokens tt, tt + 16, ...
    constexpr int NT = 16 * TT;
    // [hi / lo][token][k]: rows kStage + 8 apart (the padding spreads the
    // rows' words over the banks), the last row without its padding
    constexpr int kXRow = kStage + 8;
    __shared__ __align__(16) unsigned short xs_raw[(2 * NT - 1) * kXRow + kStage];
    auto xs_at = [&](int piece, int tok, int k) -> unsigned short * { return &xs_raw[(piece * NT + tok) * kXRow + k]; };
    __shared__ __align__(16) float xsum_s[kXsum ? kStage / kSub : 1][kXsum ? NT : 1];  // [sub-block][token]: -kOff X
    __shared__ __align__(16) uint32_t code_s[4][kMats][16 * kRowW];        // [wavefront][matrix][row image]
    const int tt = tid >> 4, part = tid & 15;
    static_assert(!XP || !kXsum || kSub == 32, "split inputs carry 32-value sums");
    bool tok_ok[TT];
    const float *xrow[TT];
    const float *nwrow = NRM ? p.norm_w + 16 * part : nullptr;
    float ssq = 0.f;  // NRM: this thread's sum of squares of its token's staged values
    const uint16_t *xhrow[TT], *xlrow[TT];
    const float *xsrow[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) {
        tok_ok[t] = m0 + 16 * t + tt < M;
        const int m = min(m0 + 16 * t + tt, M - 1);
        const size_t r = (size_t)(GROUPED ? ids[m] / p.x_div : m);
        xrow[t] = p.x + r * p.ldx + 16 * part;
        if (XP) {
            xhrow[t] = p.xh + r * p.ldxs + 16 * part;
            xlrow[t] = p.xl + r * p.ldxs + 16 * part;
            xsrow[t] = p.xsum + r * (p.ldxs / 32) + (part >> 1);
        }
    }
    // stage_load issues the whole stage's activation loads (clamped to its
    // last chunk: unconditional, so the compiler's wait counting stays exact)
    // into ld; stage_store splits every chunk and writes those of the stage.
    // XP: the pieces and sums as split by the producer (tokens past M repeat
    // the last row; their results are never stored).
    float4 ld[TT][kStageChunks][4];
    float4 ldw[NRM ? kStageChunks : 1][4];
    float lsum[TT][XP ? kStageChunks : 1];
    auto stage_load = [&](int kb, int nc) {
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int u = 0; u < kStageChunks; u++) {
                const int ko = kb + min(u, nc - 1) * kQChunk;
                if constexpr (XP) {
                    const float4 *h = reinterpret_cast<const float4 *>(xhrow[t] + ko);
                    const float4 *l = reinterpret_cast<const float4 *>(xlrow[t] + ko);
                    ld[t][u][0] = h[0];
                    ld[t][u][1] = h[1];
                    ld[t][u][2] = l[0];
                    ld[t][u][3] = l[1];
                    if (kXsum) lsum[t][XP ? u : 0] = xsrow[t][ko / 32];
                } else {
                    const float4 *src = reinterpret_cast<const float4 *>(xrow[t] + ko);
#pragma unroll
                    for (int i = 0; i < 4; i++) ld[t][u][i] = src[i];
                    if (NRM && t == 0) {
                        const float4 *nw = reinterpret_cast<const float4 *>(nwrow + ko);
#pragma unroll
                        for (int i = 0; i < 4; i++) ldw[u][i] = nw[i];
                    }
                }
            }
    };
    auto stage_store = [&](int nc) {
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int u = 0; u < kStageChunks; u++) {
                if (u >= nc) {
                    // past the range: the loads still land -- consumed here, so the
                    // compiler's wait counting sees them complete on every path
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        __asm__ volatile("" ::"v"(ld[t][u][i].x), "v"(ld[t][u][i].y), "v"(ld[t][u][i].z),
                                         "v"(ld[t][u][i].w));
                    if (XP && kXsum) __asm__ volatile("" ::"v"(lsum[t][XP ? u : 0]));
                    if (NRM && t == 0)
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            __asm__ volatile("" ::"v"(ldw[u][i].x), "v"(ldw[u][i].y), "v"(ldw[u][i].z),
                                             "v"(ldw[u][i].w));
                    continue;
                }
                uint32_t hw[8], lw[8];
                float sum = 0.f;
                if constexpr (XP) {
                    // the loaded words are the pieces: hi of values 0..15, then lo
                    __builtin_memcpy(hw, &ld[t][u][0], 32);
                    __builtin_memcpy(lw, &ld[t][u][2], 32);
                    if (kXsum) sum = lsum[t][XP ? u : 0];
                } else {
                    float v[16];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        v[4 * i] = tok_ok[t] ? ld[t][u][i].x : 0.f;
                        v[4 * i + 1] = tok_ok[t] ? ld[t][u][i].y : 0.f;
                        v[4 * i + 2] = tok_ok[t] ? ld[t][u][i].z : 0.f;
                        v[4 * i + 3] = tok_ok[t] ? ld[t][u][i].w : 0.f;
                    }
                    if constexpr (NRM) {
                        // rmsNorm's (scale x) w with the scale deferred to the
                        // product's reader: the sum of squares of x, then x w
#pragma unroll
                        for (int i = 0; i < 16; i++) ssq = fmaf(v[i], v[i], ssq);
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            v[4 * i] *= ldw[u][i].x, v[4 * i + 1] *= ldw[u][i].y;
                            v[4 * i + 2] *= ldw[u][i].z, v[4 * i + 3] *= ldw[u][i].w;
                        }
                    }
                    sum = split_run16(v, hw, lw);
                    if (kXsum && kSub == 32) sum += __shfl_xor(sum, 1, 64);  // the other half of the 32-value sub-block
                }
                const int tk = 16 * t + tt;
                uint4 *dh = reinterpret_cast<uint4 *>(xs_at(0, tk, u * kQChunk + 16 * part));
                uint4 *dl = reinterpret_cast<uint4 *>(xs_at(1, tk, u * kQChunk + 16 * part));
                dh[0] = {hw[0], hw[1], hw[2], hw[3]};
                dh[1] = {hw[4], hw[5], hw[6], hw[7]};
                dl[0] = {lw[0], lw[1], lw[2], lw[3]};
                dl[1] = {lw[4], lw[5], lw[6], lw[7]};
                if (kXsum && kSub == 32 && !(part & 1)) xsum_s[u * 8 + (part >> 1)][tk] = -QC::kOff * sum;
                if (kXsum && kSub == 16) xsum_s[u * 16 + part][tk] = -QC::kOff * sum;
            }
    };

    qf4v acc[TT], acc2[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = acc2[t] = qf4v{0.f, 0.f, 0.f, 0.f};
    // chunk cs of the stage (offset 256 cs in LDS)
    // All products of the chunk first (independent accumulators, so the
    // matrix core pipelines them), then the scales.  A step's codes are
    // decoded once for the TT token tiles.
    auto compute = [&](const QC &r, const QC &r2, int cs, float live) {
        constexpr int S = QC::kSteps;
        // steps per pass: the products of at most 16 (step, tile) pairs in registers
        constexpr int P = S * TT > 16 ? 16 / TT : S;
        const qf4v zero = {0.f, 0.f, 0.f, 0.f};
        qf4v dv[TT][S], dv2[TT][S];
        float sv[S], sv2[S];
#pragma unroll
        for (int j0 = 0; j0 < S; j0 += P) {
#pragma unroll
        for (int j = j0; j < j0 + P; j++) {
            sv2[j] = 0.f;
            const int kx = cs * kQChunk + kSub * j;
            if constexpr (kSub == 32) {
                const bf8v b = as_bf8(r.step(j, sv[j]));
                bf8v b2 = b;
                if (kPair) b2 = as_bf8(r2.step(j, sv2[j]));
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const bf8v ah = as_bf8(*reinterpret_cast<const uint4 *>(xs_at(0, 16 * t + li, kx + 8 * lg)));
                    const bf8v al = as_bf8(*reinterpret_cast<const uint4 *>(xs_at(1, 16 * t + li, kx + 8 * lg)));
                    // kOff codes: the products start from -kOff X (the staged
                    // sums of tokens 4 lg .. 4 lg + 3), so the code offset
                    // cancels inside the product: D, not D + kOff X
                    qf4v c0 = zero;
                    if constexpr (kXsum)
                        c0 = *reinterpret_cast<const qf4v *>(&xsum_s[cs * (kQChunk / kSub) + j][16 * t + 4 * lg]);
                    dv[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, b, c0, 0, 0, 0);
                    dv[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, b, dv[t][j], 0, 0, 0);
                    dv2[t][j] = zero;
                    if (kPair) {
                        dv2[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, b2, c0, 0, 0, 0);
                        dv2[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, b2, dv2[t][j], 0, 0, 0);
                    }
                }
            } else {
                const s4v b = as_s4(r.step(j, sv[j]));
                s4v b2 = b;
                if (kPair) b2 = as_s4(r2.step(j, sv2[j]));
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const s4v ah = as_s4(*reinterpret_cast<const uint2 *>(xs_at(0, 16 * t + li, kx + 4 * lg)));
                    const s4v al = as_s4(*reinterpret_cast<const uint2 *>(xs_at(1, 16 * t + li, kx + 4 * lg)));
                    dv[t][j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, b, zero, 0, 0, 0);
                    dv[t][j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al, b, dv[t][j], 0, 0, 0);
                    dv2[t][j] = zero;
                    if (kPair) {
                        dv2[t][j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, b2, zero, 0, 0, 0);
                        dv2[t][j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al, b2, dv2[t][j], 0, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int j = j0; j < j0 + P; j++) {
            const float s = sv[j] * live, s2 = sv2[j] * live;
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    acc[t][q] = fmaf(s, dv[t][j][q], acc[t][q]);
                    if (kPair) acc2[t][q] = fmaf(s2, dv2[t][j][q], acc2[t][q]);
                }
        }
        }
        if constexpr (kXsum) {
            // s D - min X, X the sub-block's activation sum: the minimum
            // terms of the chunk's 8 sub-blocks as two f32 products (no
            // FMAs per result and step), A = -kOff X[token][sub-block
            // 4 h + lg], B = min / kOff of row li (v_mfma_f32_16x16x4_f32,
            // D[token][row]: the layout of acc)
            static_assert(kSub == 32, "eight sub-blocks per chunk");
            float c0, c1, e0 = 0.f, e1 = 0.f;
            r.min_coef(lg, c0, c1);
            c0 *= live, c1 *= live;
            if (kPair) r2.min_coef(lg, e0, e1), e0 *= live, e1 *= live;
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const float x0 = xsum_s[cs * 8 + lg][16 * t + li], x1 = xsum_s[cs * 8 + 4 + lg][16 * t + li];
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x0, c0, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x1, c1, acc[t], 0, 0, 0);
                if (kPair) {
                    acc2[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x0, e0, acc2[t], 0, 0, 0);
                    acc2[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x1, e1, acc2[t], 0, 0, 0);
                }
            }
        }
    };

    // The wavefront's chunk windows: window i = lane + 64 j of the 16 rows
    // (row i / kWin, window i % kWin).  Lanes past the last window repeat it
    // and skip the LDS write.
    int prow[kP], pwin[kP], pslot[kP];
    bool pv[kP];
#pragma unroll
    for (int j = 0; j < kP; j++) {
        const int i = lane + 64 * j, ic = min(i, kPieces - 1);
        prow[j] = ic / kWin;
        pwin[j] = ic - prow[j] * kWin;
        pslot[j] = prow[j] * kRowW + 4 * pwin[j];
        pv[j] = i < kPieces;
    }
    // Ring of R items in registers, slot q refilled in place with the item R
    // ahead.  Loads are unconditional (clamped to the last item): a load
    // under a branch makes the compiler's wait counting wait for everything
    // in flight.  A window is an aligned 16-byte block holding at least one
    // byte of its chunk row, so it never leaves the row's memory page.  Rows
    // past N re-read row N - 1 (dropped at the store).
    qu4v raw[R][kMats][kP];  // native vectors: the ring stays in registers
    auto ring_load = [&](int q, int t) {
        const uint8_t *wm[kMats];
        int nrows, row0, ca;
        item(t, wm, nrows, row0, ca);
#pragma unroll
        for (int m = 0; m < kMats; m++)
#pragma unroll
            for (int j = 0; j < kP; j++) {
                const uint8_t *st =
                    wm[m] + (uint64_t)min(row0 + prow[j], nrows - 1) * p.stride + (size_t)ca * kCB;
                const int sh = (int)((uintptr_t)st & kShm);
                const int wn = (sh + kCB + 15) >> 4;
                raw[q][m][j] = *reinterpret_cast<const qu4v *>(
                    __builtin_assume_aligned(st - sh + 16 * min(pwin[j], wn - 1), 16));
            }
    };
    // Slot q's windows into the wavefront's row images.  Lanes read what other
    // lanes wrote: the fences keep the compiler from moving the reads of the
    // previous chunk past these writes, or the reads of this one before them
    // (a wavefront's LDS accesses execute in program order).
    auto ring_put = [&](int q) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
        for (int m = 0; m < kMats; m++)
#pragma unroll
            for (int j = 0; j < kP; j++)
                if (pv[j]) *reinterpret_cast<qu4v *>(&code_s[wave][m][pslot[j]]) = raw[q][m][j];
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    };

    // Item t (in ring slot t % R) into the row images, its slot refilled
    // with item t + R, and its fields read into ff.
    auto fetch = [&](int q, int t, QC (&ff)[kMats]) {
        const uint8_t *wm[kMats];
        int nrows, row0, ca;
        item(t, wm, nrows, row0, ca);
        ring_put(q);
        ring_load(q, t + R);
        const uint64_t off = (uint64_t)min(row0 + li, nrows - 1) * p.stride + (size_t)ca * kCB;
#pragma unroll
        for (int m = 0; m < kMats; m++)
            ff[m].load(&code_s[wave][m][li * kRowW], (int)((uintptr_t)(wm[m] + off) & kShm), lg);
    };
    // Two field sets: the next chunk's fields are read while the current one
    // computes (chunk cc uses fa when cc is even; R is even).
    QC fa[kMats], fb[kMats];
    // the chunks of a staged stage; chunk s0 + c + q is in slot q (s0 and c
    // are multiples of R)
    auto run_stage = [&](int s0, int nst) {
        for (int c = 0; c < nst; c += R) {
#pragma unroll
            for (int q = 0; q < R; q++) {
                const int cc = s0 + c + q;
                if (q & 1) {
                    fetch((q + 1) % R, cc + 1, fa);
                    compute(fb[0], fb[kMats - 1], min(c + q, nst - 1), c + q < nst ? 1.f : 0.f);
                } else {
                    fetch((q + 1) % R, cc + 1, fb);
                    compute(fa[0], fa[kMats - 1], min(c + q, nst - 1), c + q < nst ? 1.f : 0.f);
                }
            }
        }
    };
    // NRM: the token's sum of squares over this reduction range (the 16
    // threads of a token are 16 neighbouring lanes), added once per range
    auto flush_ss = [&] {
        if constexpr (NRM) {
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) ssq += __shfl_xor(ssq, o, 64);
            if (p.row_ss && blockIdx.x == 0 && part == 0 && tok_ok[0]) atomicAdd(p.row_ss + (m0 + tt), ssq);
        }
    };
    // The results of group g: D[token 16 t + 4 lg + r][row li]; acc cleared after.
    auto epilogue = [&](int g) {
        const Seg sg = seg_of(g);
        const int nn = (g - sg.g0) * kQRows + 16 * wave + li;
#pragma unroll
        for (int t = 0; t < TT; t++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int j = m0 + 16 * t + 4 * lg + r;  // token of result r
                if (j >= M || nn >= sg.N) continue;
                const int jrow = GROUPED ? ids[16 * t + 4 * lg + r] : j;
                float *dst = sg.y ? sg.y + (size_t)jrow * sg.ldy + nn : nullptr;
                const float v = acc[t][r];
                if ((OUT == OUT_STORE || OUT == OUT_ADD) && p.ksplit > 1) {
                    atomicAdd(dst, v);  // partial sum of this workgroup's reduction range (STORE rows zeroed first)
                } else if (OUT == OUT_STORE) {
                    *dst = v;
                } else if (OUT == OUT_ADD) {
                    *dst = *dst + v;
                } else if (OUT == OUT_SWIGLU) {
                    *dst = (v / (1.0f + expf(-v))) * acc2[t][r];
                }
            }
            if (OUT == OUT_ARGMAX) {
                // token 4 lg + r: the largest value over the 16 rows of lanes li, then the lowest row
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int j = m0 + 16 * t + 4 * lg + r;
                    const float v = acc[t][r];
                    if (sg.y && j < M && nn < sg.N) sg.y[(size_t)j * sg.ldy + nn] = v;
                    unsigned long long key = (j < M && nn < sg.N)
                                                 ? ((unsigned long long)ordered_bits_q(v) << 32) |
                                                       (unsigned long long)(0xFFFFFFFFu - (uint32_t)nn)
                                                 : 0ull;
#pragma unroll
                    for (int o = 1; o < 16; o <<= 1) {
                        const unsigned long long k2 = __shfl_xor(key, o, 64);
                        key = k2 > key ? k2 : key;
                    }
                    if (li == 0 && key) atomicMax(p.argmax + j, key);
                }
            }
            acc[t] = qf4v{0.f, 0.f, 0.f, 0.f};
            acc2[t] = qf4v{0.f, 0.f, 0.f, 0.f};
        }
    };

    if (nspan <= kStageChunks) {
        // One stage: the activations, then the ring's first items, then the
        // LDS writes -- the wait for the activations does not cover the codes
        // (loads complete in order), which stream during staging.  Then every
        // item of every group against the staged activations.
        stage_load(kbeg, nspan);
#pragma unroll
        for (int q = 0; q < R; q++) ring_load(q, q);
        stage_store(nspan);
        flush_ss();
        __syncthreads();
        fetch(0, 0, fa);
        for (int t0 = 0; t0 < nitems; t0 += R) {
#pragma unroll
            for (int q = 0; q < R; q++) {
                const int t = t0 + q, gi = t / nspan, c = t - gi * nspan;
                const float live = t < nitems ? 1.f : 0.f;
                if (q & 1) {
                    fetch((q + 1) % R, t + 1, fa);
                    compute(fb[0], fb[kMats - 1], c, live);
                } else {
                    fetch((q + 1) % R, t + 1, fb);
                    compute(fa[0], fa[kMats - 1], c, live);
                }
                if (c == nspan - 1 && t < nitems) epilogue((int)blockIdx.x + gi * (int)gridDim.x);
            }
        }
        return;
    }
    // Several stages (one group per workgroup): the first stage as above,
    // later stages wait for the ring's loads ahead of their activations.
    // kPre: the next stage's inputs are loaded into registers while this
    // stage computes, where the registers allow it without spills (the
    // one-tile single products but Q3_K's, the split-input Q4_K / IQ4_XS
    // ones and the grouped IQ4_XS pair); the last stage re-loads itself, so
    // the loads stay unconditional.
    // kPre1: the same for the one-chunk stages of the split-input Q8_0 kernel
    constexpr bool kPre1 = XP && kStageChunks == 1 && F == Q8_0;
    constexpr bool kPre = kStageChunks > 1 && (XP ? (F == Q4_K || F == IQ4_XS)
                                               : GROUPED ? (kPair && F == IQ4_XS)
                                                         : (!kPair && F != Q3_K));
    const int last_s0 = (nspan - 1) / kStageChunks * kStageChunks;
    auto prefetch = [&](int s0) {
        const int sn = min(s0, last_s0);
        stage_load(kbeg + sn * kQChunk, min(kStageChunks, nspan - sn));
    };
    {
        const int nst = kStageChunks;
        stage_load(kbeg, nst);
#pragma unroll
        for (int q = 0; q < R; q++) ring_load(q, q);
        stage_store(nst);
        __syncthreads();
        fetch(0, 0, fa);
        if constexpr (kPre || kPre1) prefetch(kStageChunks);
        if constexpr (kStageChunks == 1) {
            fetch(1, 1, fb);  // chunk 0 only; the pairs below start at chunk 1
            compute(fa[0], fa[kMats - 1], 0, 1.f);
        } else {
            run_stage(0, nst);
        }
    }
    if constexpr (kStageChunks == 1) {
        // One-chunk stages (depth 2): chunks in pairs, so that the field set
        // and the ring slot of a chunk are its parity at compile time.
        for (int s0 = 1; s0 < nspan; s0 += 2) {
            __syncthreads();  // every wavefront is done with the previous stage
            if constexpr (!kPre1) stage_load(kbeg + s0 * kQChunk, 1);
            stage_store(1);
            __syncthreads();
            if constexpr (kPre1) prefetch(s0 + 1);
            fetch(0, s0 + 1, fa);
            compute(fb[0], fb[kMats - 1], 0, 1.f);
            // chunk s0 + 1 (past the range: a dead step, so the pairs stay whole)
            const bool more = s0 + 1 < nspan;
            __syncthreads();
            if constexpr (kPre1) {
                stage_store(more ? 1 : 0);  // (the loads land either way)
            } else if (more) {
                stage_load(kbeg + (s0 + 1) * kQChunk, 1);
                stage_store(1);
            }
            __syncthreads();
            if constexpr (kPre1) prefetch(s0 + 2);
            fetch(1, s0 + 2, fb);
            compute(fa[0], fa[kMats - 1], 0, more ? 1.f : 0.f);
        }
    } else {
        for (int s0 = kStageChunks; s0 < nspan; s0 += kStageChunks) {
            const int nst = min(kStageChunks, nspan - s0);
            __syncthreads();  // every wavefront is done with the previous stage
            if constexpr (!kPre) stage_load(kbeg + s0 * kQChunk, nst);
            stage_store(nst);
            __syncthreads();
            if constexpr (kPre) prefetch(s0 + kStageChunks);
            run_stage(s0, nst);
        }
    }
    flush_ss();
    epilogue(blockIdx.x);
}

typedef void (*QGemmKernel)(QGemmParams);

template <int F, bool G, int R, bool XP> static QGemmKernel pick_q(int out, bool nrm = false) {
    if constexpr (!XP && !G && R == 2) {
        if (nrm) return out == OUT_ADD ? qgemm_kernel<F, OUT_ADD, false, 2, false, true>
                        : out == OUT_STORE ? qgemm_kernel<F, OUT_STORE, false, 2, false, true>
                                           : nullptr;
    } else {
        if (nrm) return nullptr;
    }
    if constexpr (XP) {
        // split inputs, two token tiles: the dense stores and adds of the batched passes
        if constexpr (G || R != 2)
            return nullptr;
        else
            return out == OUT_STORE ? qgemm_kernel<F, OUT_STORE, G, R, XP>
                   : out == OUT_ADD ? qgemm_kernel<F, OUT_ADD, G, R, XP>
                                    : nullptr;
    } else if constexpr (R != 2) {
        return nullptr;  // ring depth 2: stages may hold two chunks
    } else {
        switch (out) {
        case OUT_STORE: return qgemm_kernel<F, OUT_STORE, G, R, XP>;
        case OUT_SWIGLU:
            if constexpr (R == 2) return qgemm_kernel<F, OUT_SWIGLU, G, R, XP>;  // deeper rings spill
            return nullptr;
        case OUT_ADD:
            if constexpr (G) return nullptr;
            else return qgemm_kernel<F, OUT_ADD, G, R, XP>;
        case OUT_ARGMAX:
            if constexpr (G) return nullptr;
            else return qgemm_kernel<F, OUT_ARGMAX, G, R, XP>;
        default: return nullptr;
        }
    }
}

// ring depth: 4 chunks, or 2 for the two matrices of SWIGLU (the same bytes in
// flight), for reduction ranges of two chunks, for two token tiles (the
// products' registers) and for the grouped kernels (stages of two chunks)
template <bool G, bool XP> static QGemmKernel pick_qf(int fmt, int out, int K, bool nrm = false) {
    (void)K;
    switch (fmt) {  // every kernel at depth 2 (two workgroups per CU leave stages of two chunks)
    case Q4_K: return pick_q<Q4_K, G, 2, XP>(out, nrm);
    case Q6_K: return pick_q<Q6_K, G, 2, XP>(out, nrm);
    case Q8_0: return pick_q<Q8_0, G, 2, XP>(out, nrm);
    case IQ4_XS: return pick_q<IQ4_XS, G, 2, XP>(out, nrm);
    case Q3_K: return pick_q<Q3_K, G, 2, XP>(out, nrm);
    default: return nullptr;
    }
}

// The chunk windows assume a 16-byte aligned matrix (and expert slices) whose
// row stride keeps chunk addresses within the format's offsets below 16.
template <bool P, int TT = 1, int OCC = 1> static int stage_chunks_of(int fmt) {
    switch (fmt) {
    case Q4_K: return QGeom<Q4_K, P, TT, OCC>::kStageChunks;
    case Q8_0: return QGeom<Q8_0, P, TT, OCC>::kStageChunks;
    case IQ4_XS: return QGeom<IQ4_XS, P, TT, OCC>::kStageChunks;
    case Q6_K: return QGeom<Q6_K, P, TT, OCC>::kStageChunks;
    case Q3_K: return QGeom<Q3_K, P, TT, OCC>::kStageChunks;
    default: return 0;
    }
}

bool qgemm_supported(int fmt, int K, const void *w, const void *w2, uint64_t stride, uint64_t expert_stride) {
    int shm;
    switch (fmt) {
    case Q4_K: shm = QChunk<Q4_K>::kShm; break;
    case Q8_0: shm = QChunk<Q8_0>::kShm; break;
    case IQ4_XS: shm = QChunk<IQ4_XS>::kShm; break;
    case Q6_K: shm = QChunk<Q6_K>::kShm; break;
    case Q3_K: shm = QChunk<Q3_K>::kShm; break;
    default: return false;
    }
    const uintptr_t base = (uintptr_t)w | (uintptr_t)w2 | (uintptr_t)expert_stride;
    return K >= kQChunk && K % kQChunk == 0 && base % 16 == 0 && (stride & 15 & ~(uint64_t)shm) == 0;
}

__global__ void zero_rows_kernel(float *y, int ldy, int M, int N) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < M * N) y[(size_t)(i / N) * ldy + i % N] = 0.f;
}

// Workgroups wanted for one product: every CU streams weights
// (ZIGGY_HIP_QGEMM_WPC: workgroups per CU, a tuning knob).
static int qgemm_target_wgs() {
    static int t = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        const char *e = getenv("ZIGGY_HIP_QGEMM_WPC");
        const int w = e ? atoi(e) : 1;
        return n * (w >= 1 && w <= 8 ? w : 1);
    }();
    return t;
}

// Weight of the activation staging against the chunk work of one workgroup
// (ZIGGY_HIP_QGEMM_STAGE_W overrides it; a tuning knob).
static double qgemm_stage_weight() {
    static const double w = [] {
        const char *e = getenv("ZIGGY_HIP_QGEMM_STAGE_W");
        return e ? atof(e) : 0.5;
    }();
    return w;
}

hipError_t launch_qgemm_multi(int fmt, int nseg, const uint8_t *const *w, float *const *y, const int *ldy,
                              const int *N, const uint8_t *w2, uint64_t stride, const float *x, int ldx, int M, int K,
                              int out, unsigned long long *argmax, hipStream_t s, int max_split, const XPlanes *xp,
                              const RowNorm *rn) {
    if (nseg < 1 || nseg > 3 || M < 1 || ldx % 4 || (nseg > 1 && (out == OUT_SWIGLU || out == OUT_ARGMAX)))
        return hipErrorInvalidValue;
    if (rn && (!rn->w || (out != OUT_STORE && out != OUT_ADD) || (uintptr_t)rn->w % 16)) return hipErrorInvalidValue;
    QGemmParams p{w[0], w2, stride, x, y[0], M, N[0], K, ldx, ldy[0], argmax, nullptr, nullptr, nullptr, 1, 0, 1};
    int groups = 0;
    for (int i = 0; i < nseg; i++) {
        if (N[i] < 1 || !qgemm_supported(fmt, K, w[i], w2, stride, 0)) return hipErrorInvalidValue;
        if (i > 0) {
            p.ws[i - 1] = w[i];
            p.ys[i - 1] = y[i];
            p.Ns[i - 1] = N[i];
            p.ldys[i - 1] = ldy[i];
            p.gs[i - 1] = groups;
        }
        groups += (N[i] + kQRows - 1) / kQRows;
    }
    p.groups = groups;
    p.nseg = nseg;
    // split inputs (more than one token tile): the XP kernels, two token tiles per workgroup
    const bool use_xp = !rn && xp && xp->hi && xp->lo && xp->sum && xp->ld % 32 == 0 && K <= xp->ld && M > 16 &&
                        (out == OUT_STORE || out == OUT_ADD);
    const int TT = use_xp ? 2 : 1;
    const int tiles = (M + 16 * TT - 1) / (16 * TT), chunks = K / kQChunk;
    const int target = qgemm_target_wgs();
    int stage = use_xp                ? stage_chunks_of<false, 2, 2>(fmt)
                : out == OUT_SWIGLU ? stage_chunks_of<true>(fmt)
                                    : stage_chunks_of<false, 1, 2>(fmt);
    if (rn && stage > kNrmStage / kQChunk) stage = kNrmStage / kQChunk;  // the NRM kernels' stages
    // Reduction split ks (a power of two; results added atomically, plain
    // stores and adds only) and workgroups per split pg, each taking every
    // pg-th row group.  Several groups per workgroup need a one-stage range:
    // the candidate with the shortest critical path (chunks of the busiest
    // workgroup, plus its staging) wins, the smaller split on ties.
    int ks = 0, pg = groups;
    double best = 0.0;
    const bool can_split = out == OUT_STORE || out == OUT_ADD;
    for (int k = 1; k <= chunks && k <= max_split && (k == 1 || can_split); k *= 2) {
        if (chunks % k) break;
        const int nspan = chunks / k;
        if (nspan > stage || (k > 1 && nspan < 2)) continue;
        int g = target / (tiles * k);
        g = g < 1 ? 1 : g > groups ? groups : g;
        const double cost = (double)((groups + g - 1) / g) * nspan + qgemm_stage_weight() * nspan;
        if (ks == 0 || cost < best) ks = k, pg = g, best = cost;
    }
    if (ks == 0) {
        // several stages: one group per workgroup, split while row groups leave CUs idle
        ks = 1, pg = groups;
        if (can_split)
            while (groups * tiles * ks * 2 <= target && chunks % (ks * 2) == 0 && ks * 2 <= max_split) ks *= 2;
    }
    p.ksplit = ks;
    QGemmKernel k = use_xp ? pick_qf<false, true>(fmt, out, K / ks) : pick_qf<false, false>(fmt, out, K / ks, rn);
    if (!k) return hipErrorInvalidValue;
    if (rn) {
        p.norm_w = rn->w;
        p.row_ss = rn->ss;  // none: another launch over the same rows adds the sums
    }
    if (use_xp) p.xh = xp->hi, p.xl = xp->lo, p.xsum = xp->sum, p.ldxs = xp->ld;
    if (ks > 1 && out == OUT_STORE) {
        for (int i = 0; i < nseg; i++) {
            hipLaunchKernelGGL(zero_rows_kernel, dim3((M * N[i] + 255) / 256), dim3(256), 0, s, y[i], ldy[i], M, N[i]);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    hipLaunchKernelGGL(k, dim3(pg, tiles, ks), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_qgemm(int fmt, const uint8_t *w, const uint8_t *w2, uint64_t stride, const float *x, int ldx,
                        float *y, int ldy, int M, int N, int K, int out, unsigned long long *argmax, hipStream_t s,
                        int max_split, const XPlanes *xp) {
    return launch_qgemm_multi(fmt, 1, &w, &y, &ldy, &N, w2, stride, x, ldx, M, K, out, argmax, s, max_split, xp);
}

hipError_t launch_qgemm_grouped(int fmt, const uint8_t *w, const uint8_t *w2, uint64_t stride,
                                uint64_t expert_stride, const float *x, int ldx, int x_div, float *y, int ldy, int N,
                                int K, int out, const int *tiles, const int *list, const int *ntiles, int max_tiles,
                                hipStream_t s) {
    if (N < 1 || !qgemm_supported(fmt, K, w, w2, stride, expert_stride) || ldx % 4 || max_tiles < 1 || x_div < 1)
        return hipErrorInvalidValue;
    QGemmKernel k = pick_qf<true, false>(fmt, out, K);
    if (!k) return hipErrorInvalidValue;
    QGemmParams p{w, w2, stride, x, y, 16, N, K, ldx, ldy, nullptr, tiles, list, ntiles, x_div, expert_stride, 1};
    p.groups = (N + kQRows - 1) / kQRows;
    p.nseg = 1;
    // A one-stage reduction lets a workgroup take several row groups of its
    // token tile against one staging: about four workgroups per CU at the
    // largest tile count (the launch's bound; unused tiles exit at once).
    const int stage = out == OUT_SWIGLU ? stage_chunks_of<true, 1, 2>(fmt) : stage_chunks_of<false, 1, 3>(fmt);
    int pg = p.groups;
    if (K / kQChunk <= stage) {
        pg = 4 * qgemm_target_wgs() / max_tiles;
        pg = pg < 1 ? 1 : pg > p.groups ? p.groups : pg;
    }
    hipLaunchKernelGGL(k, dim3(pg, max_tiles), dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace zh
