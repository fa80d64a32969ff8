// zh_internal.h -- host-side internals of libziggy_hip: context, buffers,
// status/error plumbing and the launcher interface between the C ABI and the
// kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <type_traits>

#include "ziggy_hip.h"

struct ZiggyHipContext {
    int device = 0;
    hipStream_t stream = nullptr;
    bool seq_open = false;
    hipEvent_t seq_begin = nullptr, seq_end = nullptr;
    ZiggyHipDeviceInfo info{};
    // device scratch shared by the primitive ops (attention partials, argmax slot)
    void *scratch = nullptr;
    size_t scratch_len = 0;
    // zeroed arrival counters of the attention kernel (each launch leaves them zero)
    unsigned *counters = nullptr;
    // identity block table (kIdentityPages entries): the bridge-level attention's contiguous cache
    uint32_t *identity_pages = nullptr;
    // RoPE denominators base^(2i / n_rot) per (base, n_rot) seen, computed on the host
    struct RopeTable {
        float base;
        int n_rot;
        float *dev;
    } rope_tables[8] = {};
};

struct ZiggyHipBuffer {
    ZiggyHipContext *ctx = nullptr;
    int device = 0;  // destroy needs only this, so a buffer may outlive its context
    void *ptr = nullptr;
    size_t len = 0;
};

namespace zh {

inline void set_err(char *err, size_t len, const char *fmt, ...) {
    if (!err || len == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, len, fmt, ap);
    va_end(ap);
    err[len - 1] = 0;
}

inline int hip_fail(hipError_t e, const char *what, char *err, size_t len) {
    set_err(err, len, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    return ZIGGY_HIP_EXECUTION_FAILED;
}

#define ZH_TRY(call, what)                                          \
    do {                                                            \
        hipError_t _e = (call);                                     \
        if (_e != hipSuccess) return zh::hip_fail(_e, what, err, err_len); \
    } while (0)

// Completes an op: synchronous unless a sequence is open (bridge.m:448-485).
inline int finish_op(ZiggyHipContext *ctx, const char *what, char *err, size_t err_len) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what, err, err_len);
    if (!ctx->seq_open) {
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return hip_fail(e, what, err, err_len);
    }
    return ZIGGY_HIP_OK;
}

inline bool buf_ok(const ZiggyHipBuffer *b, size_t need) { return b && b->ptr && b->len >= need; }

// RoPE denominators base^(2i / n_rot), i < n_rot / 2, with the exponent and
// powf of the CPU path (applyRoPE, model/loader.zig:3827-3866): theta =
// pos / denom[i].  Computed on the host so the angles are the CPU path's to
// the bit; at positions in the thousands one ulp of a denominator moves an
// angle by ~1e-3 rad.
inline void rope_denominators(float base, int n_rot, float *out) {
    for (int i = 0; i < n_rot / 2; i++) out[i] = powf(base, (float)(2 * i) / (float)n_rot);
}
// The context's device table of rope_denominators(base, n_rot) (made on first use).
hipError_t ctx_rope_denom(ZiggyHipContext *ctx, float base, int n_rot, const float **out);

// ---------------- kernel launchers (implemented in the .hip files) ----------------

enum InMode : int { IN_PLAIN = 0, IN_NORM = 1, IN_SILU = 2 };
enum OutMode : int { OUT_STORE = 0, OUT_ADD = 1, OUT_SWIGLU = 2, OUT_ARGMAX = 3, OUT_WADD = 4 };

// One batch of scalar loads touching every 64-byte line of a kernel's
// parameter block (up to 12 lines): the kernel's later reads of any field hit
// the scalar cache instead of paying a memory round trip each along their
// dependent chains (segment search, then the segment's fields, then the
// addresses of the first loads).
template <class P> __device__ __forceinline__ void touch_params(const P &p) {
    static_assert(sizeof(P) <= 12 * 64, "up to 12 parameter lines");
    constexpr int L = (int)((sizeof(P) + 63) / 64) - 1;  // last line
    const uint32_t *w = reinterpret_cast<const uint32_t *>(&p);
    auto at = [&](int line) { return w[16 * (line < L ? line : L)]; };
    __asm__ volatile("" ::"s"(at(0)), "s"(at(1)), "s"(at(2)), "s"(at(3)), "s"(at(4)), "s"(at(5)), "s"(at(6)),
                     "s"(at(7)), "s"(at(8)), "s"(at(9)), "s"(at(10)), "s"(at(11)));
}

// The exact-code GEMM's activation pieces (zh_qgemm.hip): x = hi + lo with
// hi = bf16(x) and lo = bf16(x - hi), both rounded to nearest even, x = hi +
// lo to 2^-17 relative.  One run is 16 consecutive values: eight words of
// packed pieces each, and the sum of hi + lo over the run in one fixed order
// (the producers and the GEMM's own staging call this same function, so the
// sums, and hence the products, do not depend on where the split ran).
typedef float zh_f2v __attribute__((ext_vector_type(2)));
typedef __bf16 zh_b2v __attribute__((ext_vector_type(2)));
// two floats -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    const zh_b2v h = __builtin_convertvector((zh_f2v){a, b}, zh_b2v);
    uint32_t u;
    __builtin_memcpy(&u, &h, 4);
    return u;
}
__device__ __forceinline__ float split_run16(const float (&v)[16], uint32_t (&hw)[8], uint32_t (&lw)[8]) {
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float a = v[2 * i], b = v[2 * i + 1];
        const uint32_t h = pk_bf16(a, b);
        const float ha = __uint_as_float(h << 16), hb = __uint_as_float(h & 0xFFFF0000u);
        const uint32_t l = pk_bf16(a - ha, b - hb);
        hw[i] = h;
        lw[i] = l;
        sum += (ha + __uint_as_float(l << 16)) + (hb + __uint_as_float(l & 0xFFFF0000u));
    }
    return sum;
}

// Exchanges with the lane 16 or 32 apart on the vector ALU
// (v_permlane16_swap / v_permlane32_swap of gfx950) instead of an LDS-path
// bpermute.  Called with one value in both operands, the swap returns this
// lane's value and its partner's (in an order that depends on the lane), so
// a commutative op of the two is op(own, partner) in every lane: the same
// bits as `op(v, __shfl_xor(v, 16 or 32))`.
template <int D> __device__ __forceinline__ void lane_pair(uint32_t v, uint32_t &a, uint32_t &b) {
    static_assert(D == 16 || D == 32, "lane distance 16 or 32");
    if constexpr (D == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        a = r[0];
        b = r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        a = r[0];
        b = r[1];
    }
}
template <int D> __device__ __forceinline__ float xsum(float v) {
    uint32_t a, b;
    lane_pair<D>(__float_as_uint(v), a, b);
    return __uint_as_float(a) + __uint_as_float(b);
}
template <int D> __device__ __forceinline__ float xmax(float v) {
    uint32_t a, b;
    lane_pair<D>(__float_as_uint(v), a, b);
    return fmaxf(__uint_as_float(a), __uint_as_float(b));
}
template <int D> __device__ __forceinline__ unsigned long long xmax_u64(unsigned long long v) {
    uint32_t a0, b0, a1, b1;
    lane_pair<D>((uint32_t)v, a0, b0);
    lane_pair<D>((uint32_t)(v >> 32), a1, b1);
    const unsigned long long a = ((unsigned long long)a1 << 32) | a0, b = ((unsigned long long)b1 << 32) | b0;
    return a > b ? a : b;
}
template <int CTRL> __device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
    return ((unsigned long long)hi << 32) | lo;
}
// Wavefront maximum of a 64-bit key, valid in every lane: DPP within each
// 16-lane row (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror),
// then the two lane swaps across rows.  Every lane must be active.
__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long v) {
    auto mx = [](unsigned long long a, unsigned long long b) { return a > b ? a : b; };
    v = mx(v, dpp_u64<0xB1>(v));
    v = mx(v, dpp_u64<0x4E>(v));
    v = mx(v, dpp_u64<0x141>(v));
    v = mx(v, dpp_u64<0x140>(v));
    v = xmax_u64<16>(v);
    return xmax_u64<32>(v);
}
// The same for a float (max is exact in any order).
__device__ __forceinline__ float wave_max_f32(float v) {
    auto mov = [](float x, auto ctrl) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, false));
    };
    v = fmaxf(v, mov(v, std::integral_constant<int, 0xB1>{}));
    v = fmaxf(v, mov(v, std::integral_constant<int, 0x4E>{}));
    v = fmaxf(v, mov(v, std::integral_constant<int, 0x141>{}));
    v = fmaxf(v, mov(v, std::integral_constant<int, 0x140>{}));
    v = xmax<16>(v);
    return xmax<32>(v);
}

struct MvSeg {
    const uint8_t *w;       // first row of the segment
    uint64_t stride;        // bytes per row
    float *y;               // output (STORE/ADD/SWIGLU/ARGMAX logits; may be null for ARGMAX)
    const uint8_t *w2;      // SWIGLU: the "up" matrix (same format/shape as w)
    const float *x;         // input of this segment (null: MvParams::x)
    int rows;
    int fmt;
    int wg_begin;           // first workgroup of this segment
    int rows_per_wg;
    int expert_slot;        // >= 0: rows offset by entries[slot].id * rows_per_expert (MvParams::expert)
};

constexpr int kMaxSeg = 10;  // segments of one matvec launch (8 routed experts + shared + spare)

struct MvParams {
    MvSeg seg[kMaxSeg];
    int nseg;
    int cols;
    int slots;              // cols / 64
    int team;               // lanes per row team (power of two, <= 256)
    int rows_per_team;
    const float *x;         // PLAIN: input; NORM: hidden to normalise; SILU: gate
    const float *x2;        // SILU: up
    const float *norm_w;    // NORM: f32 weights
    float eps;
    unsigned long long *argmax_slot;  // ARGMAX: packed (ordered value << 32 | ~row)
    const uint32_t *expert;           // indexed: entries (ShortlistEntry {u32 id, f32 weight})
    int rows_per_expert;
    int expert_limit;                 // expert ids >= this are ignored (no rows are read)
    float weight_scale;               // WADD: y += scale * dot (scale from entries if expert set)
    const int *gate_flag;             // optional device flag (argmax output only): kernel exits if *gate_flag == 0
    // Fused prologues of the MoE decode launches (pro_in null: none).
    //   SWIGLU  the routing: every wavefront of a routed segment's workgroups
    //           finds its segment's expert from the router logits pro_in
    //           (route_id: softmax, top-k up to the slot) and offsets the
    //           segment by it; one more workgroup, route_wg (set by the
    //           launcher, past the segments), writes the whole route
    //           (uint32 entries, route_wave) to pro_out.  pro_cfg = E | k << 16 |
    //           gating << 20 | weights_norm << 24 | shared_gate << 25,
    //           pro_scale = weights scale; `expert` is unused.
    //   NORM    (f32 router) the previous layer's combine: the input is
    //           x + combine(pro_in rows, route at `expert`), computed per
    //           workgroup into LDS (cols <= kCombineMaxCols); workgroup 0
    //           writes it to pro_out (f32, not x).  pro_cfg = k | shared << 4.
    const float *pro_in;
    void *pro_out;
    uint32_t pro_cfg;
    float pro_scale;
    int route_wg;  // SWIGLU routing: the route writer workgroup (launch_matvec sets it)
};

// Values of a row one team covers (256 lanes of 64); longer rows of plain or
// SiLU inputs run as column windows (launch_matvec).
constexpr int kMaxMatvecCols = 256 * 64;
constexpr int kMaxMatvecRowLen = 4 * kMaxMatvecCols;  // plain / SiLU rows the windows serve
// Builds the launch plan (team size, rows per team, workgroup ranges) and launches.
hipError_t launch_matvec(const MvParams &p, int in_mode, int out_mode, hipStream_t s);
void plan_matvec(MvParams &p, int target_wgs);
// the workgroups a matvec grid is planned for (a whole multiple of the CU count)
int matvec_target_wgs();
// An MoE layer's gate/up (NORM, SWIGLU with the routing prologue) and down
// (PLAIN, STORE) products in one launch (moe_ffn_kernel): gate/up publishes
// its act rows, the down workgroups find their experts from gu.pro_in's
// logits and read their act rows as they are published.  Every act word
// must hold kPollEmpty before the launch; the route writer refills `refill`
// (refill_n words: the next layer's act rows) for the next launch.
// poll_err is set when a wait ran out.
hipError_t launch_moe_ffn(const MvParams &gu, const MvParams &down, int *poll_err, float *refill, int refill_n,
                          hipStream_t s);
// whether launch_moe_ffn serves these formats and row lengths
bool moe_ffn_supported(int f1, int f2, int gate_cols, int down_cols);

hipError_t launch_dequant(int fmt, const uint8_t *w, uint64_t stride, float *out, int rows, int cols,
                          hipStream_t s);

// small ops (zh_ops.hip)
hipError_t launch_rms_norm(const float *x, const float *w, float *out, int n, float eps, float off, hipStream_t s);
hipError_t launch_rms_norm_per_head(const float *x, const float *w, float *out, int heads, int hd, float eps,
                                    float off, hipStream_t s);
hipError_t launch_rope(const float *src, float *dst, int heads, int hd, int rope_dim, int pos, const float *denom,
                       int style, hipStream_t s);
hipError_t launch_store_kv_half(const float *src, __half *dst, int count, hipStream_t s);
hipError_t launch_silu_mul(float *gate, const float *up, int n, hipStream_t s);
// Spans of floats a pass kernel clears on the way, for the accumulating
// products after it (up to four; n 0: none).
struct ZeroSpans {
    float *p[4];
    size_t n[4];
};
// The deferred RMSNorm's scale of row m (RowNorm): 1 / sqrt(ss[m] / n + eps);
// ss null: 1.
struct RowScale {
    const float *ss;
    int n;
    float eps;
};
// rows x n: gate = silu(r gate) * (r up), r the row's scale (silu_mul with
// the deferred norm of the gate/up products), clearing z on the way
hipError_t launch_silu_mul_rows(float *gate, const float *up, int rows, int n, RowScale rs, const ZeroSpans &z,
                                hipStream_t s);
hipError_t launch_zero_spans(const ZeroSpans &z, hipStream_t s);
hipError_t launch_add(float *dst, const float *src, int n, hipStream_t s);
hipError_t launch_argmax(const float *x, int n, uint32_t *out_token, unsigned long long *tmp, hipStream_t s);
hipError_t launch_topk(const float *x, int n, int k, void *entries, hipStream_t s);
// Output shortlist (zh_sample.hip): the top k (<= 64) of n (<= 262144) values
// as entries {u32 id, f32 value}, highest first, ties to the lower id; keys:
// shortlist_scratch_keys(n) packed keys of device scratch.
size_t shortlist_scratch_keys(int n);
hipError_t launch_shortlist(const float *x, int n, int k, unsigned long long *keys, uint32_t *entries,
                            hipStream_t s);
hipError_t launch_normalize_topk(void *entries, int k, int softmax, int normalize, float scale, hipStream_t s);
hipError_t launch_weighted_sum_topk(float *dst, const float *src, const void *entries, int n, int slot,
                                    hipStream_t s);
hipError_t launch_sigmoid_scale_add(float *dst, const float *src, const float *scalar, int n, hipStream_t s);
hipError_t launch_argmax_finalize(const unsigned long long *slot, uint32_t *state, hipStream_t s);
hipError_t launch_fill_u64(unsigned long long *p, unsigned long long v, int n, hipStream_t s);
// per-row argmax keys (value, then the lowest index) of rows x n values, ld
// apart, max-ed into slots[row] (zero beforehand)
hipError_t launch_argmax_rows(const float *x, int rows, int n, int ld, unsigned long long *slots, hipStream_t s);

// Rows of activations split once for the exact-code GEMM (split_run16): row r
// of the pieces at hi + r ld and lo + r ld, its 32-value sums at sum + r ld / 32
// (ld a multiple of 32).  A producer writes them next to (or instead of the
// GEMM re-splitting) its f32 rows; launch_gemm takes them as a hint.
struct XPlanes {
    uint16_t *hi, *lo;
    float *sum;
    int ld;
};
// rows x n values of x (row stride ldx, n a multiple of 32) into xp
hipError_t launch_split_rows(const float *x, int ldx, int rows, int n, const XPlanes &xp, hipStream_t s);
// gate = silu(gate) * up (as launch_silu_mul, rows x n, row stride n), also into xp
hipError_t launch_silu_mul_split(float *gate, const float *up, int rows, int n, const XPlanes &xp, hipStream_t s);
// MFMA GEMM for M >= 8 tokens (zh_gemm.hip): Y[m][n] (=, +=) sum_k W[n][k] X[m][k]
// (OUT_STORE / OUT_ADD / OUT_SWIGLU with w2 / OUT_ARGMAX into argmax[M]).
// max_split bounds the reduction split of the exact-code kernel, whose
// partial results add atomically: 1 keeps a += product deterministic, 2 a
// product into a cleared output (0 + a + b is the same in either order).
// xp (optional): the same input already split (XPlanes), used when the
// exact-code kernel runs.
hipError_t launch_gemm(int fmt, const uint8_t *w, const uint8_t *w2, uint64_t stride, const float *x, int ldx,
                       float *y, int ldy, int M, int N, int K, int out, unsigned long long *argmax, hipStream_t s,
                       bool precise = false, int max_split = 16, const XPlanes *xp = nullptr);
// The deferred RMSNorm of a product's input rows (rmsNorm, model/loader.zig:
// 3404-3426, with its scale moved past the product): the product takes
// x * w, and each row's sum of squares of x is added to ss[row] (when ss is
// set), so that its reader scales the result by 1 / sqrt(ss / K + eps).
struct RowNorm {
    const float *w;
    float *ss;
};
// Up to three matrices of one format, row stride and reduction length against
// one input (stores or adds): one launch on the exact-code kernel, else one
// product each.  rn (the exact-code kernel only; see gemm_rownorm_supported):
// the deferred norm of the input.
hipError_t launch_gemm_multi(int fmt, int nseg, const uint8_t *const *w, float *const *y, const int *ldy,
                             const int *N, uint64_t stride, const float *x, int ldx, int M, int K, int out,
                             hipStream_t s, int max_split = 16, const XPlanes *xp = nullptr,
                             const RowNorm *rn = nullptr);
// whether launch_gemm_multi takes a RowNorm for these matrices
bool gemm_rownorm_supported(int fmt, int K, const void *w, uint64_t stride);
// xp (optional): the normed rows also split into xp (as launch_split_rows),
// in the same launch where the row fits.
hipError_t launch_rms_norm_rows(const float *x, const float *w, float *out, int rows, int n, float eps, hipStream_t s,
                                float *clear0 = nullptr, size_t n0 = 0, float *clear1 = nullptr, size_t n1 = 0,
                                float *clear2 = nullptr, size_t n2 = 0, const XPlanes *xp = nullptr);
// Grouped by expert (MoE prefill): token tiles from launch_moe_group; W of expert e
// starts expert_stride bytes after W of expert e - 1; x row = id / x_div, y row = id.
hipError_t launch_gemm_grouped(int fmt, const uint8_t *w, const uint8_t *w2, uint64_t stride, uint64_t expert_stride,
                               const float *x, int ldx, int x_div, float *y, int ldy, int N, int K, int out,
                               const int *tiles, const int *list, const int *ntiles, int max_tiles, hipStream_t s);
// Exact-code MFMA kernel (zh_qgemm.hip) for the quantized formats, K a multiple of 256.
bool qgemm_supported(int fmt, int K, const void *w, const void *w2, uint64_t stride, uint64_t expert_stride);
hipError_t launch_qgemm(int fmt, const uint8_t *w, const uint8_t *w2, uint64_t stride, const float *x, int ldx,
                        float *y, int ldy, int M, int N, int K, int out, unsigned long long *argmax, hipStream_t s,
                        int max_split = 16, const XPlanes *xp = nullptr);
// Up to three matrices of one format, row stride and reduction length against
// one input in one launch (matrix i: rows N[i], output y[i] with row stride ldy[i]).
hipError_t launch_qgemm_multi(int fmt, int nseg, const uint8_t *const *w, float *const *y, const int *ldy,
                              const int *N, const uint8_t *w2, uint64_t stride, const float *x, int ldx, int M, int K,
                              int out, unsigned long long *argmax, hipStream_t s, int max_split = 16,
                              const XPlanes *xp = nullptr, const RowNorm *rn = nullptr);
hipError_t launch_qgemm_grouped(int fmt, const uint8_t *w, const uint8_t *w2, uint64_t stride,
                                uint64_t expert_stride, const float *x, int ldx, int x_div, float *y, int ldy, int N,
                                int K, int out, const int *tiles, const int *list, const int *ntiles, int max_tiles,
                                hipStream_t s);
hipError_t launch_moe_group(const uint32_t *route, int route_stride, int M, int k, int E, int *list, int *tiles,
                            int *ntiles, hipStream_t s);

// MoE routing and combine (zh_moe.hip)
// `tokens` rows: logits row t at logits + t * logits_stride, route row t at route + t * (2k + 2)
hipError_t launch_moe_route(const float *logits, int E, int k, int gating, int weights_norm, float weights_scale,
                            int has_shared_gate, uint32_t *route, hipStream_t s, int tokens = 1,
                            int logits_stride = 0);
// hidden[t] += combine of tmp rows t * k .. t * k + k - 1 (and shared row sh_tmp[t]) for `tokens` rows
hipError_t launch_moe_combine(float *hidden, const float *tmp, const uint32_t *route, int H, int k, int has_shared,
                              hipStream_t s, int tokens = 1, const float *sh_tmp = nullptr);

// attention (zh_attn.hip)
struct AttnParams {
    const float *q;            // [head_count * head_dim]: raw projection (fused) or roped q (plain)
    __half *k_cache;           // layer base applied: [rows][kv_dim], row = kv_row(position)
    __half *v_cache;
    // paged cache: position t lives in row (page_table[t >> page_shift] << page_shift) + (t & page mask);
    // a contiguous cache passes an identity table (kIdentityPages entries per context)
    const uint32_t *page_table;
    int page_shift;
    float *out;                // [head_count * head_dim]
    float *part_o;             // [kv_heads][max_splits][8][head_dim]
    float *part_ml;            // [kv_heads][max_splits][8][2]
    unsigned *counters;        // [kv_heads] arrival counters, zero between launches
    int head_count, head_count_kv, head_dim, kv_dim;
    int position;              // attend to [window_start, position]
    const int *position_dev;   // if set, position is read from device memory (graph replay)
    int window_start;
    float scale;
    int max_splits;            // grid width; splits used grow with the position up to this
    // fused mode (k_new set): q/k/v epilogue of the projection and the K/V store
    const float *k_new, *v_new;              // [kv_dim] raw k and v of this step
    const float *q_bias, *k_bias, *v_bias;   // optional
    const float *q_norm, *k_norm;            // optional per-head RMSNorm weights [head_dim]
    float eps, rope_base;
    const float *rope_denom;   // optional [n_rot / 2]: base^(2i / n_rot) from the host's powf (else powf here)
    int rope_dim, rope_style;
    int ctx;                   // cache capacity in positions (no store at or past it)
    // several queries (plain mode, matrix-core kernel): queries at positions
    // position .. position + n_query - 1, rows q_stride / out_stride floats apart
    int n_query, q_stride, out_stride;
    // Polled merge (single query, matrix-core kernel; no counters): every word
    // of part_o / part_ml starts as kPollEmpty, the splits store their partials
    // with device-scope stores, and each split merges its own slice of the
    // head's outputs as soon as every split's partials of that slice are there.
    // The launch refills the other set (reset_o / reset_ml, laid out as
    // part_o / part_ml) with kPollEmpty for the next launch; `poll_err` is set
    // when a wait runs out of its bound (a split never came), and the output
    // is then not valid.
    float *reset_o, *reset_ml;
    int *poll_err;
    int poll_merge;
    int min_tiles;  // 32-position tiles per split at least (0: the default)
    // launch_qkv_attention: the next launch's q / k / v words ([q][k][v], laid
    // out as q, k_new and v_new), refilled with kPollEmpty by this one
    float *qkv_refill;
};
constexpr uint32_t kPollEmpty = 0xFFFFFFFFu;  // a NaN pattern no arithmetic here produces
hipError_t launch_attention(const AttnParams &p, hipStream_t s);
// A decode step's q/k/v projection (qkv: fused RMSNorm, up to three segments
// in at most two formats, plain stores) and its single-query attention
// (fused mode with the polled merge) in one launch (qkv_attn_kernel): the
// projection workgroups store q, k and v with device-scope stores, the
// attention workgroups issue their K loads first and read their head's q, k
// and v as they land.  Every q/k/v word (a.q, a.k_new, a.v_new: the
// segments' outputs) must hold kPollEmpty before the launch; the launch
// refills a.qkv_refill (the same layout) for the next one.
hipError_t launch_qkv_attention(const MvParams &qkv, const AttnParams &a, hipStream_t s, bool v_now = false);
// whether a decode from `position` wants launch_qkv_attention's v_now variant
// (the V tiles issued right after the q/k/v wait, for long contexts)
bool qkv_attention_v_now(int position, int max_splits);
// whether launch_qkv_attention serves these formats (q's, and the other
// segments' if different) and shapes
bool qkv_attention_supported(int f1, int f2, int hidden, int head_dim, int group);
// The polled merge covers the single-query matrix-core kernel with at most 64 splits.
bool attention_poll_supported(int head_dim, int max_splits);
// Minimum tiles per split of a polled launch (ZIGGY_HIP_ATTN_MIN_TILES, a tuning knob; default 6).
int attention_poll_min_tiles();
constexpr int kKvPageShift = 6;  // a session's KV page: 64 positions (two 32-position attention tiles)
constexpr int kIdentityPages = 65536;  // a context's identity table: contiguous caches of up to 4M positions
hipError_t launch_iota_u32(uint32_t *p, int n, hipStream_t s);
// q/k/v epilogue of n_query tokens (rows q_stride / kv_dim apart): roped q to
// q_out (may be q), k and v stored to the cache at position + m.
// rs: the q/k/v rows come from products with a deferred norm (RowNorm): each
// token's row is scaled first.  z: spans cleared on the way.
hipError_t launch_attention_prep(const AttnParams &p, float *q_out, hipStream_t s, RowScale rs = RowScale{},
                                 const ZeroSpans &z = ZeroSpans{});
bool attention_multi_supported(int head_dim);
// workgroups along the query axis of a multi-query launch (its partials and
// arrival counters: head_count_kv * groups slots of kMultiHeads heads each)
int attention_query_groups(int head_count, int head_count_kv, int n_query);
constexpr int kMultiHeads = 16;  // (query, head) pairs per multi-query workgroup
// Splits of the attention grid for kv_heads heads and up to max_positions keys.
int attention_splits(int kv_heads, int max_positions);
size_t attention_scratch_floats(int head_count, int head_dim, int max_splits);
// Validates a bridge-level attention call (ziggy_hip_attention_fused_f32's
// arguments) and fills every field of *p but the partials and counters.
int attention_call_params(const ZiggyHipBuffer *q, const ZiggyHipBuffer *kc, const ZiggyHipBuffer *vc,
                          const ZiggyHipBuffer *out, uint32_t heads, uint32_t heads_kv, uint32_t hd, uint32_t kv_dim,
                          uint32_t ctx_len, uint32_t pos, uint32_t layer_base, uint32_t window_start, float scale,
                          float softcap, AttnParams *p, char *err, size_t err_len);
// Per-device address of the allocation-free attention's static scratch;
// called once per device by context creation, with that device current.
int noalloc_init_device(int device, char *err, size_t err_len);

}  // namespace zh
