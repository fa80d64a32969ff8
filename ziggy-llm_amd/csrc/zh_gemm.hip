// zh_gemm.hip -- the dense path for M >= 8 tokens (speculative verify,
// prefill, grouped MoE experts) on the matrix cores.
//
//   Y[m][n] (=, +=) sum_k W[n][k] * X[m][k]     for tokens m < M, rows n < N
//
// W is a quantized (or f16/f32) GGUF matrix in its native row layout; each
// lane decodes the four consecutive weights its MFMA A fragment needs with
// the bit-exact decoders of zh_quant.h (dequant_value: the reference's own
// binary32 operation order).  Weights and activations enter the matrix
// cores as bf16 pairs: v = hi + lo with hi = bf16(v), lo = bf16(v - hi),
// and each 16x16x16 tile accumulates hi*hi + hi*lo + lo*hi in f32 -- about
// 16 significant bits per operand, so the products carry ~2^-16 relative
// error (lo*lo, below that, is dropped).  Accumulation is f32.
//
// Tiling: a workgroup computes 16 rows x 16 tokens over the whole reduction
// dimension; its four wavefronts take interleaved 16-value steps of K and
// their partial tiles meet in LDS.  The grid has up to 1024 row tiles (more
// rows loop) by ceil(M / 16) token tiles.  Decode-sized M (8 .. 16) keeps
// the kernel bound by the weight stream; the token tile is re-read from L2.
//
// MFMA operand layout (v_mfma_f32_16x16x16_bf16, wave64): lane l holds
// A[l % 16][4 (l / 16) + 0..3], B[4 (l / 16) + 0..3][l % 16], and the result
// D[4 (l / 16) + 0..3][l % 16].  Here A = the row tile of W, B = the token
// tile of X transposed, D[i][j] = Y[token j][row i].
#include <cstdlib>

#include "zh_internal.h"
#include "zh_quant.h"

namespace zh {

typedef short bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// bf16 round-to-nearest-even of a finite f32 (the bits of the upper half).
__device__ __forceinline__ uint32_t bf16_bits(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

// hi / lo bf16 halves of four values, packed as MFMA operands.
__device__ __forceinline__ void split4(const float (&v)[4], bf16x4 &hi, bf16x4 &lo) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t h = bf16_bits(v[i]);
        const float r = v[i] - __uint_as_float(h << 16);
        hi[i] = (short)h;
        lo[i] = (short)bf16_bits(r);
    }
}

// Weights k .. k+3 (k a multiple of 4) of one row, bit-exact.
template <int F> __device__ __forceinline__ void weights4(const uint8_t *__restrict__ row, int k, float (&w)[4]) {
    if constexpr (F == F32) {
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = __uint_as_float(ld4(row + 4 * (k + i)));
    } else if constexpr (F == F16) {
        const uint2 v = ld8(row + 2 * k);
        w[0] = h2f(v.x), w[1] = h2f(v.x >> 16), w[2] = h2f(v.y), w[3] = h2f(v.y >> 16);
    } else {
        constexpr int V = Geom<F>::kValues, B = Geom<F>::kBytes;
        const uint8_t *blk = row + (size_t)(k / V) * B;
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = dequant_value<F>(blk, k % V + i);
    }
}

struct GemmParams {
    const uint8_t *w;     // W row 0
    const uint8_t *w2;    // SWIGLU: the up matrix (same format and shape)
    uint64_t stride;      // bytes per W row
    const float *x;       // [M][ldx]
    float *y;             // [M][ldy]
    int M, N, K, ldx, ldy;
    unsigned long long *argmax;  // ARGMAX: [M] packed (ordered value << 32 | ~row)
    // grouped (experts): token tile t of blockIdx.y is group_tiles[t] = {expert, first, count};
    // its tokens are group_list[first .. first + count), x row = id / x_div, y row = id
    const int *group_tiles, *group_list, *group_ntiles;
    int x_div;
    uint64_t expert_stride;  // bytes between consecutive experts' W
};

__device__ __forceinline__ uint32_t ordered_bits_g(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// PRECISE: f32 operands on v_mfma_f32_16x16x4_f32 (products as exact as the
// matvec path's fmaf), four instructions per 16-value step: instruction i
// takes value 4 (l / 16) + i of each lane, so the four together cover the
// same 16 reduction indices as the bf16 instructions.  Used where a result
// feeds a discrete choice (the MoE router's top-k).
template <int F, int OUT, bool GROUPED, bool PRECISE = false>
__global__ void __launch_bounds__(256) gemm_kernel(GemmParams p) {
    constexpr bool kPair = OUT == OUT_SWIGLU;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lq = lane >> 4;
    int m0 = blockIdx.y * 16, M = p.M;
    const int *ids = nullptr;
    if (GROUPED) {
        // one expert's token tile: up to 16 of its routed (token, slot) ids
        if ((int)blockIdx.y >= *p.group_ntiles) return;
        const int *gt = p.group_tiles + 3 * blockIdx.y;
        p.w += (uint64_t)gt[0] * p.expert_stride;
        if (kPair) p.w2 += (uint64_t)gt[0] * p.expert_stride;
        ids = p.group_list + gt[1];
        m0 = 0;
        M = gt[2];
    }
    const int m = min(m0 + li, M - 1);  // this lane's X token (clamped; dropped at the store)
    const float *xrow = p.x + (size_t)(GROUPED ? ids[m] / p.x_div : m) * p.ldx;
    const int j = m0 + li;                // token of this lane's results
    const int jrow = GROUPED ? (j < M ? ids[j] : 0) : j;  // its y row
    __shared__ float part[4][kPair ? 2 : 1][64][4];
    float best = -INFINITY;
    int best_n = 0x7fffffff;
    const int ntiles = (p.N + 15) / 16;
    // row tiles n0 = 16 * (blockIdx.x + t * gridDim.x)
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int n0 = 16 * tile;
        const int n = min(n0 + li, p.N - 1);  // this lane's W row (clamped)
        const uint8_t *wrow = p.w + (uint64_t)n * p.stride;
        const uint8_t *wrow2 = kPair ? p.w2 + (uint64_t)n * p.stride : nullptr;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
        for (int k = 16 * wave + 4 * lq; k < p.K; k += 64) {
            float wv[4], xv[4];
            weights4<F>(wrow, k, wv);
            const float4 xx = *reinterpret_cast<const float4 *>(xrow + k);
            xv[0] = xx.x, xv[1] = xx.y, xv[2] = xx.z, xv[3] = xx.w;
            if constexpr (PRECISE && !kPair) {
#pragma unroll
                for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[i], xv[i], acc, 0, 0, 0);
                continue;
            }
            bf16x4 ah, al, bh, bl;
            split4(wv, ah, al);
            split4(xv, bh, bl);
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bl, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al, bh, acc, 0, 0, 0);
            if (kPair) {
                weights4<F>(wrow2, k, wv);
                split4(wv, ah, al);
                acc2 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bh, acc2, 0, 0, 0);
                acc2 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bl, acc2, 0, 0, 0);
                acc2 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al, bh, acc2, 0, 0, 0);
            }
        }
        // the four wavefronts' partial tiles meet in LDS
#pragma unroll
        for (int r = 0; r < 4; r++) {
            part[wave][0][lane][r] = acc[r];
            if (kPair) part[wave][kPair ? 1 : 0][lane][r] = acc2[r];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float v = (part[0][0][lane][r] + part[1][0][lane][r]) + (part[2][0][lane][r] + part[3][0][lane][r]);
                const int nn = n0 + 4 * lq + r;  // row of result r
                if (j >= M || nn >= p.N) continue;
                float *dst = p.y ? p.y + (size_t)jrow * p.ldy + nn : nullptr;
                if (OUT == OUT_STORE) {
                    *dst = v;
                } else if (OUT == OUT_ADD) {
                    *dst = *dst + v;
                } else if (OUT == OUT_SWIGLU) {
                    const int c = kPair ? 1 : 0;
                    const float u =
                        (part[0][c][lane][r] + part[1][c][lane][r]) + (part[2][c][lane][r] + part[3][c][lane][r]);
                    *dst = (v / (1.0f + expf(-v))) * u;
                } else if (OUT == OUT_ARGMAX) {
                    if (dst) *dst = v;
                    if (v > best || (v == best && nn < best_n)) {
                        best = v;
                        best_n = nn;
                    }
                }
            }
        }
        __syncthreads();  // part is reused by the next tile
    }
    if (OUT == OUT_ARGMAX && wave == 0) {
        // lanes j, j + 16, j + 32, j + 48 hold this token's rows; the packed
        // maximum picks the largest value, then the lowest row
        unsigned long long key = best_n == 0x7fffffff ? 0ull
                                 : ((unsigned long long)ordered_bits_g(best) << 32) |
                                       (unsigned long long)(0xFFFFFFFFu - (uint32_t)best_n);
        unsigned long long o = __shfl_xor(key, 16, 64);
        key = o > key ? o : key;
        o = __shfl_xor(key, 32, 64);
        key = o > key ? o : key;
        if (lq == 0 && j < M && key) atomicMax(p.argmax + jrow, key);
    }
}

typedef void (*GemmKernel)(GemmParams);

template <int F> static GemmKernel pick_gemm(int out) {
    switch (out) {
    case OUT_STORE: return gemm_kernel<F, OUT_STORE, false>;
    case OUT_ADD: return gemm_kernel<F, OUT_ADD, false>;
    case OUT_SWIGLU: return gemm_kernel<F, OUT_SWIGLU, false>;
    case OUT_ARGMAX: return gemm_kernel<F, OUT_ARGMAX, false>;
    default: return nullptr;
    }
}
template <int F> static GemmKernel pick_grouped(int out) {
    switch (out) {
    case OUT_STORE: return gemm_kernel<F, OUT_STORE, true>;
    case OUT_SWIGLU: return gemm_kernel<F, OUT_SWIGLU, true>;
    default: return nullptr;
    }
}

// ZIGGY_HIP_QGEMM=0 keeps every M >= 8 product on this file's kernel (the
// exact-code kernel of zh_qgemm.hip otherwise takes the quantized formats).
static bool qgemm_enabled() {
    static const bool on = [] {
        const char *e = getenv("ZIGGY_HIP_QGEMM");
        return !(e && e[0] == '0');
    }();
    return on;
}

template <int F> static GemmKernel pick_precise(int out) {
    return out == OUT_STORE ? gemm_kernel<F, OUT_STORE, false, true> : nullptr;
}

hipError_t launch_gemm(int fmt, const uint8_t *w, const uint8_t *w2, uint64_t stride, const float *x, int ldx,
                       float *y, int ldy, int M, int N, int K, int out, unsigned long long *argmax, hipStream_t s,
                       bool precise, int max_split, const XPlanes *xp) {
    if (M < 1 || N < 1 || K < 16 || K % 16 || ldx % 4) return hipErrorInvalidValue;
    if (!precise && qgemm_enabled() && qgemm_supported(fmt, K, w, w2, stride, 0))
        return launch_qgemm(fmt, w, w2, stride, x, ldx, y, ldy, M, N, K, out, argmax, s, max_split, xp);
    GemmKernel k = nullptr;
    if (precise) {
        switch (fmt) {
        case Q4_K: k = pick_precise<Q4_K>(out); break;
        case Q6_K: k = pick_precise<Q6_K>(out); break;
        case Q8_0: k = pick_precise<Q8_0>(out); break;
        case Q3_K: k = pick_precise<Q3_K>(out); break;
        case IQ4_XS: k = pick_precise<IQ4_XS>(out); break;
        case F16: k = pick_precise<F16>(out); break;
        case F32: k = pick_precise<F32>(out); break;
        default: break;
        }
        fmt = -1;  // chosen
    }
    switch (fmt) {
    case Q4_K: k = pick_gemm<Q4_K>(out); break;
    case Q6_K: k = pick_gemm<Q6_K>(out); break;
    case Q8_0: k = pick_gemm<Q8_0>(out); break;
    case Q3_K: k = pick_gemm<Q3_K>(out); break;
    case IQ4_XS: k = pick_gemm<IQ4_XS>(out); break;
    case F16: k = pick_gemm<F16>(out); break;
    case F32: k = pick_gemm<F32>(out); break;
    default: break;
    }
    if (!k) return hipErrorInvalidValue;
    GemmParams p{w, w2, stride, x, y, M, N, K, ldx, ldy, argmax, nullptr, nullptr, nullptr, 1, 0};
    // at most 1024 row tiles in flight per token tile; larger N loops (grid-stride)
    const int tiles = (N + 15) / 16;
    hipLaunchKernelGGL(k, dim3(tiles < 1024 ? tiles : 1024, (M + 15) / 16), dim3(256), 0, s, p);
    return hipGetLastError();
}

bool gemm_rownorm_supported(int fmt, int K, const void *w, uint64_t stride) {
    return qgemm_enabled() && qgemm_supported(fmt, K, w, nullptr, stride, 0);
}

hipError_t launch_gemm_multi(int fmt, int nseg, const uint8_t *const *w, float *const *y, const int *ldy,
                             const int *N, uint64_t stride, const float *x, int ldx, int M, int K, int out,
                             hipStream_t s, int max_split, const XPlanes *xp, const RowNorm *rn) {
    if (nseg < 1 || nseg > 3 || (out != OUT_STORE && out != OUT_ADD)) return hipErrorInvalidValue;
    bool one = qgemm_enabled();
    for (int i = 0; i < nseg && one; i++) one = qgemm_supported(fmt, K, w[i], nullptr, stride, 0);
    if (one)
        return launch_qgemm_multi(fmt, nseg, w, y, ldy, N, nullptr, stride, x, ldx, M, K, out, nullptr, s, max_split,
                                  xp, rn);
    if (rn) return hipErrorInvalidValue;  // the other kernels take normed rows
    for (int i = 0; i < nseg; i++) {
        const hipError_t e = launch_gemm(fmt, w[i], nullptr, stride, x, ldx, y[i], ldy[i], M, N[i], K, out, nullptr, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gemm_grouped(int fmt, const uint8_t *w, const uint8_t *w2, uint64_t stride, uint64_t expert_stride,
                               const float *x, int ldx, int x_div, float *y, int ldy, int N, int K, int out,
                               const int *tiles, const int *list, const int *ntiles, int max_tiles, hipStream_t s) {
    if (N < 1 || K < 16 || K % 16 || ldx % 4 || max_tiles < 1 || x_div < 1) return hipErrorInvalidValue;
    if (qgemm_enabled() && qgemm_supported(fmt, K, w, w2, stride, expert_stride))
        return launch_qgemm_grouped(fmt, w, w2, stride, expert_stride, x, ldx, x_div, y, ldy, N, K, out, tiles, list,
                                    ntiles, max_tiles, s);
    GemmKernel k = nullptr;
    switch (fmt) {
    case Q4_K: k = pick_grouped<Q4_K>(out); break;
    case Q6_K: k = pick_grouped<Q6_K>(out); break;
    case Q8_0: k = pick_grouped<Q8_0>(out); break;
    case Q3_K: k = pick_grouped<Q3_K>(out); break;
    case IQ4_XS: k = pick_grouped<IQ4_XS>(out); break;
    default: break;
    }
    if (!k) return hipErrorInvalidValue;
    GemmParams p{w, w2, stride, x, y, 16, N, K, ldx, ldy, nullptr, tiles, list, ntiles, x_div, expert_stride};
    const int rt = (N + 15) / 16;
    hipLaunchKernelGGL(k, dim3(rt < 1024 ? rt : 1024, max_tiles), dim3(256), 0, s, p);
    return hipGetLastError();
}

// Groups the routed (token, slot) assignments of M tokens by expert.  Route
// row t (route_stride words) holds the k {id, weight} entries of token t;
// assignment a = t * k + s.  Writes list (the assignments grouped by expert;
// within an expert in arrival order, which does not change any result: each
// token's output column depends only on its own operands), tiles
// {expert, first, count} of at most 16 assignments in expert order, and
// their number.  One workgroup of 1024: one expert per thread for the
// counts' scan, up to four assignments per thread.
constexpr int kGroupMaxAssign = 4096;

__global__ void __launch_bounds__(1024) moe_group_kernel(const uint32_t *__restrict__ route, int route_stride, int M,
                                                         int k, int E, int *__restrict__ list, int *__restrict__ tiles,
                                                         int *__restrict__ ntiles) {
    __shared__ int cnt[1024];
    __shared__ int wsum[2][16];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = M * k;
    cnt[t] = 0;
    __syncthreads();
    int pos[4], ex[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int a = t + 1024 * i;
        ex[i] = -1;
        pos[i] = 0;
        if (a < n) {
            const uint32_t e = route[(size_t)(a / k) * route_stride + 2 * (a % k)];
            if (e < (uint32_t)E) {
                ex[i] = (int)e;
                pos[i] = atomicAdd(&cnt[e], 1);
            }
        }
    }
    __syncthreads();
    // inclusive scans of the counts and of the tiles per expert
    const int c = t < E ? cnt[t] : 0, tc = (c + 15) >> 4;
    int sc = c, st = tc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int vc = __shfl_up(sc, o, 64), vt = __shfl_up(st, o, 64);
        if (lane >= o) sc += vc, st += vt;
    }
    if (lane == 63) wsum[0][wave] = sc, wsum[1][wave] = st;
    __syncthreads();
    for (int w = 0; w < wave; w++) sc += wsum[0][w], st += wsum[1][w];
    const int off = sc - c, toff = st - tc;
    if (t == 1023) *ntiles = st;
    __syncthreads();  // every count read before the offsets replace them
    cnt[t] = off;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (ex[i] >= 0) list[cnt[ex[i]] + pos[i]] = t + 1024 * i;
    for (int f = 0; f < tc; f++) {
        int *d = tiles + 3 * (toff + f);
        d[0] = t;
        d[1] = off + 16 * f;
        d[2] = min(16, c - 16 * f);
    }
}

hipError_t launch_moe_group(const uint32_t *route, int route_stride, int M, int k, int E, int *list, int *tiles,
                            int *ntiles, hipStream_t s) {
    if (E < 1 || E > 1024 || M < 1 || k < 1 || M * k > kGroupMaxAssign) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(1024), 0, s, route, route_stride, M, k, E, list, tiles, ntiles);
    return hipGetLastError();
}

// Per-token RMSNorm of M rows (rmsNorm, model/loader.zig:3404-3426, for each
// token): out[m] = (scale_m * x[m]) * w; one workgroup per token.  V: rows of
// up to 8192 values (multiples of 4, 16-byte aligned) held in registers, every
// load in flight at once.  The workgroups also clear up to three float ranges
// (outputs that products then accumulate onto).  SPLIT (V rows of up to
// 4096 values, a multiple of 32): the normed row also goes out as the GEMM's
// pieces (XPlanes), through LDS, one 16-value run per thread as
// split_rows_kernel splits it: the same values, pieces and sums.
struct NormClear {
    float *p[3];
    size_t n[3];
};
constexpr int kNormSplitMax = 4096;
template <bool V, bool SPLIT = false>
__global__ void __launch_bounds__(256) rms_norm_rows_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                            float *__restrict__ out, int n, float eps, NormClear cl,
                                                            XPlanes xp = XPlanes{}) {
    static_assert(!SPLIT || V, "the split takes the register rows");
    const int tid = threadIdx.x;
    const float *xr = x + (size_t)blockIdx.x * n;
    float *orow = out + (size_t)blockIdx.x * n;
    __shared__ float red[4];
    float ss = 0.f;
    float4 v[8], wv[8];
    const int n4 = n / 4;
    if (V) {
        const float4 *x4 = reinterpret_cast<const float4 *>(xr), *w4 = reinterpret_cast<const float4 *>(w);
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = x4[min(tid + 256 * j, n4 - 1)];
#pragma unroll
        for (int j = 0; j < 8; j++) wv[j] = w4[min(tid + 256 * j, n4 - 1)];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (tid + 256 * j < n4)
                ss = fmaf(v[j].w, v[j].w, fmaf(v[j].z, v[j].z, fmaf(v[j].y, v[j].y, fmaf(v[j].x, v[j].x, ss))));
    } else {
        for (int i = tid; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
    }
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
    if (V) {
        float4 *o4 = reinterpret_cast<float4 *>(orow);
        __shared__ __align__(16) float rowv[SPLIT ? kNormSplitMax : 4];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (tid + 256 * j < n4) {
                const float4 o = {(scale * v[j].x) * wv[j].x, (scale * v[j].y) * wv[j].y, (scale * v[j].z) * wv[j].z,
                                  (scale * v[j].w) * wv[j].w};
                o4[tid + 256 * j] = o;
                if (SPLIT) *reinterpret_cast<float4 *>(&rowv[4 * (tid + 256 * j)]) = o;
            }
        if constexpr (SPLIT) {
            __syncthreads();
            const int runs = n >> 4, r = min(tid, runs - 1);
            float rv[16];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4 q = *reinterpret_cast<const float4 *>(&rowv[16 * r + 4 * c]);
                rv[4 * c] = q.x, rv[4 * c + 1] = q.y, rv[4 * c + 2] = q.z, rv[4 * c + 3] = q.w;
            }
            uint32_t hw[8], lw[8];
            float sum = split_run16(rv, hw, lw);
            sum += __shfl_xor(sum, 1, 64);  // the other run of the 32-value sum
            if (tid < runs) {
                uint4 *dh = reinterpret_cast<uint4 *>(xp.hi + (size_t)blockIdx.x * xp.ld + 16 * r);
                uint4 *dl = reinterpret_cast<uint4 *>(xp.lo + (size_t)blockIdx.x * xp.ld + 16 * r);
                dh[0] = {hw[0], hw[1], hw[2], hw[3]};
                dh[1] = {hw[4], hw[5], hw[6], hw[7]};
                dl[0] = {lw[0], lw[1], lw[2], lw[3]};
                dl[1] = {lw[4], lw[5], lw[6], lw[7]};
                if (!(r & 1)) xp.sum[(size_t)blockIdx.x * (xp.ld / 32) + (r >> 1)] = sum;
            }
        }
    } else {
        for (int i = tid; i < n; i += 256) orow[i] = (scale * xr[i]) * w[i];
    }
#pragma unroll
    for (int r = 0; r < 3; r++)
        for (size_t i = (size_t)blockIdx.x * 256 + tid; i < cl.n[r]; i += (size_t)gridDim.x * 256) cl.p[r][i] = 0.f;
}

hipError_t launch_rms_norm_rows(const float *x, const float *w, float *out, int rows, int n, float eps, hipStream_t s,
                                float *clear0, size_t n0, float *clear1, size_t n1, float *clear2, size_t n2,
                                const XPlanes *xp) {
    if (rows < 1 || n < 1 || (n0 && !clear0) || (n1 && !clear1) || (n2 && !clear2)) return hipErrorInvalidValue;
    const NormClear cl{{clear0, clear1, clear2}, {n0, n1, n2}};
    const bool v = n % 4 == 0 && n <= 8 * 256 * 4 && ((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) % 16 == 0;
    if (xp) {
        // the split in the norm's launch where it fits, else a split launch after it
        if (v && n % 32 == 0 && n <= kNormSplitMax && xp->hi && xp->lo && xp->sum && xp->ld % 32 == 0 && xp->ld >= n) {
            hipLaunchKernelGGL((rms_norm_rows_kernel<true, true>), dim3(rows), dim3(256), 0, s, x, w, out, n, eps, cl,
                               *xp);
            return hipGetLastError();
        }
        hipError_t e = launch_rms_norm_rows(x, w, out, rows, n, eps, s, clear0, n0, clear1, n1, clear2, n2);
        return e != hipSuccess ? e : launch_split_rows(out, n, rows, n, *xp, s);
    }
    if (v)
        hipLaunchKernelGGL(rms_norm_rows_kernel<true>, dim3(rows), dim3(256), 0, s, x, w, out, n, eps, cl);
    else
        hipLaunchKernelGGL(rms_norm_rows_kernel<false>, dim3(rows), dim3(256), 0, s, x, w, out, n, eps, cl);
    return hipGetLastError();
}

}  // namespace zh
