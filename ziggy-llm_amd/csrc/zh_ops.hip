// zh_ops.hip -- small decode-step kernels: norms, RoPE, binary16 KV store,
// SwiGLU, residual add, greedy argmax and the MoE routing helpers.
//
// Semantics follow the reference's CPU path (model/loader.zig) and, where the
// GPU entry point has its own contract, the Metal kernels it replaces
// (runtime/metal/matvec.metal); each kernel cites its source.
#include "zh_internal.h"
#include "zh_quant.h"

namespace zh {

__device__ __forceinline__ float block_sum(float v, float *lds) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    if ((threadIdx.x & 63) == 0) lds[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += lds[i];
    __syncthreads();
    return t;
}

// rmsNorm (model/loader.zig:3404-3426): out = (scale * x) * (w + offset).
__global__ void rms_norm_kernel(const float *__restrict__ x, const float *__restrict__ w, float *__restrict__ out,
                                int n, float eps, float off) {
    __shared__ float lds[16];
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(x[i], x[i], ss);
    ss = block_sum(ss, lds);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = (scale * x[i]) * (w[i] + off);
}

// rmsNormPerHeadWithOffset (model/loader.zig:1777-1812); one workgroup per head.
__global__ void rms_norm_per_head_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                         float *__restrict__ out, int hd, float eps, float off) {
    __shared__ float lds[16];
    const float *hx = x + (size_t)blockIdx.x * hd;
    float *ho = out + (size_t)blockIdx.x * hd;
    float ss = 0.f;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) ss = fmaf(hx[i], hx[i], ss);
    ss = block_sum(ss, lds);
    const float scale = 1.0f / sqrtf(ss / (float)hd + eps);
    for (int i = threadIdx.x; i < hd; i += blockDim.x) ho[i] = (scale * hx[i]) * (w[i] + off);
}

// applyRoPE (model/loader.zig:3827-3866): style 0 rotates pairs (2i, 2i+1),
// style 1 (NeoX) rotates (i, i + n_rot/2); theta = pos / base^(2i / n_rot).
// Dimensions at or beyond n_rot are copied unchanged.
__global__ void rope_kernel(const float *__restrict__ src, float *__restrict__ dst, int heads, int hd, int n_rot,
                            float pos, const float *__restrict__ denom, int style) {
    const int half = n_rot / 2;
    const int tid = blockIdx.x * blockDim.x + threadIdx.x;
    const int per_head = hd - half;  // pairs + untouched tail entries
    if (tid >= heads * per_head) return;
    const int h = tid / per_head, i = tid % per_head;
    const float *s = src + (size_t)h * hd;
    float *d = dst + (size_t)h * hd;
    if (i < half) {
        const int a = style == 0 ? 2 * i : i, b = style == 0 ? 2 * i + 1 : i + half;
        const float theta = pos / denom[i];
        const float c = cosf(theta), sn = sinf(theta);
        const float x0 = s[a], x1 = s[b];
        d[a] = fmaf(x0, c, -x1 * sn);
        d[b] = fmaf(x0, sn, x1 * c);
    } else {
        const int t = n_rot + (i - half);
        if (t < hd && src != dst) d[t] = s[t];
    }
}

// store_kv_half (matvec.metal:246-255): f32 -> binary16, round to nearest even.
__global__ void store_kv_half_kernel(const float *__restrict__ src, __half *__restrict__ dst, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = __float2half_rn(src[i]);
}

// siluInPlace then gate *= up (model/loader.zig:1277-1279, 4004-4024).
__global__ void silu_mul_kernel(float *__restrict__ g, const float *__restrict__ u, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float v = g[i];
        g[i] = (v / (1.0f + expf(-v))) * u[i];
    }
}

// silu_mul over rows x n with the deferred norm of the gate/up products:
// g = silu(r g) * (r u), r the row's scale; then the spans z cleared.
__global__ void silu_mul_rows_kernel(float *__restrict__ g, const float *__restrict__ u, int rows, int n,
                                     RowScale rs, ZeroSpans z) {
    const size_t total = (size_t)rows * n, nthr = (size_t)gridDim.x * blockDim.x;
    const size_t gi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (size_t i = gi; i < total; i += nthr) {
        const int row = (int)(i / n);
        const float r = rs.ss ? 1.0f / sqrtf(rs.ss[row] / (float)rs.n + rs.eps) : 1.0f;
        const float v = r * g[i];
        g[i] = (v / (1.0f + expf(-v))) * (r * u[i]);
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
        for (size_t i = gi; i < z.n[j]; i += nthr) z.p[j][i] = 0.f;
}

__global__ void zero_spans_kernel(ZeroSpans z) {
    const size_t nthr = (size_t)gridDim.x * blockDim.x, gi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; j++)
        for (size_t i = gi; i < z.n[j]; i += nthr) z.p[j][i] = 0.f;
}

// Rows of x into the exact-code GEMM's pieces (split_run16): thread t takes
// run t of the row-major runs (16 values; n a multiple of 32, so the two runs
// of a 32-value sum sit in neighbouring lanes).  SILU: the values are
// silu(x) * up first (as silu_mul_kernel), also stored back into x.
template <bool SILU>
__global__ void split_rows_kernel(float *__restrict__ x, const float *__restrict__ up, int ldx, int rows, int n,
                                  XPlanes xp) {
    const int runs = n >> 4;
    const long long total = (long long)rows * runs;
    const long long gi = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const bool ok = gi < total;
    const long long g = ok ? gi : total - 1;  // past the end: the last run again, nothing stored
    const int row = (int)(g / runs), r = (int)(g - (long long)row * runs);
    float *src = x + (size_t)row * ldx + 16 * r;
    float v[16];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float4 q = reinterpret_cast<const float4 *>(src)[c];
        v[4 * c] = q.x, v[4 * c + 1] = q.y, v[4 * c + 2] = q.z, v[4 * c + 3] = q.w;
    }
    if (SILU) {
        const float *u = up + (size_t)row * ldx + 16 * r;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 q = reinterpret_cast<const float4 *>(u)[c];
            const float uq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float g0 = v[4 * c + i];
                v[4 * c + i] = (g0 / (1.0f + expf(-g0))) * uq[i];
            }
        }
        if (ok) {
#pragma unroll
            for (int c = 0; c < 4; c++)
                reinterpret_cast<float4 *>(src)[c] = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
        }
    }
    uint32_t hw[8], lw[8];
    float sum = split_run16(v, hw, lw);
    sum += __shfl_xor(sum, 1, 64);  // the other run of the 32-value sum
    if (ok) {
        uint4 *dh = reinterpret_cast<uint4 *>(xp.hi + (size_t)row * xp.ld + 16 * r);
        uint4 *dl = reinterpret_cast<uint4 *>(xp.lo + (size_t)row * xp.ld + 16 * r);
        dh[0] = {hw[0], hw[1], hw[2], hw[3]};
        dh[1] = {hw[4], hw[5], hw[6], hw[7]};
        dl[0] = {lw[0], lw[1], lw[2], lw[3]};
        dl[1] = {lw[4], lw[5], lw[6], lw[7]};
        if (!(r & 1)) xp.sum[(size_t)row * (xp.ld / 32) + (r >> 1)] = sum;
    }
}

__global__ void add_kernel(float *__restrict__ dst, const float *__restrict__ src, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = dst[i] + src[i];
}

__device__ __forceinline__ uint32_t ordered_bits_ops(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Greedy argmax, first maximum wins (model/loader.zig:3910-3920): per-workgroup
// best packed as (ordered value << 32 | ~index), merged with a 64-bit atomicMax.
__global__ void argmax_kernel(const float *__restrict__ x, int n, unsigned long long *slot) {
    __shared__ unsigned long long keys[256];
    unsigned long long best = 0ull;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const unsigned long long k =
            ((unsigned long long)ordered_bits_ops(x[i]) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
        best = k > best ? k : best;
    }
    keys[threadIdx.x] = best;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s && keys[threadIdx.x + s] > keys[threadIdx.x]) keys[threadIdx.x] = keys[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0 && keys[0]) atomicMax(slot, keys[0]);
}

// The same over `rows` rows of n values (ld apart): blockIdx.y is the row,
// slots[row] its packed (value, lowest index) key; slots start at zero.
__global__ void argmax_rows_kernel(const float *__restrict__ x, int n, int ld, unsigned long long *slots) {
    __shared__ unsigned long long keys[256];
    const float *xr = x + (size_t)blockIdx.y * ld;
    unsigned long long best = 0ull;
#pragma unroll 4
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const unsigned long long k =
            ((unsigned long long)ordered_bits_ops(xr[i]) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
        best = k > best ? k : best;
    }
    keys[threadIdx.x] = best;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s && keys[threadIdx.x + s] > keys[threadIdx.x]) keys[threadIdx.x] = keys[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0 && keys[0]) atomicMax(slots + blockIdx.y, keys[0]);
}

// Writes the token of a packed argmax slot (and the reference's {bits, token}
// state pair when state_pair != 0).
__global__ void argmax_finalize_kernel(const unsigned long long *slot, uint32_t *out, int state_pair) {
    const unsigned long long k = *slot;
    const uint32_t token = 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull);
    if (state_pair) {
        out[0] = (uint32_t)(k >> 32);
        out[1] = token;
    } else {
        out[0] = token;
    }
}

__global__ void iota_u32_kernel(uint32_t *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = (uint32_t)i;
}

__global__ void fill_u64_kernel(unsigned long long *p, unsigned long long v, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

struct Entry {
    uint32_t id;
    float score;
};

// Top-k shortlist (topk_f32, matvec.metal:1568-1651): descending scores, ties
// to the lower index; k rounds of a workgroup argmax over the remaining values.
__global__ void topk_kernel(const float *__restrict__ x, int n, int k, Entry *__restrict__ out,
                            unsigned char *__restrict__ taken) {
    __shared__ unsigned long long keys[256];
    for (int i = threadIdx.x; i < n; i += blockDim.x) taken[i] = 0;
    __syncthreads();
    for (int r = 0; r < k; r++) {
        unsigned long long best = 0ull;
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            if (taken[i]) continue;
            const unsigned long long key =
                ((unsigned long long)ordered_bits_ops(x[i]) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
            best = key > best ? key : best;
        }
        keys[threadIdx.x] = best;
        __syncthreads();
        for (int s = blockDim.x / 2; s > 0; s >>= 1) {
            if ((int)threadIdx.x < s && keys[threadIdx.x + s] > keys[threadIdx.x]) keys[threadIdx.x] = keys[threadIdx.x + s];
            __syncthreads();
        }
        const unsigned long long w = keys[0];
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t idx = 0xFFFFFFFFu - (uint32_t)(w & 0xFFFFFFFFull);
            out[r].id = idx;
            out[r].score = idx < (uint32_t)n ? x[idx] : -INFINITY;
            if (idx < (uint32_t)n) taken[idx] = 1;
        }
        __syncthreads();
    }
}

// normalize_topk_f32 (matvec.metal:1653-1696).
__global__ void normalize_topk_kernel(Entry *e, int k, int apply_softmax, int normalize, float scale) {
    if (threadIdx.x != 0 || k <= 0 || k > 64) return;
    float w[64];
    float total = 0.f, mx = -INFINITY;
    if (apply_softmax) {
        for (int i = 0; i < k; i++) mx = fmaxf(mx, e[i].score);
        for (int i = 0; i < k; i++) {
            w[i] = expf(e[i].score - mx);
            total += w[i];
        }
    } else {
        for (int i = 0; i < k; i++) {
            const float v = (isfinite(e[i].score) && e[i].score > 0.f) ? e[i].score : 0.f;
            w[i] = v;
            total += v;
        }
    }
    if (!(total > 0.f) || !isfinite(total)) {
        for (int i = 0; i < k; i++) e[i].score = 0.f;
        return;
    }
    const float inv = normalize ? 1.0f / total : 1.0f;
    for (int i = 0; i < k; i++) e[i].score = w[i] * inv * scale;
}

// weighted_sum_topk_f32 (matvec.metal:1808-1818).
__global__ void weighted_sum_topk_kernel(float *dst, const float *src, const Entry *e, int n, int slot) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] += src[i] * e[slot].score;
}

// sigmoid_scale_add_f32 (matvec.metal:1820-1830); sigmoid as sigmoidScalar
// (model/loader.zig:4026-4033).
__global__ void sigmoid_scale_add_kernel(float *dst, const float *src, const float *scalar, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = scalar[0];
    float g;
    if (v >= 0.f) {
        g = 1.0f / (1.0f + expf(-v));
    } else {
        const float e = expf(v);
        g = e / (1.0f + e);
    }
    dst[i] += src[i] * g;
}

static inline int cdiv(long long a, int b) { return (int)((a + b - 1) / b); }

hipError_t launch_rms_norm(const float *x, const float *w, float *out, int n, float eps, float off, hipStream_t s) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(1024), 0, s, x, w, out, n, eps, off);
    return hipGetLastError();
}
hipError_t launch_rms_norm_per_head(const float *x, const float *w, float *out, int heads, int hd, float eps,
                                    float off, hipStream_t s) {
    hipLaunchKernelGGL(rms_norm_per_head_kernel, dim3(heads), dim3(hd >= 256 ? 256 : 64 * ((hd + 63) / 64)), 0, s,
                       x, w, out, hd, eps, off);
    return hipGetLastError();
}
hipError_t launch_rope(const float *src, float *dst, int heads, int hd, int rope_dim, int pos, const float *denom,
                       int style, hipStream_t s) {
    const int n_rot = rope_dim < hd ? rope_dim : hd;
    const int per_head = hd - n_rot / 2;
    const int n = heads * per_head;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, src, dst, heads, hd, n_rot, (float)pos, denom,
                       style);
    return hipGetLastError();
}
hipError_t launch_store_kv_half(const float *src, __half *dst, int count, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    hipLaunchKernelGGL(store_kv_half_kernel, dim3(cdiv(count, 256)), dim3(256), 0, s, src, dst, count);
    return hipGetLastError();
}
static bool spans_ok(const ZeroSpans &z) {
    for (int j = 0; j < 4; j++)
        if (z.n[j] && !z.p[j]) return false;
    return true;
}

hipError_t launch_silu_mul_rows(float *gate, const float *up, int rows, int n, RowScale rs, const ZeroSpans &z,
                                hipStream_t s) {
    if (!gate || !up || rows < 1 || n < 1 || !spans_ok(z) || (rs.ss && rs.n < 1)) return hipErrorInvalidValue;
    const size_t total = (size_t)rows * n, want = (total + 255) / 256;
    const int blocks = (int)(want < 2048 ? want : 2048);
    hipLaunchKernelGGL(silu_mul_rows_kernel, dim3(blocks), dim3(256), 0, s, gate, up, rows, n, rs, z);
    return hipGetLastError();
}

hipError_t launch_zero_spans(const ZeroSpans &z, hipStream_t s) {
    if (!spans_ok(z)) return hipErrorInvalidValue;
    size_t most = 0;
    for (int j = 0; j < 4; j++) most = z.n[j] > most ? z.n[j] : most;
    if (!most) return hipSuccess;
    const size_t want = (most + 255) / 256;
    const int blocks = (int)(want < 1024 ? want : 1024);
    hipLaunchKernelGGL(zero_spans_kernel, dim3(blocks), dim3(256), 0, s, z);
    return hipGetLastError();
}

hipError_t launch_silu_mul(float *gate, const float *up, int n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, gate, up, n);
    return hipGetLastError();
}
static bool split_args_ok(int ldx, int rows, int n, const XPlanes &xp) {
    return rows > 0 && n > 0 && n % 32 == 0 && ldx % 4 == 0 && ldx >= n && xp.hi && xp.lo && xp.sum &&
           xp.ld % 32 == 0 && xp.ld >= n;
}
hipError_t launch_split_rows(const float *x, int ldx, int rows, int n, const XPlanes &xp, hipStream_t s) {
    if (!split_args_ok(ldx, rows, n, xp)) return hipErrorInvalidValue;
    const long long runs = (long long)rows * (n / 16);
    hipLaunchKernelGGL(split_rows_kernel<false>, dim3((unsigned)((runs + 255) / 256)), dim3(256), 0, s,
                       const_cast<float *>(x), nullptr, ldx, rows, n, xp);
    return hipGetLastError();
}
hipError_t launch_silu_mul_split(float *gate, const float *up, int rows, int n, const XPlanes &xp, hipStream_t s) {
    if (!split_args_ok(n, rows, n, xp) || !up) return hipErrorInvalidValue;
    const long long runs = (long long)rows * (n / 16);
    hipLaunchKernelGGL(split_rows_kernel<true>, dim3((unsigned)((runs + 255) / 256)), dim3(256), 0, s, gate, up, n,
                       rows, n, xp);
    return hipGetLastError();
}
hipError_t launch_add(float *dst, const float *src, int n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(add_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, dst, src, n);
    return hipGetLastError();
}
hipError_t launch_iota_u32(uint32_t *p, int n, hipStream_t s) {
    hipLaunchKernelGGL(iota_u32_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, p, n);
    return hipGetLastError();
}
hipError_t launch_fill_u64(unsigned long long *p, unsigned long long v, int n, hipStream_t s) {
    hipLaunchKernelGGL(fill_u64_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, p, v, n);
    return hipGetLastError();
}
hipError_t launch_argmax(const float *x, int n, uint32_t *out_token, unsigned long long *tmp, hipStream_t s) {
    hipError_t e = launch_fill_u64(tmp, 0ull, 1, s);
    if (e != hipSuccess) return e;
    int grid = cdiv(n, 256 * 16);
    if (grid > 1024) grid = 1024;
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL(argmax_kernel, dim3(grid), dim3(256), 0, s, x, n, tmp);
    hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(1), 0, s, tmp, out_token, 0);
    return hipGetLastError();
}
hipError_t launch_argmax_rows(const float *x, int rows, int n, int ld, unsigned long long *slots, hipStream_t s) {
    if (rows < 1 || n < 1 || ld < n) return hipErrorInvalidValue;
    int grid = cdiv(n, 256 * 16);
    if (grid > 1024) grid = 1024;
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(grid, rows), dim3(256), 0, s, x, n, ld, slots);
    return hipGetLastError();
}
hipError_t launch_argmax_finalize(const unsigned long long *slot, uint32_t *state, hipStream_t s) {
    hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(1), 0, s, slot, state, 1);
    return hipGetLastError();
}
hipError_t launch_topk(const float *x, int n, int k, void *entries, hipStream_t s) {
    // the "taken" flags live right after the k entries (callers size the buffer)
    unsigned char *taken = reinterpret_cast<unsigned char *>(reinterpret_cast<Entry *>(entries) + 64);
    hipLaunchKernelGGL(topk_kernel, dim3(1), dim3(256), 0, s, x, n, k, reinterpret_cast<Entry *>(entries), taken);
    return hipGetLastError();
}
hipError_t launch_normalize_topk(void *entries, int k, int softmax, int normalize, float scale, hipStream_t s) {
    hipLaunchKernelGGL(normalize_topk_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<Entry *>(entries), k, softmax,
                       normalize, scale);
    return hipGetLastError();
}
hipError_t launch_weighted_sum_topk(float *dst, const float *src, const void *entries, int n, int slot,
                                    hipStream_t s) {
    hipLaunchKernelGGL(weighted_sum_topk_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, dst, src,
                       reinterpret_cast<const Entry *>(entries), n, slot);
    return hipGetLastError();
}
hipError_t launch_sigmoid_scale_add(float *dst, const float *src, const float *scalar, int n, hipStream_t s) {
    hipLaunchKernelGGL(sigmoid_scale_add_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, dst, src, scalar, n);
    return hipGetLastError();
}

}  // namespace zh
