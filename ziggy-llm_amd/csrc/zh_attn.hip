// zh_attn.hip -- GQA split-K flash-decoding over the binary16 KV cache.
//
// Reference semantics: computeAttention (model/loader.zig:1397-1438) for one
// query position: per query head h, kv head = h / (heads / kv_heads); scores
// s_t = dot(q_h, k_t) * scale for t in [window_start, pos]; softmax; out_h =
// sum_t p_t v_t.  The Metal kernel it replaces (attention_fused_f32,
// matvec.metal:1274-1389) runs one threadgroup per query head; here the
// context is split into 64-position chunks so the grid grows with context:
//   pass 1: one workgroup per (chunk, kv head) computes the scores of all
//           query heads of the group, the chunk max m, the sum l of
//           exp(s - m) and the unnormalised sum of exp(s - m) v;
//   pass 2: one workgroup per query head merges the chunks (log-sum-exp).
// The position may be read from device memory so a captured graph can be
// replayed at successive positions; chunks past the position exit at once.
#include "zh_internal.h"
#include "zh_quant.h"

namespace zh {

constexpr int kChunk = 64;
constexpr int kMaxGroup = 8;

__device__ __forceinline__ float wmax(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wsum(float v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int HD>
__global__ void __launch_bounds__(256) attn_partial_kernel(AttnParams p) {
    const int split = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int pos = p.position_dev ? *p.position_dev : p.position;
    const int t0 = p.window_start + split * kChunk;
    if (t0 > pos) return;
    const int n = min(kChunk, pos + 1 - t0);
    const int G = p.head_count / p.head_count_kv;

    __shared__ float q_s[kMaxGroup][HD];
    __shared__ float s_s[kMaxGroup][kChunk];
    __shared__ float red[256 / (HD / 2)][kMaxGroup][HD];

    // Every K and V load of this workgroup is issued first; the q staging,
    // the score math and the softmax statistics run while they are in flight.
    constexpr int DPT = HD / 4;                 // K dims per lane (4 lanes per position)
    constexpr int NP = HD / 2, NS = 256 / NP;   // V: lanes own a dim pair, NS position subsets
    constexpr int PPT = kChunk / NS;            // V positions per lane
    const int pi = tid >> 2, part = tid & 3;
    const int dp = tid % NP, ps = tid / NP;
    uint4 kraw[DPT / 8];
    uint32_t vraw[PPT];
    {
        const __half *krow = p.k_cache + (size_t)(t0 + pi) * p.kv_dim + (size_t)kvh * HD + part * DPT;
#pragma unroll
        for (int c = 0; c < DPT / 8; c++)
            kraw[c] = pi < n ? *reinterpret_cast<const uint4 *>(krow + 8 * c) : make_uint4(0, 0, 0, 0);
        const __half *vcol = p.v_cache + (size_t)t0 * p.kv_dim + (size_t)kvh * HD + 2 * dp;
#pragma unroll
        for (int j = 0; j < PPT; j++) {
            const int pv = ps + NS * j;
            vraw[j] = pv < n ? *reinterpret_cast<const uint32_t *>(vcol + (size_t)pv * p.kv_dim) : 0u;
        }
    }

    for (int i = tid; i < G * HD; i += 256) q_s[i / HD][i % HD] = p.q[(size_t)(kvh * G) * HD + i];
    __syncthreads();

    // scores: 4 lanes per position, each covering HD/4 dimensions
    {
        float acc[kMaxGroup];
#pragma unroll
        for (int g = 0; g < kMaxGroup; g++) acc[g] = 0.f;
#pragma unroll
        for (int c = 0; c < DPT / 8; c++) {
            const uint32_t w[4] = {kraw[c].x, kraw[c].y, kraw[c].z, kraw[c].w};
            float k[8];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                k[2 * j] = h2f(w[j]);
                k[2 * j + 1] = h2f(w[j] >> 16);
            }
#pragma unroll
            for (int g = 0; g < kMaxGroup; g++) {
                if (g < G) {
#pragma unroll
                    for (int j = 0; j < 8; j++) acc[g] = fmaf(q_s[g][part * DPT + 8 * c + j], k[j], acc[g]);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; g++) {
            acc[g] += __shfl_xor(acc[g], 1, 64);
            acc[g] += __shfl_xor(acc[g], 2, 64);
        }
        if (part == 0) {
#pragma unroll
            for (int g = 0; g < kMaxGroup; g++)
                if (g < G) s_s[g][pi] = pi < n ? acc[g] * p.scale : -INFINITY;
        }
    }
    __syncthreads();

    // chunk softmax statistics: wave w handles heads w, w+4
    const int wave = tid >> 6, lane = tid & 63;
    float *ml = p.part_ml + ((size_t)kvh * p.max_splits + split) * kMaxGroup * 2;
    for (int g = wave; g < G; g += 4) {
        const float v = s_s[g][lane];
        const float m = wmax(v);
        const float e = lane < n ? expf(v - m) : 0.f;
        const float l = wsum(e);
        s_s[g][lane] = e;
        if (lane == 0) {
            ml[2 * g] = m;
            ml[2 * g + 1] = l;
        }
    }
    __syncthreads();

    // values: unnormalised sum of exp(s - m) v over this lane's positions
    {
        float o0[kMaxGroup], o1[kMaxGroup];
#pragma unroll
        for (int g = 0; g < kMaxGroup; g++) o0[g] = o1[g] = 0.f;
#pragma unroll
        for (int j = 0; j < PPT; j++) {
            const int pv = ps + NS * j;
            const float v0 = h2f(vraw[j]), v1 = h2f(vraw[j] >> 16);
#pragma unroll
            for (int g = 0; g < kMaxGroup; g++) {
                if (g < G) {
                    const float w = pv < n ? s_s[g][pv] : 0.f;
                    o0[g] = fmaf(w, v0, o0[g]);
                    o1[g] = fmaf(w, v1, o1[g]);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; g++) {
            if (g < G) {
                red[ps][g][2 * dp] = o0[g];
                red[ps][g][2 * dp + 1] = o1[g];
            }
        }
        __syncthreads();
        float *po = p.part_o + ((size_t)kvh * p.max_splits + split) * kMaxGroup * HD;
        for (int i = tid; i < G * HD; i += 256) {
            const int g = i / HD, d = i % HD;
            float sacc = 0.f;
#pragma unroll
            for (int k = 0; k < NS; k++) sacc += red[k][g][d];
            po[(size_t)g * HD + d] = sacc;
        }
    }
}

// One workgroup per query head.  Thread (d, sg) folds splits sg, sg + S, ...
// (S = 256 / HD split groups) for dimension d; the split statistics are
// staged in LDS once, and the S partial sums are combined in LDS.
template <int HD>
__global__ void __launch_bounds__(256) attn_merge_kernel(AttnParams p) {
    constexpr int S = 256 / HD;
    const int h = blockIdx.x, tid = threadIdx.x, d = tid % HD, sg = tid / HD;
    const int pos = p.position_dev ? *p.position_dev : p.position;
    const int G = p.head_count / p.head_count_kv, kvh = h / G, g = h % G;
    const int nsplit = (pos - p.window_start) / kChunk + 1;
    const float *ml = p.part_ml + (size_t)kvh * p.max_splits * kMaxGroup * 2 + 2 * g;
    const float *po = p.part_o + (size_t)kvh * p.max_splits * kMaxGroup * HD + (size_t)g * HD + d;
    constexpr int kStage = 1024;  // splits whose statistics fit the LDS stage
    __shared__ float m_s[kStage], l_s[kStage], red[256];
    __shared__ float wmax_s[4];

    float M = -INFINITY;
    for (int s = tid; s < nsplit; s += 256) {
        const float m = ml[(size_t)s * kMaxGroup * 2], l = ml[(size_t)s * kMaxGroup * 2 + 1];
        if (s < kStage) m_s[s] = m, l_s[s] = l;
        M = fmaxf(M, m);
    }
    M = wmax(M);
    if ((tid & 63) == 0) wmax_s[tid >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(wmax_s[0], wmax_s[1]), fmaxf(wmax_s[2], wmax_s[3]));

    float num = 0.f, den = 0.f;
    int s = sg;
    // 4 splits per step: their loads are independent of each other
    for (; s + 3 * S < nsplit; s += 4 * S) {
        float o[4], m[4], l[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int su = s + u * S;
            o[u] = po[(size_t)su * kMaxGroup * HD];
            if (su < kStage) {
                m[u] = m_s[su], l[u] = l_s[su];
            } else {
                m[u] = ml[(size_t)su * kMaxGroup * 2], l[u] = ml[(size_t)su * kMaxGroup * 2 + 1];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float w = expf(m[u] - M);
            den = fmaf(w, l[u], den);
            num = fmaf(w, o[u], num);
        }
    }
    for (; s < nsplit; s += S) {
        const float m = s < kStage ? m_s[s] : ml[(size_t)s * kMaxGroup * 2];
        const float l = s < kStage ? l_s[s] : ml[(size_t)s * kMaxGroup * 2 + 1];
        const float w = expf(m - M);
        den = fmaf(w, l, den);
        num = fmaf(w, po[(size_t)s * kMaxGroup * HD], num);
    }
    if (S > 1) {
        red[tid] = num;
        __syncthreads();
        if (sg == 0)
            for (int k = 1; k < S; k++) num += red[k * HD + d];
        __syncthreads();
        red[tid] = den;
        __syncthreads();
        if (sg == 0)
            for (int k = 1; k < S; k++) den += red[k * HD + d];
    }
    if (sg == 0) p.out[(size_t)h * HD + d] = num / den;
}

size_t attention_scratch_floats(int head_count, int head_dim, int max_splits) {
    (void)head_count;
    // part_o + part_ml for up to `head_count` kv heads
    return (size_t)head_count * max_splits * kMaxGroup * (head_dim + 2);
}

hipError_t launch_attention(const AttnParams &p, hipStream_t s) {
    if (p.head_count % p.head_count_kv || p.head_count / p.head_count_kv > kMaxGroup) return hipErrorInvalidValue;
    const dim3 grid(p.max_splits, p.head_count_kv);
    if (p.head_dim == 128) {
        hipLaunchKernelGGL(attn_partial_kernel<128>, grid, dim3(256), 0, s, p);
        hipLaunchKernelGGL(attn_merge_kernel<128>, dim3(p.head_count), dim3(256), 0, s, p);
    } else if (p.head_dim == 64) {
        hipLaunchKernelGGL(attn_partial_kernel<64>, grid, dim3(256), 0, s, p);
        hipLaunchKernelGGL(attn_merge_kernel<64>, dim3(p.head_count), dim3(256), 0, s, p);
    } else if (p.head_dim == 256) {
        hipLaunchKernelGGL(attn_partial_kernel<256>, grid, dim3(256), 0, s, p);
        hipLaunchKernelGGL(attn_merge_kernel<256>, dim3(p.head_count), dim3(256), 0, s, p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace zh
