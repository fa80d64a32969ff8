// zh_attn.hip -- GQA split-K flash-decoding over the binary16 KV cache.
//
// Reference semantics: computeAttention (model/loader.zig:1397-1438) for one
// query position: per query head h, kv head = h / (heads / kv_heads); scores
// s_t = dot(q_h, k_t) * scale for t in [window_start, pos]; softmax; out_h =
// sum_t p_t v_t.  The Metal kernel it replaces (attention_fused_f32,
// matvec.metal:1274-1389) runs one threadgroup per query head.
//
// Here one workgroup handles one kv head (all G query heads of its group)
// over a contiguous range of 64-position chunks, with an online softmax
// across its chunks; the number of splits grows with the position up to
// max_splits, so long contexts keep about one workgroup per CU busy.  Each
// split writes (m, l, unnormalised o) per query head; the last workgroup of
// a kv head to finish (arrival counter) merges the splits with log-sum-exp
// and resets the counter, so replays of a captured graph need no memset.
//
// In the session ("fused") mode the kernel also runs the q/k/v epilogue of
// the projection: + bias, per-head RMSNorm of q and k
// (rmsNormPerHeadWithOffset, model/loader.zig:1777-1812), RoPE (applyRoPE,
// :3827-3866) of q in every workgroup, and of k in the workgroup whose range
// holds the current position, which stores k and v to the cache as binary16
// (store_kv_half, matvec.metal:246-255) and uses the stored values for that
// position.  The position may be read from device memory (graph replay).
#include <cstdlib>
#include <type_traits>

#include "zh_internal.h"
#include "zh_quant.h"

namespace zh {

constexpr int kChunk = 64;
constexpr int kMaxGroup = 8;
constexpr int QV_MAX = 8;  // q values per thread at most (8 heads of 256)

__device__ __forceinline__ float wmax(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wsum(float v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// RoPE angles of one position, once per workgroup: cs[i], sn[i] for pair i
// of the n_rot rotated dims, theta = pos / base^(2i / n_rot) (applyRoPE,
// model/loader.zig:3827-3866).
__device__ __forceinline__ void rope_table(int n_rot, float base, int pos, float *cs, float *sn) {
    const int t = threadIdx.x;
    if (t < n_rot / 2) {
        const float e = (float)(2 * t) / (float)n_rot;
        const float theta = (float)pos / powf(base, e);
        float sv, cv;
        sincosf(theta, &sv, &cv);
        cs[t] = cv;
        sn[t] = sv;
    }
}

// Per-head RMSNorm (rmsNormPerHeadWithOffset, model/loader.zig:1777-1812) of
// the V values this thread holds (element tid + 256 i, heads of HD values;
// a wavefront never spans two heads since HD >= 64), then the values go to
// dst (LDS) and are rotated pairwise with the RoPE table.  `n` elements in all.
template <int HD, int V>
__device__ __forceinline__ void norm_rope(float (&x)[V], int n, const float *norm_w, float eps, int n_rot, int style,
                                          const float *cs, const float *sn, float *dst, float *red) {
    const int tid = threadIdx.x, wave = tid >> 6;
    constexpr int WPH = HD / 64;  // wavefronts per head
    if (norm_w) {
#pragma unroll
        for (int i = 0; i < V; i++) {
            const int idx = tid + 256 * i;
            const float ss = wsum(idx < n ? x[i] * x[i] : 0.f);
            if ((tid & 63) == 0) red[4 * i + wave] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < V; i++) {
            const int idx = tid + 256 * i;
            float tot = 0.f;
            const int w0 = wave / WPH * WPH;
            for (int w = 0; w < WPH; w++) tot += red[4 * i + w0 + w];
            const float scale = 1.0f / sqrtf(tot / (float)HD + eps);
            if (idx < n) x[i] = (scale * x[i]) * norm_w[idx % HD];
        }
    }
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int idx = tid + 256 * i;
        if (idx < n) dst[idx] = x[i];
    }
    __syncthreads();
    const int half = n_rot / 2;
    for (int q = tid; q < (n / HD) * half; q += 256) {
        const int h = q / half, t = q % half;
        const int a = h * HD + (style == 0 ? 2 * t : t), c = h * HD + (style == 0 ? 2 * t + 1 : t + half);
        const float x0 = dst[a], x1 = dst[c];
        dst[a] = fmaf(x0, cs[t], -x1 * sn[t]);
        dst[c] = fmaf(x0, sn[t], x1 * cs[t]);
    }
    __syncthreads();
}

// Sum / max over the 16 position quads of a wavefront (lane bits 2..5).
__device__ __forceinline__ float quads_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}
__device__ __forceinline__ float quads_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false)));
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// Workgroup (split, kv head).  Wavefront w takes positions 16w..16w+15 of
// every 64-position chunk of the split and keeps its own online softmax
// (running max m, sum l, unnormalised o per query head): no workgroup
// barrier inside the chunk loop.  Scores: lane = (position, quarter of the
// head dims), a quad reduction finishes each dot.  Values: lane owns HD/64
// dims and takes the probabilities of the 16 positions by readlane.
// GG: query heads per kv head when it is 1, 2, 4 or 8 (compile-time loops),
// 0 for any group size up to 8.
template <int HD, int GG>
__global__ void __launch_bounds__(256) attn_kernel(AttnParams p) {
    const int split = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int pos = p.position_dev ? *p.position_dev : p.position;
    const int n_total = pos + 1 - p.window_start;
    const int nch = (n_total + kChunk - 1) / kChunk;
    const int per = (nch + p.max_splits - 1) / p.max_splits;  // chunks per split
    const int nsplit = (nch + per - 1) / per;
    if (split >= nsplit) return;
    const int c_begin = split * per, c_end = min(c_begin + per, nch);
    constexpr int KG = GG ? GG : kMaxGroup;  // head loop bound
    const int G = GG ? GG : p.head_count / p.head_count_kv;
    const bool fused = p.k_new != nullptr;
    const int wave = tid >> 6, lane = tid & 63;

    constexpr int DQ = HD / 4;    // K dims per lane
    constexpr int DPL = HD / 64;  // V dims per lane
    __shared__ float q_s[kMaxGroup][HD];
    __shared__ float wo[4][kMaxGroup][HD];
    __shared__ float wm[4][kMaxGroup], wl[4][kMaxGroup];
    __shared__ float kn_s[HD], vn_s[HD];  // this step's k and v (binary16-rounded)
    __shared__ float red16[4 * QV_MAX];
    __shared__ float cs_s[HD / 2], sn_s[HD / 2];
    __shared__ float fm_s[kMaxGroup], fl_s[kMaxGroup];
    __shared__ int last_s;

    const int pk = lane >> 2, quarter = lane & 3;
    const size_t kv_off = (size_t)kvh * HD;

    // Loads of one chunk for this wavefront.  Positions past the end re-read
    // position `pos` (valid memory; masked below), so the loads are unconditional.
    using VW = typename std::conditional<DPL == 1, uint16_t, typename std::conditional<DPL == 2, uint32_t, uint2>::type>::type;
    auto load_chunk = [&](int c, uint4 (&kr)[DQ / 8], VW (&vr)[16]) {
        const int tw = p.window_start + c * kChunk + 16 * wave;
        const __half *krow = p.k_cache + (size_t)min(tw + pk, pos) * p.kv_dim + kv_off + quarter * DQ;
#pragma unroll
        for (int j = 0; j < DQ / 8; j++) kr[j] = *reinterpret_cast<const uint4 *>(krow + 8 * j);
#pragma unroll
        for (int j = 0; j < 16; j++)
            vr[j] = *reinterpret_cast<const VW *>(p.v_cache + (size_t)min(tw + j, pos) * p.kv_dim + kv_off + lane * DPL);
    };

    // q (and this step's k / v) first, so waiting for them does not wait
    // for the K/V chunk loads issued next.
    constexpr int QV = kMaxGroup * HD / 256;  // q values per thread at most
    const int nq = G * HD;
    const bool own_pos = fused && c_end == nch;  // this split holds the current position
    float qv[QV], kx[1] = {0.f}, vx = 0.f;
#pragma unroll
    for (int i = 0; i < QV; i++) {
        const int idx = tid + 256 * i;
        qv[i] = 0.f;
        if (idx < nq) {
            qv[i] = p.q[(size_t)kvh * nq + idx];
            if (fused && p.q_bias) qv[i] += p.q_bias[(size_t)kvh * nq + idx];
        }
    }
    if (own_pos && tid < HD) {
        kx[0] = p.k_new[kv_off + tid];
        vx = p.v_new[kv_off + tid];
        if (p.k_bias) kx[0] += p.k_bias[kv_off + tid];
        if (p.v_bias) vx += p.v_bias[kv_off + tid];
    }
    uint4 kraw[DQ / 8];
    VW vraw[16];
    load_chunk(c_begin, kraw, vraw);

    if (fused) {
        const int n_rot = p.rope_dim < HD ? p.rope_dim : HD;
        rope_table(n_rot, p.rope_base, pos, cs_s, sn_s);
        norm_rope<HD, QV>(qv, nq, p.q_norm, p.eps, n_rot, p.rope_style, cs_s, sn_s, &q_s[0][0], red16);
        if (own_pos) {
            norm_rope<HD, 1>(kx, HD, p.k_norm, p.eps, n_rot, p.rope_style, cs_s, sn_s, kn_s, red16);
            if (tid < HD) {
                const __half kh = __float2half_rn(kn_s[tid]), vh = __float2half_rn(vx);
                if (pos < p.ctx) {
                    const size_t idx = (size_t)pos * p.kv_dim + kv_off + tid;
                    p.k_cache[idx] = kh;
                    p.v_cache[idx] = vh;
                }
                kn_s[tid] = __half2float(kh);
                vn_s[tid] = __half2float(vh);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < QV; i++) {
            const int idx = tid + 256 * i;
            if (idx < nq) q_s[idx / HD][idx % HD] = qv[i];
        }
    }
    __syncthreads();

    float m[KG], l[KG], o[KG][DPL];
#pragma unroll
    for (int g = 0; g < KG; g++) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int d = 0; d < DPL; d++) o[g][d] = 0.f;
    }

    auto process = [&](int c, const uint4 (&kr)[DQ / 8], const VW (&vr)[16]) {
        const int tw = p.window_start + c * kChunk + 16 * wave;
        const int nw = min(16, pos + 1 - tw);  // valid positions of this wavefront (uniform)
        if (nw <= 0) return;
        // scores
        const bool kcur = fused && tw + pk == pos;  // this step's k, from LDS
        float acc[KG];
#pragma unroll
        for (int g = 0; g < KG; g++) acc[g] = 0.f;
#pragma unroll
        for (int j = 0; j < DQ / 8; j++) {
            const uint32_t w[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
            float k[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                k[2 * i] = h2f(w[i]);
                k[2 * i + 1] = h2f(w[i] >> 16);
            }
            if (kcur) {
#pragma unroll
                for (int i = 0; i < 8; i++) k[i] = kn_s[quarter * DQ + 8 * j + i];
            }
#pragma unroll
            for (int g = 0; g < KG; g++) {
                if (g < G) {
                    const float4 qa = *reinterpret_cast<const float4 *>(&q_s[g][quarter * DQ + 8 * j]);
                    const float4 qb = *reinterpret_cast<const float4 *>(&q_s[g][quarter * DQ + 8 * j + 4]);
                    acc[g] = fmaf(qa.x, k[0], acc[g]);
                    acc[g] = fmaf(qa.y, k[1], acc[g]);
                    acc[g] = fmaf(qa.z, k[2], acc[g]);
                    acc[g] = fmaf(qa.w, k[3], acc[g]);
                    acc[g] = fmaf(qb.x, k[4], acc[g]);
                    acc[g] = fmaf(qb.y, k[5], acc[g]);
                    acc[g] = fmaf(qb.z, k[6], acc[g]);
                    acc[g] = fmaf(qb.w, k[7], acc[g]);
                }
            }
        }
        float e[KG];
#pragma unroll
        for (int g = 0; g < KG; g++) {
            if (g < G) {
                float sc = acc[g];
                sc += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sc), 0xB1, 0xF, 0xF, false));
                sc += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sc), 0x4E, 0xF, 0xF, false));
                sc = pk < nw ? sc * p.scale : -INFINITY;
                const float m_new = fmaxf(m[g], quads_max(sc));
                const float alpha = expf(m[g] - m_new);  // 0 on the first chunk
                e[g] = pk < nw ? expf(sc - m_new) : 0.f;
                l[g] = fmaf(l[g], alpha, quads_sum(quarter == 0 ? e[g] : 0.f));
                m[g] = m_new;
#pragma unroll
                for (int d = 0; d < DPL; d++) o[g][d] *= alpha;
            }
        }
        // values
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (j < nw) {
                float v[DPL];
                const VW raw = vr[j];
                if constexpr (DPL == 1) {
                    v[0] = h2f((uint32_t)raw);
                } else if constexpr (DPL == 2) {
                    v[0] = h2f((uint32_t)raw);
                    v[1] = h2f((uint32_t)raw >> 16);
                } else {
                    v[0] = h2f(raw.x);
                    v[1] = h2f(raw.x >> 16);
                    v[2] = h2f(raw.y);
                    v[3] = h2f(raw.y >> 16);
                }
                if (fused && tw + j == pos) {
#pragma unroll
                    for (int d = 0; d < DPL; d++) v[d] = vn_s[lane * DPL + d];
                }
#pragma unroll
                for (int g = 0; g < KG; g++) {
                    if (g < G) {
                        const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[g]), 4 * j));
#pragma unroll
                        for (int d = 0; d < DPL; d++) o[g][d] = fmaf(pj, v[d], o[g][d]);
                    }
                }
            }
        }
    };

    // Two chunk buffers alternate, so a buffer is never copied (a copy would
    // wait for the loads in flight into its source).
    uint4 kb[DQ / 8];
    VW vb[16];
    for (int c = c_begin; c < c_end; c += 2) {
        load_chunk(min(c + 1, c_end - 1), kb, vb);
        process(c, kraw, vraw);
        if (c + 1 < c_end) {
            load_chunk(min(c + 2, c_end - 1), kraw, vraw);
            process(c + 1, kb, vb);
        }
    }

    // combine the four wavefronts' softmax states
#pragma unroll
    for (int g = 0; g < KG; g++) {
        if (g < G) {
#pragma unroll
            for (int d = 0; d < DPL; d++) wo[wave][g][lane * DPL + d] = o[g][d];
            if (lane == 0) {
                wm[wave][g] = m[g];
                wl[wave][g] = l[g];
            }
        }
    }
    __syncthreads();
    if (tid < G) {
        const int g = tid;
        const float M = fmaxf(fmaxf(wm[0][g], wm[1][g]), fmaxf(wm[2][g], wm[3][g]));
        float L = 0.f;
        for (int w = 0; w < 4; w++) L = fmaf(wl[w][g], expf(wm[w][g] - M), L);  // empty wavefronts: exp(-inf) = 0
        fm_s[g] = M;
        fl_s[g] = L;
    }
    __syncthreads();
    const size_t pbase = ((size_t)kvh * p.max_splits + split) * kMaxGroup;
    for (int i = tid; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        const float M = fm_s[g];
        float sacc = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) sacc = fmaf(wo[w][g][d], expf(wm[w][g] - M), sacc);
        if (nsplit == 1) {
            p.out[(size_t)(kvh * G + g) * HD + d] = sacc / fl_s[g];
        } else {
            p.part_o[(pbase + g) * HD + d] = sacc;
        }
    }
    if (nsplit == 1) return;
    if (tid < G) {
        p.part_ml[(pbase + tid) * 2] = fm_s[tid];
        p.part_ml[(pbase + tid) * 2 + 1] = fl_s[tid];
    }

    // Arrival: the workgroup barrier orders every thread's partial stores
    // before thread 0's agent-scope release (one L2 write-back per workgroup);
    // the counter tells the last arrival of this kv head, which acquires
    // (invalidates its stale cache lines) and merges.
    __syncthreads();
    if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const unsigned old = __hip_atomic_fetch_add(&p.counters[kvh], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_s = old == (unsigned)(nsplit - 1);
        if (last_s) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (!last_s) return;

    // Merge: item (quad of 4 dims of one head, split group sg) folds splits
    // sg, sg + SG, ... with an online log-sum-exp, four splits' loads at a
    // time; the SG groups then combine through LDS (the wo buffer is free).
    const float *ml = p.part_ml + (size_t)kvh * p.max_splits * kMaxGroup * 2;
    const float *po = p.part_o + (size_t)kvh * p.max_splits * kMaxGroup * HD;
    constexpr int Q4 = HD / 4;
    const int nquads = G * Q4;
    const int SG = nquads >= 256 ? 1 : 256 / nquads;
    float *mg = &wo[0][0][0];  // [SG][nquads][6]: M, L, O[4]
    for (int it = tid; it < nquads * SG; it += 256) {
        const int quad = it % nquads, sg = it / nquads, g = quad / Q4, d4 = (quad % Q4) * 4;
        float M = -INFINITY, L = 0.f, O[4] = {0.f, 0.f, 0.f, 0.f};
        auto fold = [&](float m, float l, const float4 o) {
            const float Mn = fmaxf(M, m);
            const float a = expf(M - Mn), b = expf(m - Mn);
            L = fmaf(L, a, l * b);
            O[0] = fmaf(O[0], a, o.x * b);
            O[1] = fmaf(O[1], a, o.y * b);
            O[2] = fmaf(O[2], a, o.z * b);
            O[3] = fmaf(O[3], a, o.w * b);
            M = Mn;
        };
        int sp = sg;
        for (; sp + 3 * SG < nsplit; sp += 4 * SG) {
            float m4[4], l4[4];
            float4 o4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const size_t e = (size_t)(sp + u * SG) * kMaxGroup + g;
                m4[u] = ml[e * 2];
                l4[u] = ml[e * 2 + 1];
                o4[u] = *reinterpret_cast<const float4 *>(po + e * HD + d4);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) fold(m4[u], l4[u], o4[u]);
        }
        for (; sp < nsplit; sp += SG) {
            const size_t e = (size_t)sp * kMaxGroup + g;
            fold(ml[e * 2], ml[e * 2 + 1], *reinterpret_cast<const float4 *>(po + e * HD + d4));
        }
        float *dst = mg + ((size_t)sg * nquads + quad) * 6;
        dst[0] = M;
        dst[1] = L;
        dst[2] = O[0], dst[3] = O[1], dst[4] = O[2], dst[5] = O[3];
    }
    __syncthreads();
    for (int quad = tid; quad < nquads; quad += 256) {
        float M = -INFINITY;
        for (int sg = 0; sg < SG; sg++) M = fmaxf(M, mg[((size_t)sg * nquads + quad) * 6]);
        float L = 0.f, O[4] = {0.f, 0.f, 0.f, 0.f};
        for (int sg = 0; sg < SG; sg++) {
            const float *src = mg + ((size_t)sg * nquads + quad) * 6;
            const float w = expf(src[0] - M);  // split groups without splits: exp(-inf) = 0
            L = fmaf(src[1], w, L);
#pragma unroll
            for (int k = 0; k < 4; k++) O[k] = fmaf(src[2 + k], w, O[k]);
        }
        const int g = quad / Q4, d4 = (quad % Q4) * 4;
        float *dst = p.out + (size_t)(kvh * G + g) * HD + d4;
#pragma unroll
        for (int k = 0; k < 4; k++) dst[k] = O[k] / L;
    }
    if (tid == 0) __hip_atomic_store(&p.counters[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

size_t attention_scratch_floats(int head_count, int head_dim, int max_splits) {
    // part_o + part_ml for up to `head_count` kv heads
    return (size_t)head_count * max_splits * kMaxGroup * (head_dim + 2);
}

// Target workgroups of the attention grid at the longest context;
// ZIGGY_HIP_ATTN_WGS overrides it (a tuning knob).
static int attention_target_wgs() {
    static int t = [] {
        const char *e = getenv("ZIGGY_HIP_ATTN_WGS");
        const int v = e ? atoi(e) : 256;
        return v > 0 ? v : 256;
    }();
    return t;
}

int attention_splits(int kv_heads, int max_positions) {
    // a bounded number of splits (the merge reads them all); never more
    // splits than 64-position chunks
    const int chunks = (max_positions + kChunk - 1) / kChunk;
    int s = attention_target_wgs() / (kv_heads > 0 ? kv_heads : 1);
    if (s < 1) s = 1;
    return s < chunks ? s : chunks;
}

hipError_t launch_attention(const AttnParams &p, hipStream_t s) {
    if (p.head_count_kv <= 0 || p.head_count % p.head_count_kv || p.head_count / p.head_count_kv > kMaxGroup ||
        p.max_splits < 1 || !p.counters)
        return hipErrorInvalidValue;
    const dim3 grid(p.max_splits, p.head_count_kv);
    const int G = p.head_count / p.head_count_kv;
    auto go = [&](auto hd_tag) {
        constexpr int HD = decltype(hd_tag)::value;
        switch (G) {
        case 1: hipLaunchKernelGGL((attn_kernel<HD, 1>), grid, dim3(256), 0, s, p); break;
        case 2: hipLaunchKernelGGL((attn_kernel<HD, 2>), grid, dim3(256), 0, s, p); break;
        case 4: hipLaunchKernelGGL((attn_kernel<HD, 4>), grid, dim3(256), 0, s, p); break;
        case 8: hipLaunchKernelGGL((attn_kernel<HD, 8>), grid, dim3(256), 0, s, p); break;
        default: hipLaunchKernelGGL((attn_kernel<HD, 0>), grid, dim3(256), 0, s, p); break;
        }
    };
    switch (p.head_dim) {
    case 64: go(std::integral_constant<int, 64>{}); break;
    case 128: go(std::integral_constant<int, 128>{}); break;
    case 256: go(std::integral_constant<int, 256>{}); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace zh
