// zh_attn.hip -- GQA split-K flash-decoding over the binary16 KV cache.
//
// Reference semantics: computeAttention (model/loader.zig:1397-1438) for one
// query position: per query head h, kv head = h / (heads / kv_heads); scores
// s_t = dot(q_h, k_t) * scale for t in [window_start, pos]; softmax; out_h =
// sum_t p_t v_t.  The Metal kernel it replaces (attention_fused_f32,
// matvec.metal:1274-1389) runs one threadgroup per query head.
//
// Here one workgroup handles one kv head (all G query heads of its group)
// over a contiguous range of positions; the number of splits grows with the
// position up to max_splits, so long contexts keep every CU busy.  Each
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

// Sum over aligned groups of n lanes (n = 4, 8 or 16) of a 16-lane row; the
// total is valid in every lane of the group.
__device__ __forceinline__ float group_sum16(float v, int n) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
    if (n >= 8) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
    if (n >= 16) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)); // row_mirror
    return v;
}
// Sum over the lanes of a 16-lane row with the same (lane mod n) (n = 4, 8
// or 16): every such lane holds the total.
__device__ __forceinline__ float rows_sum16(float v, int n) {
    if (n <= 8) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
    if (n <= 4) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
    return v;
}

// Max / sum over aligned groups of 32 lanes (half wavefronts); the total is
// valid in every lane of the group.
__device__ __forceinline__ float half_max32(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    return fmaxf(v, __shfl_xor(v, 16, 64));
}
__device__ __forceinline__ float half_sum32(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    return v + __shfl_xor(v, 16, 64);
}

// Workgroup (split, kv head) attends over a contiguous range of positions,
// in passes of PPP positions: lane (position pw, dims block sub) of wavefront
// w takes position pw + PPW w of each pass and dims 16 sub .. 16 sub + 15
// (LP = HD / 16 lanes per position, PPW = 64 / LP positions per wavefront).
// The K and V loads of NP passes are in flight at once (a ring refilled in
// place; short ranges issue all their loads up front).  Scores finish with
// an LP-lane DPP sum; every lane keeps an online softmax (m, l, o) for its
// own position stream, so the pass loop has no cross-lane traffic beyond
// the score sum.  The workgroup then merges its streams (max through LDS,
// row sums by DPP, row partials through LDS).  With several splits, each
// writes (m, l, unnormalised o) per query head with write-through stores;
// the last workgroup of a kv head to arrive (arrival counter) merges the
// splits with log-sum-exp and resets the counter, so replays of a captured
// graph need no memset.
// GG: query heads per kv head when it is 1, 2, 4 or 8 (compile-time loops),
// 0 for any group size up to 8.
template <int HD, int GG>
__global__ void __launch_bounds__(256) attn_kernel(AttnParams p) {
    constexpr int LP = HD / 16;   // lanes per position
    constexpr int PPW = 64 / LP;  // positions per wavefront and pass
    constexpr int PPP = 4 * PPW;  // positions per pass
    constexpr int NP = 4;         // passes in flight
    constexpr int KG = GG ? GG : kMaxGroup;  // head loop bound
    const int split = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, sub = lane % LP, pw = lane / LP;
    const int pos = p.position_dev ? *p.position_dev : p.position;
    const int n_total = pos + 1 - p.window_start;
    const int units = (n_total + PPP - 1) / PPP;
    const int per = (units + p.max_splits - 1) / p.max_splits;  // passes per split
    const int nsplit = (units + per - 1) / per;
    if (split >= nsplit) return;
    const int u_begin = split * per, npass = min(per, units - u_begin);
    const int G = GG ? GG : p.head_count / p.head_count_kv;
    const bool fused = p.k_new != nullptr;
    const bool own_pos = fused && u_begin + npass == units;  // this split holds the current position

    __shared__ float q_s[kMaxGroup][HD];
    __shared__ float kn_s[HD], vn_s[HD];  // this step's k and v (binary16-rounded)
    __shared__ float red16[4 * QV_MAX];
    __shared__ float cs_s[HD / 2], sn_s[HD / 2];
    __shared__ float ml_s[PPP][kMaxGroup][2];
    __shared__ float fm_s[kMaxGroup], fl_s[kMaxGroup];
    constexpr int NR = 16;  // row partials of the stream sums (4 per wavefront)
    __shared__ float rows_s[NR][KG * HD <= 512 ? KG * HD : 512];
    __shared__ int last_s;

    const size_t kv_off = (size_t)kvh * HD;
    // stream position of pass i (may pass the end: loads clamp, scores mask)
    auto pos_of = [&](int i) { return p.window_start + (u_begin + i) * PPP + wave * PPW + pw; };

    // q (and this step's k / v) first: waiting for them must not wait for
    // the K/V loads issued next (vmcnt completes in order)
    constexpr int QV = kMaxGroup * HD / 256;
    const int nq = G * HD;
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
    __builtin_amdgcn_sched_barrier(0);
    uint4 kr[NP][2], vr[NP][2];
    auto row_off = [&](int i) { return (size_t)min(pos_of(min(i, npass - 1)), pos) * p.kv_dim + kv_off + 16 * sub; };
    auto load_k = [&](int i, uint4 (&k)[2]) {
        const uint4 *kp = reinterpret_cast<const uint4 *>(p.k_cache + row_off(i));
        k[0] = kp[0];
        k[1] = kp[1];
    };
    auto load_v = [&](int i, uint4 (&v)[2]) {
        const uint4 *vp = reinterpret_cast<const uint4 *>(p.v_cache + row_off(i));
        v[0] = vp[0];
        v[1] = vp[1];
    };
    // all K slots, then all V slots: the order the group loop consumes them
#pragma unroll
    for (int j = 0; j < NP; j++) {
        load_k(j, kr[j]);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < NP; j++) {
        load_v(j, vr[j]);
        __builtin_amdgcn_sched_barrier(0);
    }

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

    // Softmax in base 2: scores carry scale * log2(e), so exp2 gives the
    // exponentials (the max-subtracted arguments stay in [-126, 0]).
    const float sl2 = p.scale * 1.44269504088896340736f;
    float m[KG], l[KG], o[KG][16];
#pragma unroll
    for (int g = 0; g < KG; g++) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int d = 0; d < 16; d++) o[g][d] = 0.f;
    }
    // Groups of NP passes: the scores of the whole group first (each K slot
    // is refilled as soon as its scores are done), then one rescale of the
    // stream state to the group max, then the values (each V slot refilled
    // after use).
    for (int i0 = 0; i0 < npass; i0 += NP) {
        float sc[NP][KG];
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const int i = i0 + j;
            const int ps = pos_of(i);
            const bool valid = i < npass && ps <= pos;
            float k[16];
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const uint32_t kw[4] = {kr[j][c].x, kr[j][c].y, kr[j][c].z, kr[j][c].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    k[8 * c + 2 * e] = h2f(kw[e]);
                    k[8 * c + 2 * e + 1] = h2f(kw[e] >> 16);
                }
            }
            if (fused && ps == pos) {  // this step's k (the cache row was loaded before the store)
#pragma unroll
                for (int d = 0; d < 16; d++) k[d] = kn_s[16 * sub + d];
            }
            __builtin_amdgcn_sched_barrier(0);
            load_k(i + NP, kr[j]);  // unconditional (clamped): keeps the slot in place
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int g = 0; g < KG; g++) {
                float acc = 0.f;
                if (g < G) {
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const float4 qq = *reinterpret_cast<const float4 *>(&q_s[g][16 * sub + 4 * c]);
                        acc = fmaf(qq.x, k[4 * c], acc);
                        acc = fmaf(qq.y, k[4 * c + 1], acc);
                        acc = fmaf(qq.z, k[4 * c + 2], acc);
                        acc = fmaf(qq.w, k[4 * c + 3], acc);
                    }
                    acc = group_sum16(acc, LP);  // the position's score in every lane of its group
                }
                sc[j][g] = valid ? acc * sl2 : -INFINITY;
            }
        }
        float alpha[KG];
#pragma unroll
        for (int g = 0; g < KG; g++) {
            float gm = m[g];
#pragma unroll
            for (int j = 0; j < NP; j++) gm = fmaxf(gm, sc[j][g]);
            alpha[g] = gm == -INFINITY ? 1.f : exp2f(m[g] - gm);  // 0 on the stream's first scores
            m[g] = gm;
            l[g] *= alpha[g];
        }
#pragma unroll
        for (int g = 0; g < KG; g++)
            if (g < G) {
#pragma unroll
                for (int d = 0; d < 16; d++) o[g][d] *= alpha[g];
            }
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const int i = i0 + j;
            const int ps = pos_of(i);
            float v[16];
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const uint32_t vw[4] = {vr[j][c].x, vr[j][c].y, vr[j][c].z, vr[j][c].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[8 * c + 2 * e] = h2f(vw[e]);
                    v[8 * c + 2 * e + 1] = h2f(vw[e] >> 16);
                }
            }
            if (fused && ps == pos) {
#pragma unroll
                for (int d = 0; d < 16; d++) v[d] = vn_s[16 * sub + d];
            }
            __builtin_amdgcn_sched_barrier(0);
            load_v(i + NP, vr[j]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int g = 0; g < KG; g++) {
                if (g < G) {
                    const float e = sc[j][g] == -INFINITY ? 0.f : exp2f(sc[j][g] - m[g]);
                    l[g] += e;
#pragma unroll
                    for (int d = 0; d < 16; d++) o[g][d] = fmaf(e, v[d], o[g][d]);
                }
            }
        }
    }

    // ---- merge the workgroup's PPP position streams ----
    const int stream = wave * PPW + pw;
    if (sub == 0) {
#pragma unroll
        for (int g = 0; g < KG; g++)
            if (g < G) ml_s[stream][g][0] = m[g], ml_s[stream][g][1] = l[g];
    }
    __syncthreads();
    {
        // 32 lanes per head g: lane (tid & 31) folds streams tid & 31,
        // + 32, ...; then a 32-lane max and sum, and one lane writes the
        // head's (M, L)
        const int g = tid >> 5, r = tid & 31;
        float mm = -INFINITY;
        if (g < G)
            for (int st = r; st < PPP; st += 32) mm = fmaxf(mm, ml_s[st][g][0]);
        mm = half_max32(mm);
        float ll = 0.f;
        if (g < G)
            for (int st = r; st < PPP; st += 32) {
                const float ms = ml_s[st][g][0];
                ll += ms == -INFINITY ? 0.f : ml_s[st][g][1] * exp2f(ms - mm);
            }
        ll = half_sum32(ll);
        if (g < G && r == 31) {
            fm_s[g] = mm;
            fl_s[g] = ll;
        }
    }
    __syncthreads();
    // scale each stream to the workgroup max, sum the streams of a 16-lane
    // row by DPP, then the 16 row partials through LDS (in head blocks of
    // at most 512 values)
    for (int gb = 0; gb < KG; gb += (512 / HD > 0 ? 512 / HD : 1)) {
        const int gn = min(512 / HD > 0 ? 512 / HD : 1, G - gb);  // heads in this block
        if (gn <= 0) break;
#pragma unroll
        for (int g = 0; g < KG; g++) {
            if (g >= gb && g < gb + gn) {
                const float w = m[g] == -INFINITY ? 0.f : exp2f(m[g] - fm_s[g]);
#pragma unroll
                for (int d = 0; d < 16; d++) {
                    float t = o[g][d] * w;
                    t = rows_sum16(t, LP);  // sum over the row's position streams
                    if ((lane & 15) < LP) rows_s[wave * 4 + (lane >> 4)][(g - gb) * HD + 16 * sub + d] = t;
                }
            }
        }
        __syncthreads();
        for (int it = tid; it < gn * HD; it += 256) {
            float acc = 0.f;
#pragma unroll
            for (int r = 0; r < NR; r++) acc += rows_s[r][it];
            const int g = gb + it / HD, d = it % HD;
            if (nsplit == 1) {
                p.out[(size_t)(kvh * G + g) * HD + d] = acc / fl_s[g];
            } else {
                const size_t e = (((size_t)kvh * p.max_splits + split) * kMaxGroup + g) * HD + d;
                __hip_atomic_store(p.part_o + e, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();
    }
    if (nsplit == 1) return;
    if (tid < G) {
        const size_t e = ((size_t)kvh * p.max_splits + split) * kMaxGroup + tid;
        const unsigned long long v = (unsigned long long)__float_as_uint(fm_s[tid]) |
                                     ((unsigned long long)__float_as_uint(fl_s[tid]) << 32);
        __hip_atomic_store(reinterpret_cast<unsigned long long *>(p.part_ml) + e, v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }

    // Arrival: every thread's partial stores (agent scope, write-through)
    // complete before the workgroup barrier; thread 0 then releases and
    // counts.  The last arrival of this kv head acquires and merges.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(&p.counters[kvh], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        last_s = old == (unsigned)(nsplit - 1);
        if (last_s) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (!last_s) return;

    // Merge: item (pair of dims of one head) folds every split with an
    // online log-sum-exp (base 2), sixteen splits' loads in flight.
    const unsigned long long *ml = reinterpret_cast<const unsigned long long *>(p.part_ml) +
                                   (size_t)kvh * p.max_splits * kMaxGroup;
    const unsigned long long *po = reinterpret_cast<const unsigned long long *>(p.part_o) +
                                   (size_t)kvh * p.max_splits * kMaxGroup * (HD / 2);
    for (int it = tid; it < G * HD / 2; it += 256) {
        const int g = it / (HD / 2), d2 = it % (HD / 2);
        float M = -INFINITY, L = 0.f, O0 = 0.f, O1 = 0.f;
        for (int s0 = 0; s0 < nsplit; s0 += 16) {
            unsigned long long mlv[16], ov[16];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const size_t e = (size_t)min(s0 + u, nsplit - 1) * kMaxGroup + g;
                mlv[u] = __hip_atomic_load(ml + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ov[u] = __hip_atomic_load(po + e * (HD / 2) + d2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int u = 0; u < 16; u++) {
                if (s0 + u < nsplit) {
                    const float ms = __uint_as_float((uint32_t)mlv[u]), ls = __uint_as_float((uint32_t)(mlv[u] >> 32));
                    const float o0 = __uint_as_float((uint32_t)ov[u]), o1 = __uint_as_float((uint32_t)(ov[u] >> 32));
                    const float Mn = fmaxf(M, ms);  // every split holds a position: ms is finite
                    const float a = exp2f(M - Mn), b = exp2f(ms - Mn);
                    L = fmaf(L, a, ls * b);
                    O0 = fmaf(O0, a, o0 * b);
                    O1 = fmaf(O1, a, o1 * b);
                    M = Mn;
                }
            }
        }
        float *dst = p.out + (size_t)(kvh * G + g) * HD + 2 * d2;
        dst[0] = O0 / L;
        dst[1] = O1 / L;
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
