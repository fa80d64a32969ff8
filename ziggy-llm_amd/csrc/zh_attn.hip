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
#include <cstring>
#include <type_traits>

#include "zh_internal.h"
#include "zh_mv.h"
#include "zh_quant.h"

namespace zh {

constexpr int kChunk = 64;
constexpr int kMergeSplits = 32;  // splits the merge folds per round of loads
constexpr int kMaxGroup = 8;
constexpr int QV_MAX = 8;  // q values per thread at most (8 heads of 256)

__device__ __forceinline__ float wsum(float v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// RoPE angles of one position, once per workgroup: cs[i], sn[i] for pair i
// of the n_rot rotated dims, theta = pos / base^(2i / n_rot) (applyRoPE,
// model/loader.zig:3827-3866).
// Cache row of position t, through the page table (a page is 1 << page_shift
// consecutive positions in consecutive rows; a contiguous cache passes the
// identity table).
// The table is read through the constant address space: with a uniform t
// that is a scalar load, whose wait does not cover the vector loads in flight
// (a vector load's wait would, vmcnt completing in order).
typedef const __attribute__((address_space(4))) uint32_t *const_u32_ptr;
// Pages hold 1 << kKvPageShift positions (the launcher checks page_shift).
__device__ __forceinline__ size_t kv_row(const AttnParams &p, int t) {
    constexpr int m = (1 << kKvPageShift) - 1;
    const uint32_t page = ((const_u32_ptr)p.page_table)[t >> kKvPageShift];
    return ((size_t)page << kKvPageShift) + (size_t)(t & m);
}

// This thread's RoPE denominator base^(2t / n_rot) (t = threadIdx.x < n_rot / 2): the host's table when
// given, read early so that its wait does not cover the K/V loads issued after it.
// Split in two so a kernel can issue the table read early and use it late:
// rope_den_load reads the table entry unconditionally (a valid dummy
// address without the table), rope_den_finish picks the value.
__device__ __forceinline__ float rope_den_load(int n_rot, const float *denom, const float *dummy) {
    const int half = n_rot / 2 > 0 ? n_rot / 2 : 1;
    return (denom ? denom : dummy)[min((int)threadIdx.x, half - 1)];
}
__device__ __forceinline__ float rope_den_finish(float d, int n_rot, float base, const float *denom) {
    const int t = threadIdx.x;
    if (t >= n_rot / 2) return 1.f;
    return denom ? d : powf(base, (float)(2 * t) / (float)n_rot);
}
__device__ __forceinline__ float rope_den(int n_rot, float base, const float *denom, const float *dummy) {
    return rope_den_finish(rope_den_load(n_rot, denom, dummy), n_rot, base, denom);
}
__device__ __forceinline__ void rope_table(int n_rot, float den, int pos, float *cs, float *sn) {
    const int t = threadIdx.x;
    if (t < n_rot / 2) {
        const float theta = (float)pos / den;
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
__device__ __forceinline__ void norm_rope_w(float (&x)[V], int n, bool has_norm, const float (&nw)[V], float eps,
                                            int n_rot, int style, const float *cs, const float *sn, float *dst,
                                            float *red);
template <int HD, int V>
__device__ __forceinline__ void norm_rope(float (&x)[V], int n, const float *norm_w, float eps, int n_rot, int style,
                                          const float *cs, const float *sn, float *dst, float *red) {
    float nw[V];
#pragma unroll
    for (int i = 0; i < V; i++) nw[i] = norm_w && threadIdx.x + 256 * i < n ? norm_w[(threadIdx.x + 256 * i) % HD] : 0.f;
    norm_rope_w<HD, V>(x, n, norm_w != nullptr, nw, eps, n_rot, style, cs, sn, dst, red);
}
// The same with the norm weights of this thread's values already loaded
// (nw[i] = norm_w[(tid + 256 i) % HD]), so that no load waits inside.
template <int HD, int V>
__device__ __forceinline__ void norm_rope_w(float (&x)[V], int n, bool has_norm, const float (&nw)[V], float eps,
                                            int n_rot, int style, const float *cs, const float *sn, float *dst,
                                            float *red) {
    const int tid = threadIdx.x, wave = tid >> 6;
    constexpr int WPH = HD / 64;  // wavefronts per head
    if (has_norm) {
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
            if (idx < n) x[i] = (scale * x[i]) * nw[i];
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

// Max / sum over aligned groups of n lanes (n = 4, 8, 16 or 32), valid in
// every lane of the group: DPP within 16-lane rows, a lane swap across rows.
// Each step pairs a lane with one holding the other half of its group's
// partial (the mirrors reach the other quad / half row, whose lanes all hold
// the same value by then), so the bits equal an xor butterfly's of ascending
// distance.
__device__ __forceinline__ float lanes_max(float v, int n) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    if (n >= 8) v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    if (n >= 16) v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    if (n >= 32) v = xmax<16>(v);
    return v;
}
__device__ __forceinline__ float lanes_sum(float v, int n) {
    v = group_sum16(v, min(n, 16));
    if (n >= 32) v = xsum<16>(v);
    return v;
}

// Max / sum over aligned groups of 32 lanes (half wavefronts); the total is
// valid in every lane of the group.
__device__ __forceinline__ float half_max32(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    return xmax<16>(v);
}
__device__ __forceinline__ float half_sum32(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    return xsum<16>(v);
}

// Arrival of a split and, in the last workgroup of a kv head (partials slot)
// to arrive, the merge of every split (partials stored with agent-scope
// write-through); out_of(g) is head g's output row.  A partials slot holds VS
// heads per split; the merge folds MS splits per round of loads (VS x MS =
// 256: one thread per (head, split) pair).
template <int HD, int KG, class OutOf, int VS = kMaxGroup, int MS = kMergeSplits>
__device__ __forceinline__ void split_merge(const AttnParams &p, int kvh, int G, int nsplit, int *last_ptr,
                                            OutOf out_of) {
    static_assert(VS * MS == 256, "one thread per (head, split) pair");
    const int tid = threadIdx.x;
    int &last_s = *last_ptr;
    constexpr int IPTM = (KG * HD / 2 + 255) / 256;
    __shared__ float fm_merge[VS], fl_merge[VS], fa_merge[VS];
    float acc_merge[IPTM][2];
    // Every thread's partial stores (agent scope, write-through)
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

    // Merge, one round of loads: every split's (m, l) of every head (one per
    // thread) and, for each item (pair of dims of one head), every split's
    // partial, all in flight together; the weights exp2(m_s - M) / L go
    // through LDS.
    __shared__ float wt_s[VS][MS];
    const unsigned long long *ml = reinterpret_cast<const unsigned long long *>(p.part_ml) +
                                   (size_t)kvh * p.max_splits * VS;
    const unsigned long long *po = reinterpret_cast<const unsigned long long *>(p.part_o) +
                                   (size_t)kvh * p.max_splits * VS * (HD / 2);
    constexpr int IPT = IPTM;  // items per thread at most
    for (int s0 = 0; s0 < nsplit; s0 += MS) {
        const int ns = min(MS, nsplit - s0);
        unsigned long long ov[IPT][MS];
#pragma unroll
        for (int k = 0; k < IPT; k++) {
            const int it = min(tid + 256 * k, G * HD / 2 - 1);
            const int g = it / (HD / 2), d2 = it % (HD / 2);
#pragma unroll
            for (int u = 0; u < MS; u++) {
                const size_t e = (size_t)(s0 + min(u, ns - 1)) * VS + g;
                ov[k][u] = __hip_atomic_load(po + e * (HD / 2) + d2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        {
            // thread (g, u) = (tid / MS, tid % MS)
            const int g = tid / MS, u = tid % MS;
            float ms = -INFINITY, ls = 0.f;
            if (g < G && u < ns) {
                const unsigned long long v = __hip_atomic_load(ml + (size_t)(s0 + u) * VS + g, __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT);
                ms = __uint_as_float((uint32_t)v);
                ls = __uint_as_float((uint32_t)(v >> 32));
            }
            // max and weighted sum over the MS lanes of head g (a wavefront holds 64 / MS heads)
            float mx = ms;
#pragma unroll
            for (int o = MS / 2; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            // fold into the running (M, L) of earlier rounds
            const float Mp = s0 == 0 ? -INFINITY : fm_merge[g < VS ? g : 0];
            const float M = fmaxf(mx, Mp);
            const float w = ms == -INFINITY ? 0.f : exp2f(ms - M);
            float lw = ls * w;
#pragma unroll
            for (int o = MS / 2; o >= 1; o >>= 1) lw += __shfl_xor(lw, o, 64);
            __syncthreads();  // earlier round's weights read
            if (g < G) {
                wt_s[g][u] = w;
                if (u == 0) {
                    const float a = Mp == -INFINITY ? 0.f : exp2f(Mp - M);
                    fa_merge[g] = a;  // rescale of the earlier rounds' sums
                    fl_merge[g] = (s0 == 0 ? 0.f : fl_merge[g] * a) + lw;
                    fm_merge[g] = M;
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int k = 0; k < IPT; k++) {
            const int it = tid + 256 * k;
            if (it >= G * HD / 2) continue;
            const int g = it / (HD / 2);
            float O0 = 0.f, O1 = 0.f;
#pragma unroll
            for (int u = 0; u < MS; u++) {
                if (u < ns) {
                    const float w = wt_s[g][u];
                    O0 = fmaf(__uint_as_float((uint32_t)ov[k][u]), w, O0);
                    O1 = fmaf(__uint_as_float((uint32_t)(ov[k][u] >> 32)), w, O1);
                }
            }
            if (s0 > 0) {
                const float a = fa_merge[g];
                O0 = fmaf(acc_merge[k][0], a, O0);
                O1 = fmaf(acc_merge[k][1], a, O1);
            }
            acc_merge[k][0] = O0;
            acc_merge[k][1] = O1;
        }
    }
#pragma unroll
    for (int k = 0; k < IPT; k++) {
        const int it = tid + 256 * k;
        if (it >= G * HD / 2) continue;
        const int g = it / (HD / 2), d2 = it % (HD / 2);
        float *dst = out_of(g) + 2 * d2;
        dst[0] = acc_merge[k][0] / fl_merge[g];
        dst[1] = acc_merge[k][1] / fl_merge[g];
    }
    if (tid == 0) __hip_atomic_store(&p.counters[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- polled merge (AttnParams::poll_merge) ----

// Refills this workgroup's partials slot of the other set with kPollEmpty
// (VS heads of HD values and their (m, l) pairs), for the next launch.
template <int HD, int VS>
__device__ __forceinline__ void poll_reset_slot(const AttnParams &p, int kvh, int split) {
    const size_t e = ((size_t)kvh * p.max_splits + split) * VS;
    uint4 *o = reinterpret_cast<uint4 *>(p.reset_o + e * HD);
    const uint4 empty = make_uint4(kPollEmpty, kPollEmpty, kPollEmpty, kPollEmpty);
    for (int i = threadIdx.x; i < VS * HD / 4; i += 256) o[i] = empty;
    if (threadIdx.x < VS) reinterpret_cast<uint2 *>(p.reset_ml)[e + threadIdx.x] = make_uint2(kPollEmpty, kPollEmpty);
}

// PQ: this workgroup's slice (split of max_splits) of kv head kvh's words of
// the next launch's q, k and v ([q: head_count HD][k: kv_dim][v: kv_dim]
// from qkv_refill) back to kPollEmpty.
template <int HD>
__device__ __forceinline__ void qkv_reset_slice(const AttnParams &p, int kvh, int split, int nq) {
    const int per_head = nq + 2 * HD, per = (per_head + p.max_splits - 1) / p.max_splits;
    const int lo = split * per, hi = min(lo + per, per_head);
    const size_t Q = (size_t)p.head_count * HD, KV = (size_t)p.head_count_kv * HD;
    for (int i = lo + (int)threadIdx.x; i < hi; i += 256) {
        const size_t o = i < nq        ? (size_t)kvh * nq + i
                         : i < nq + HD ? Q + (size_t)kvh * HD + (i - nq)
                                       : Q + KV + (size_t)kvh * HD + (i - nq - HD);
        p.qkv_refill[o] = __uint_as_float(kPollEmpty);
    }
}

__device__ __forceinline__ bool poll_empty(unsigned long long v) {
    return (uint32_t)v == kPollEmpty || (uint32_t)(v >> 32) == kPollEmpty;
}

// Bound of a polled wait: about a quarter of a second, far past any real wait
// (microseconds); on expiry the flag is set and the workgroup goes on.
constexpr long kPollSpin = 1L << 18;

// Split `split` of nsplit merges pairs [split * per, (split + 1) * per) of the
// head's G * HD / 2 output pairs, per = ceil(pairs / nsplit).  SL lanes serve
// one pair (SL = the power of two at or above nsplit, at least 4 and at most
// 32; a lane holds splits lane, lane + SL, ... up to 64), so 256 / SL pairs go
// at once, and kR such rounds are polled and folded together (at 4k
// positions: 23 splits of 12 pairs, 8 pairs a round).  Each lane polls its
// splits' partial pair and (m, l) until neither is kPollEmpty (device-scope
// loads: the partials come from other CUs), then the SL lanes fold them:
// M = max m_s, w_s = 2^(m_s - M), out = (sum w_s o_s) / (sum w_s l_s), with
// register-to-register lane exchanges (lanes_max / lanes_sum: an LDS-path
// shuffle took about 0.1 us a step here, and a round has ten steps).  The
// fold's order is fixed by the lanes, so the result does not depend on which
// split stored first.
template <int HD, int VS>
__device__ __forceinline__ void polled_merge(const AttnParams &p, int kvh, int split, int G, int nsplit, float *out) {
    const int npairs = G * HD / 2;
    const int per = (npairs + nsplit - 1) / nsplit;
    const int first = split * per, last = min(first + per, npairs);
    const unsigned long long *po = reinterpret_cast<const unsigned long long *>(p.part_o) +
                                   (size_t)kvh * p.max_splits * VS * (HD / 2);
    const unsigned long long *ml = reinterpret_cast<const unsigned long long *>(p.part_ml) +
                                   (size_t)kvh * p.max_splits * VS;
    const int SL = nsplit <= 4 ? 4 : nsplit <= 8 ? 8 : nsplit <= 16 ? 16 : 32;
    const int tid = threadIdx.x, lane = tid & (SL - 1), row = tid / SL, rows = 256 / SL;
    constexpr int kC = 2;  // splits per lane (SL = 32: 64 splits)
    constexpr int kR = 2;  // rounds of pairs polled together
    for (int i0 = first; i0 < last; i0 += kR * rows) {
        int g[kR], d2[kR];
        unsigned long long ov[kR][kC], mv[kR][kC];
        bool need[kR][kC];
#pragma unroll
        for (int r = 0; r < kR; r++) {
            const int it = min(i0 + r * rows + row, last - 1);
            g[r] = it / (HD / 2);
            d2[r] = it % (HD / 2);
#pragma unroll
            for (int c = 0; c < kC; c++) {
                need[r][c] = lane + SL * c < nsplit && i0 + r * rows < last;
                ov[r][c] = mv[r][c] = 0ull;
            }
        }
        long spin = 0;
        for (;;) {
#pragma unroll
            for (int r = 0; r < kR; r++)
#pragma unroll
                for (int c = 0; c < kC; c++) {
                    const int sp = min(lane + SL * c, nsplit - 1);
                    if (need[r][c]) {
                        ov[r][c] = __hip_atomic_load(po + ((size_t)sp * VS + g[r]) * (HD / 2) + d2[r],
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        mv[r][c] = __hip_atomic_load(ml + (size_t)sp * VS + g[r], __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            bool waiting = false;
#pragma unroll
            for (int r = 0; r < kR; r++)
#pragma unroll
                for (int c = 0; c < kC; c++) {
                    need[r][c] = need[r][c] && (poll_empty(ov[r][c]) || poll_empty(mv[r][c]));
                    waiting = waiting || need[r][c];
                }
            if (!__any(waiting)) break;
            if (++spin > kPollSpin) {
                if ((tid & 63) == 0) __hip_atomic_store(p.poll_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        // the kR folds side by side (independent chains; a round past the
        // slice folds zeros and stores nothing)
        float mx[kR], O0[kR], O1[kR], L[kR];
#pragma unroll
        for (int r = 0; r < kR; r++) {
            mx[r] = -INFINITY;
#pragma unroll
            for (int c = 0; c < kC; c++)
                if (lane + SL * c < nsplit) mx[r] = fmaxf(mx[r], __uint_as_float((uint32_t)mv[r][c]));
            mx[r] = lanes_max(mx[r], SL);
        }
#pragma unroll
        for (int r = 0; r < kR; r++) {
            O0[r] = O1[r] = L[r] = 0.f;
#pragma unroll
            for (int c = 0; c < kC; c++) {
                const float m = lane + SL * c < nsplit ? __uint_as_float((uint32_t)mv[r][c]) : -INFINITY;
                const float w = m == -INFINITY ? 0.f : exp2f(m - mx[r]);
                O0[r] = fmaf(__uint_as_float((uint32_t)ov[r][c]), w, O0[r]);
                O1[r] = fmaf(__uint_as_float((uint32_t)(ov[r][c] >> 32)), w, O1[r]);
                L[r] = fmaf(__uint_as_float((uint32_t)(mv[r][c] >> 32)), w, L[r]);
            }
            O0[r] = lanes_sum(O0[r], SL);
            O1[r] = lanes_sum(O1[r], SL);
            L[r] = lanes_sum(L[r], SL);
        }
#pragma unroll
        for (int r = 0; r < kR; r++)
            if (lane == 0 && i0 + r * rows + row < last) {
                float *dst = out + (size_t)g[r] * HD + 2 * d2[r];
                dst[0] = O0[r] / L[r];
                dst[1] = O1[r] / L[r];
            }
    }
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
    auto row_off = [&](int i) { return kv_row(p, min(pos_of(min(i, npass - 1)), pos)) * p.kv_dim + kv_off + 16 * sub; };
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
        rope_table(n_rot, rope_den(n_rot, p.rope_base, p.rope_denom, p.q), pos, cs_s, sn_s);
        norm_rope<HD, QV>(qv, nq, p.q_norm, p.eps, n_rot, p.rope_style, cs_s, sn_s, &q_s[0][0], red16);
        if (own_pos) {
            norm_rope<HD, 1>(kx, HD, p.k_norm, p.eps, n_rot, p.rope_style, cs_s, sn_s, kn_s, red16);
            if (tid < HD) {
                const __half kh = __float2half_rn(kn_s[tid]), vh = __float2half_rn(vx);
                if (pos < p.ctx) {
                    const size_t idx = kv_row(p, pos) * p.kv_dim + kv_off + tid;
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

    split_merge<HD, GG ? GG : kMaxGroup>(p, kvh, G, nsplit, &last_s,
                                         [&](int g) { return p.out + (size_t)(kvh * G + g) * HD; });
}

// ---------------------------------------------------------------------------
// Matrix-core variant (head_dim 64 and 128): the same grid, splits, fused
// q/k/v epilogue, partials and last-arriver merge as attn_kernel, with the
// position loop on v_mfma_f32_16x16x32_f16.
//
// A wavefront takes tiles of 32 positions (units u_begin + wave + 4 t).
//   scores  S[pos][col] = sum_d K[pos][d] Q[d][col]: A = K rows as stored
//           (binary16, exact), B = the query pieces: column 2g + 0 holds
//           binary16(q_g * scale * log2 e), column 2g + 1 the binary16 of
//           the remainder, so S[pos][2g] + S[pos][2g + 1] is the score of
//           head g to ~2^-22 relative (products of binary16 values are exact
//           in the f32 accumulator).  Two 16-row tiles per 32 positions,
//           head_dim / 32 k-steps each.
//   softmax online per column (base 2), the row pieces summed by one DPP.
//   values  O[col][dim] += sum_pos P[col][pos] V[pos][dim]: A = the
//           probabilities split the same way (column 2g + 0: binary16(p),
//           2g + 1: binary16(p - hi)), laid out exactly as the scores came
//           out of the first product; B = V rows: each lane reads 16 bytes
//           (dims 8j .. 8j + 7) of eight rows, and product q (0..7) takes
//           element q of each, so its output column j stands for dim 8j + q.
//   A reduction index (k) may be assigned to (lane group, element) in any way
//   as long as A and B agree; both products use that freedom.
// The workgroup merges its four wavefronts through LDS (max, rescale, sum of
// the two pieces of each head) and continues as attn_kernel does.
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

// per-component select (a select of whole vector structs becomes a select of
// their addresses, which keeps the arrays holding them out of registers)
__device__ __forceinline__ void pick4(bool c, const uint4 &a, uint4 &dst) {
    dst.x = c ? a.x : dst.x;
    dst.y = c ? a.y : dst.y;
    dst.z = c ? a.z : dst.z;
    dst.w = c ? a.w : dst.w;
}

__device__ __forceinline__ h8v as_h8(uint4 v) {
    h8v r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// MQ: several queries at consecutive positions (plain mode, q already
// normed and rotated, their K/V rows already in the cache).  Workgroup z takes
// queries qbase .. qbase + nqw - 1 (16 / Gq of them): query head g of query j
// becomes column pair ("virtual head") j Gq + g, whose causal range ends at
// its own position; splits cover the range of the last query.  A wavefront
// holds two 16-column query tiles (virtual heads 0-7 and 8-15) against the
// same K/V registers, so the K/V range is read once per 16 virtual heads.
// PQ (single query, fused mode): the projection's q, k and v come from
// workgroups of the same launch (qkv_attn_kernel) with device-scope stores
// over words that hold kPollEmpty until then.  They are read after the K and
// V tile loads are issued, again while any word of the head's still holds
// kPollEmpty (bounded: on expiry the error flag is set and the values are
// taken as they are); each workgroup then refills its slice of the next
// launch's q/k/v words (qkv_refill) with kPollEmpty.
// VNOW (with PQ): the V tiles issued right after the q/k/v wait, under the q
// prologue, instead of after it; the host picks it for long contexts (a
// split's many tiles make the V stream the longer part there; with few, the
// prologue is, and loads queued ahead of it delay it).
template <int HD, int GG, bool MQ, bool PQ = false, bool VNOW = false>
__device__ __forceinline__ void attn_mfma_body(const AttnParams &p, const int split, const int kvh, const int qz) {
    static_assert(!PQ || !MQ, "polled q/k/v: single query");
    constexpr int KS = HD / 32;  // 32-dim steps of the scores, 32-dim chunks of the values
    constexpr int TP = 32;       // positions per wavefront tile
    constexpr int QS = HD + 8;   // padded row of the query pieces (binary16)
    constexpr int LPR = HD / 8;  // lanes per value row (8 dims each)
    constexpr int NT = MQ ? 2 : 1;      // 16-column query tiles per wavefront
    constexpr int VG = kMaxGroup * NT;  // (virtual) heads per workgroup at most
    static_assert(!MQ || VG == kMultiHeads, "multi-query partials are sized by kMultiHeads");
    touch_params(p);
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
    const int Gq = GG ? GG : p.head_count / p.head_count_kv;  // query heads per kv head
    const int qpw = MQ ? VG / Gq : 1, qbase = MQ ? qz * qpw : 0;
    const int nqw = MQ ? min(qpw, p.n_query - qbase) : 1;
    const int slot = MQ ? kvh + p.head_count_kv * qz : kvh;  // partials / arrival counter
    const int G = MQ ? nqw * Gq : Gq;                                  // (virtual) heads of the workgroup
    const bool fused = !MQ && p.k_new != nullptr;
    const size_t kv_off = (size_t)kvh * HD;
    constexpr int QV = VG * HD / 256;
    const int nq = G * HD;
    const int n_rot_f = p.rope_dim < HD ? p.rope_dim : HD;

    // The prologue's loads first, none depending on the position, all
    // unconditional (clamped indices, a valid dummy address for an absent
    // bias or norm), and none used before the K loads are issued: a load
    // under a branch, or one whose value is used at once, makes the compiler
    // wait for it there, and each such wait is a memory round trip before
    // the K stream starts.
    float qv[QV], qb[QV], kx[1] = {0.f}, kb = 0.f, vx = 0.f, vb = 0.f, qnw[QV], knw[1];
    const float rden_raw = rope_den_load(n_rot_f, p.rope_denom, p.q);
    {
        const float *qn = p.q_norm ? p.q_norm : p.q, *kn = p.k_norm ? p.k_norm : p.q;
#pragma unroll
        for (int i = 0; i < QV; i++) qnw[i] = qn[(tid + 256 * i) % HD];
        knw[0] = kn[tid % HD];
        const float *qbp = fused && p.q_bias ? p.q_bias : p.q;
#pragma unroll
        for (int i = 0; i < QV; i++) {
            const int idx = min(tid + 256 * i, nq - 1);
            if (MQ) {
                const int gv = idx / HD, j = gv / Gq;
                qv[i] = p.q[(size_t)(qbase + j) * p.q_stride + (size_t)(kvh * Gq + gv - j * Gq) * HD + idx % HD];
            } else {
                if constexpr (!PQ) qv[i] = p.q[(size_t)kvh * nq + idx];  // PQ: polled below
                qb[i] = qbp[(size_t)kvh * nq + idx];
            }
        }
        // plain mode reads q in place of the absent k / v and ignores it
        const float *knp = fused ? p.k_new : p.q, *vnp = fused ? p.v_new : p.q;
        const float *kbp = fused && p.k_bias ? p.k_bias : p.q, *vbp = fused && p.v_bias ? p.v_bias : p.q;
        if constexpr (!PQ) {
            kx[0] = knp[kv_off + tid % HD];
            vx = vnp[kv_off + tid % HD];
        }
        kb = kbp[kv_off + tid % HD];
        vb = vbp[kv_off + tid % HD];
    }
    // the position through the scalar cache (a scalar load: its wait does not
    // cover the vector loads above)
    typedef const __attribute__((address_space(4))) int *const_i32_ptr;
    const int pos0 = p.position_dev ? *(const_i32_ptr)p.position_dev : p.position;
    const int pos = pos0 + qbase + nqw - 1;  // the last query's position
    int pos_col[NT];                         // causal end of column li of tile nt
#pragma unroll
    for (int nt = 0; nt < NT; nt++) pos_col[nt] = MQ ? pos0 + qbase + ((li >> 1) + 8 * nt) / Gq : pos;
    // tiles start on a multiple of 32 positions at or below window_start, so
    // a tile never crosses a page; positions below the window are masked
    const int wb = p.window_start & ~(TP - 1);
    const int n_total = pos + 1 - wb;
    const int units = (n_total + TP - 1) / TP;
    // tiles per split; a single query takes at least kMinTiles per split
    // (fewer partials to merge: 6 tiles took 12.8 -> 12.5 us at 4k positions,
    // 8 tiles 12.3 us, 10 tiles 14.6 us, the same grid at 16k, where every
    // split holds more)
    const int min_tiles = MQ ? 1 : p.min_tiles > 0 ? p.min_tiles : 8;
    const int per = max((units + p.max_splits - 1) / p.max_splits, min_tiles);
    const int nsplit = (units + per - 1) / per;
    const bool polled = !MQ && p.poll_merge;
    // the other set's slot of this workgroup, refilled for the next launch
    // (after the K loads: stores ahead of them would delay them)
    auto refill_other = [&]() {
        if (polled) poll_reset_slot<HD, VG>(p, kvh, split);
        if constexpr (PQ) qkv_reset_slice<HD>(p, kvh, split, nq);
    };
    if (split >= nsplit) {
        refill_other();
        return;
    }
    const int u_begin = split * per, nu = min(per, units - u_begin);
    const int ntw = nu > wave ? (nu - wave + 3) / 4 : 0;  // this wavefront's tiles
    const bool two = NT > 1 && G > kMaxGroup;                 // the second query tile is in use
    const bool own_pos = fused && u_begin + nu == units;  // this split holds the current position

    __shared__ float q_s[VG][HD];
    __shared__ float kn_s[HD];
    __shared__ __align__(16) unsigned short kn_h[HD], vn_h[HD];
    __shared__ float red16[4 * QV_MAX];
    __shared__ float cs_s[HD / 2], sn_s[HD / 2];
    __shared__ __align__(16) unsigned short qp_s[16 * NT][QS];
    __shared__ float mlw_s[4][16 * NT][2];
    __shared__ __align__(16) float o_s[4][VG][HD];
    __shared__ float fm_s[VG], fl_s[VG];
    __shared__ int last_s;

    // the wavefront index as a scalar: tile positions, and the page-table
    // reads below, are uniform, so the reads are scalar loads whose waits do
    // not cover the vector loads in flight
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    auto p0_of = [&](int t) { return wb + (u_begin + wv + 4 * t) * TP; };
    // where tile t's loads go: past the wavefront's own tiles (the first two
    // are loaded whatever its count, the ring refills in pairs) they re-read
    // the split's last tile, which the workgroup reads anyway, rather than
    // the next split's rows (5.6 MB more HBM reads per launch at 4k)
    auto lp0_of = [&](int t) { return wb + (u_begin + min(wv + 4 * t, nu - 1)) * TP; };
    // a tile's 32 positions lie in one page (tiles start at multiples of 32 and
    // pages hold 64 or more): one table read per tile, rows of the page after
    // it.  A tile past pos (its rows all clamp to pos) reads pos's entry, so
    // the table is never read past the context.
    auto tile_row = [&](int b) {
        const int bb = min(b, pos);
        return (long long)kv_row(p, bb) - bb;
    };
    // the first two tiles' pages (scalar loads), then the K loads
    const long long tb_first[2] = {tile_row(lp0_of(0)), tile_row(lp0_of(1))};
    __builtin_amdgcn_sched_barrier(0);

    // tile t: positions p0(t) .. p0(t) + 31; K fragments [row tile][k-step]
    // (row p0 + 16 rt + li, dims 32 ks + 8 lg .. + 7), V fragments [row e]
    // (rows 4 lg + e and 16 + 4 lg + e - 4, dims 8 li .. 8 li + 7).  Rows
    // past pos re-read row pos (masked below).
    auto load_k = [&](int t, uint4 (&k)[2][KS]) {
        const int b = lp0_of(t);
        const long long tb = t < 2 ? tb_first[t] : tile_row(b);
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
            const __half *src = p.k_cache + (size_t)(tb + min(b + 16 * rt + li, pos)) * p.kv_dim + kv_off + 8 * lg;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) k[rt][ks] = *reinterpret_cast<const uint4 *>(src + 32 * ks);
        }
    };
    auto vrow = [&](int e) { return e < 4 ? 4 * lg + e : 12 + 4 * lg + e; };
    auto load_v = [&](int t, uint4 (&v)[8]) {
        const int b = lp0_of(t);
        const long long tb = t < 2 ? tb_first[t] : tile_row(b);
#pragma unroll
        for (int e = 0; e < 8; e++)
            v[e] = *reinterpret_cast<const uint4 *>(p.v_cache + (size_t)(tb + min(b + vrow(e), pos)) * p.kv_dim +
                                                    kv_off + 8 * (li % LPR));
    };
    // Unconditional (clamped) loads: a load under a branch leaves the
    // compiler's wait counting unsure of what is in flight, and the first
    // wait for q would then cover every K/V load as well.
    // K now, V after the q prologue: the prologue's VALU work runs while K
    // streams in (a wavefront stalls at issue once its loads fill the queue)
    uint4 kr[2][2][KS];
    uint4 vr[2][8];
    load_k(0, kr[0]);
    load_k(1, kr[1]);
    // the other sets' refill goes out now, while the workgroup waits for q
    // (after the K loads, which it would otherwise delay; no set it refills
    // is read by this launch), not at its end
    refill_other();
    // the RoPE table depends only on the position: built while q is still
    // on its way (a barrier orders it before its readers: the poll loop's,
    // or norm_rope_w's own)
    const float rden = fused ? rope_den_finish(rden_raw, n_rot_f, p.rope_base, p.rope_denom) : 1.f;
    if (fused) rope_table(n_rot_f, rden, pos, cs_s, sn_s);
    if constexpr (PQ) {
        // this head's q, k and v as the projection workgroups store them
        const uint32_t *qw = reinterpret_cast<const uint32_t *>(p.q) + (size_t)kvh * nq;
        const uint32_t *kw = reinterpret_cast<const uint32_t *>(p.k_new) + kv_off + tid % HD;
        const uint32_t *vw = reinterpret_cast<const uint32_t *>(p.v_new) + kv_off + tid % HD;
        for (long spin = 0;; spin++) {
            bool empty = false;
#pragma unroll
            for (int i = 0; i < QV; i++) {
                const uint32_t u = __hip_atomic_load(qw + min(tid + 256 * i, nq - 1), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
                qv[i] = __uint_as_float(u);
                empty = empty || u == kPollEmpty;
            }
            const uint32_t uk = __hip_atomic_load(kw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t uv = __hip_atomic_load(vw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            kx[0] = __uint_as_float(uk);
            vx = __uint_as_float(uv);
            empty = empty || uk == kPollEmpty || uv == kPollEmpty;
            if (!__syncthreads_or(empty)) break;
            if (spin > kPollSpin) {
                if (tid == 0) __hip_atomic_store(p.poll_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if constexpr (VNOW) {
            load_v(0, vr[0]);
            load_v(1, vr[1]);
        }
    }
    // the projection biases (the bias reads above are dummies when absent)
    if (fused) {
#pragma unroll
        for (int i = 0; i < QV; i++)
            if (p.q_bias && tid + 256 * i < nq) qv[i] += qb[i];
        if (own_pos && tid < HD) {
            if (p.k_bias) kx[0] += kb;
            if (p.v_bias) vx += vb;
        }
    }
#pragma unroll
    for (int i = 0; i < QV; i++)
        if (tid + 256 * i >= nq) qv[i] = 0.f;

    if (fused) {
        const int n_rot = n_rot_f;
        norm_rope_w<HD, QV>(qv, nq, p.q_norm != nullptr, qnw, p.eps, n_rot, p.rope_style, cs_s, sn_s, &q_s[0][0],
                            red16);
        if (own_pos) {
            norm_rope_w<HD, 1>(kx, HD, p.k_norm != nullptr, knw, p.eps, n_rot, p.rope_style, cs_s, sn_s, kn_s, red16);
            if (tid < HD) {
                const __half kh = __float2half_rn(kn_s[tid]), vh = __float2half_rn(vx);
                if (pos < p.ctx) {
                    const size_t idx = kv_row(p, pos) * p.kv_dim + kv_off + tid;
                    p.k_cache[idx] = kh;
                    p.v_cache[idx] = vh;
                }
                kn_h[tid] = __half_as_ushort(kh);
                vn_h[tid] = __half_as_ushort(vh);
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
    // query pieces, scaled to base-2 scores
    const float sl2 = p.scale * 1.44269504088896340736f;
    for (int it = tid; it < 16 * NT * HD; it += 256) {
        const int col = it / HD, d = it % HD, g = col >> 1;
        unsigned short h = 0;
        if (g < G) {
            const float v = q_s[g][d] * sl2;
            const __half hi = __float2half_rn(v);
            h = (col & 1) ? __half_as_ushort(__float2half_rn(v - __half2float(hi))) : __half_as_ushort(hi);
        }
        qp_s[col][d] = h;
    }
    __syncthreads();
    if constexpr (!(PQ && VNOW)) {
        load_v(0, vr[0]);
        load_v(1, vr[1]);
    }
    h8v qf[NT][KS];
    bool col_ok[NT];
    float m[NT], lsum[NT];  // for column li of tile nt
    f4v o[NT][8];           // [nt][q]: rows 4 lg + r, dims 8 li + q
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
            qf[nt][ks] = as_h8(*reinterpret_cast<const uint4 *>(&qp_s[16 * nt + li][32 * ks + 8 * lg]));
        col_ok[nt] = 16 * nt + li < 2 * G;
        m[nt] = -INFINITY;
        lsum[nt] = 0.f;
#pragma unroll
        for (int q = 0; q < 8; q++) o[nt][q] = f4v{0.f, 0.f, 0.f, 0.f};
    }

    for (int t0 = 0; t0 < ntw; t0 += 2) {
        float sc[NT][2][2][4];
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const bool have = t0 + tt < ntw;
            const int b = p0_of(t0 + tt);
            if (have && own_pos && pos >= b && pos < b + TP) {
                // this step's k and v replace the rows of pos (loaded before the store)
#pragma unroll
                for (int rt = 0; rt < 2; rt++) {
                    const bool me = b + 16 * rt + li == pos;
#pragma unroll
                    for (int ks = 0; ks < KS; ks++) {
                        const uint4 kn = *reinterpret_cast<const uint4 *>(&kn_h[32 * ks + 8 * lg]);
                        pick4(me, kn, kr[tt][rt][ks]);
                    }
                }
                const uint4 vn = *reinterpret_cast<const uint4 *>(&vn_h[8 * (li % LPR)]);
#pragma unroll
                for (int e = 0; e < 8; e++) pick4(b + vrow(e) == pos, vn, vr[tt][e]);
            }
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    f4v acc = {0.f, 0.f, 0.f, 0.f};
                    if (have && (nt == 0 || two)) {
#pragma unroll
                        for (int ks = 0; ks < KS; ks++)
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(kr[tt][rt][ks]), qf[nt][ks], acc, 0, 0,
                                                                         0);
                    }
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        // rows 4 lg + r of the tile; the two pieces of a head sit in lanes 2g, 2g + 1
                        float v = acc[r];
                        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
                        const int pr = b + 16 * rt + 4 * lg + r;
                        const bool valid = have && col_ok[nt] && pr <= pos_col[nt] && pr >= p.window_start;
                        sc[nt][tt][rt][r] = valid ? v : -INFINITY;
                    }
                }
        }
        if (t0 + 2 < ntw) {  // the next two tiles into the K slots just consumed
            load_k(t0 + 2, kr[0]);
            load_k(t0 + 3, kr[1]);
        }
        h8v pf[NT][2];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float mt = -INFINITY;
#pragma unroll
            for (int tt = 0; tt < 2; tt++)
#pragma unroll
                for (int rt = 0; rt < 2; rt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) mt = fmaxf(mt, sc[nt][tt][rt][r]);
            mt = xmax<32>(xmax<16>(mt));
            const float mn = fmaxf(m[nt], mt);
            const float alpha = m[nt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[nt] - mn);
            m[nt] = mn;
            float ps = 0.f;
#pragma unroll
            for (int tt = 0; tt < 2; tt++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float s = sc[nt][tt][e >> 2][e & 3];
                    const float pv = s == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s - mn);
                    ps += pv;
                    const _Float16 hi = (_Float16)pv;
                    pf[nt][tt][e] = (li & 1) ? (_Float16)(pv - (float)hi) : hi;
                }
            lsum[nt] = lsum[nt] * alpha + ps;
            if (t0 > 0) {
                // rows 4 lg + r of O are columns 4 lg + r of P: their alpha
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float a = __shfl(alpha, 4 * lg + r, 64);
#pragma unroll
                    for (int q = 0; q < 8; q++) o[nt][q][r] *= a;
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            if (t0 + tt >= ntw) continue;
            // product q takes dim 8 j + q of every row: output column j stands for dim 8 j + q
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const uint32_t sel = (q & 1) ? 0x07060302u : 0x05040100u;
                uint32_t w[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint4 &r = vr[tt][e];
                    w[e] = (q >> 1) == 0 ? r.x : (q >> 1) == 1 ? r.y : (q >> 1) == 2 ? r.z : r.w;
                }
                uint4 bv;
                bv.x = __builtin_amdgcn_perm(w[1], w[0], sel);
                bv.y = __builtin_amdgcn_perm(w[3], w[2], sel);
                bv.z = __builtin_amdgcn_perm(w[5], w[4], sel);
                bv.w = __builtin_amdgcn_perm(w[7], w[6], sel);
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    if (nt == 0 || two)
                        o[nt][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[nt][tt], as_h8(bv), o[nt][q], 0, 0, 0);
            }
        }
        if (t0 + 2 < ntw) {
            load_v(t0 + 2, vr[0]);
            load_v(t0 + 3, vr[1]);
        }
    }

    // ---- merge the four wavefronts ----
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        float l = lsum[nt];
        l = xsum<32>(xsum<16>(l));
        if (lg == 0) {
            mlw_s[wave][16 * nt + li][0] = m[nt];
            mlw_s[wave][16 * nt + li][1] = l;
        }
    }
    __syncthreads();
    // rows 4 lg + 2 hh + {0, 1} of tile nt are the two pieces of head
    // 8 nt + 2 lg + hh (same max): summed here, scaled to the workgroup max,
    // one row per head
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int head = 8 * nt + 2 * lg + hh, row = 2 * head;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < 4; w++) M = fmaxf(M, mlw_s[w][row][0]);
            const float mw = mlw_s[wave][row][0];
            const float f = mw == -INFINITY ? 0.f : exp2f(mw - M);
            if (head < G && li < LPR) {
                const f4v *on = o[nt];
                float4 a, b;
                a.x = (on[0][2 * hh] + on[0][2 * hh + 1]) * f;
                a.y = (on[1][2 * hh] + on[1][2 * hh + 1]) * f;
                a.z = (on[2][2 * hh] + on[2][2 * hh + 1]) * f;
                a.w = (on[3][2 * hh] + on[3][2 * hh + 1]) * f;
                b.x = (on[4][2 * hh] + on[4][2 * hh + 1]) * f;
                b.y = (on[5][2 * hh] + on[5][2 * hh + 1]) * f;
                b.z = (on[6][2 * hh] + on[6][2 * hh + 1]) * f;
                b.w = (on[7][2 * hh] + on[7][2 * hh + 1]) * f;
                *reinterpret_cast<float4 *>(&o_s[wave][head][8 * li]) = a;
                *reinterpret_cast<float4 *>(&o_s[wave][head][8 * li + 4]) = b;
            }
        }
    if (tid < G) {
        const int row = 2 * tid;
        float M = -INFINITY, L = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, mlw_s[w][row][0]);
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float mw = mlw_s[w][row][0];
            if (mw != -INFINITY) L += mlw_s[w][row][1] * exp2f(mw - M);
        }
        fm_s[tid] = M;
        fl_s[tid] = L;
    }
    __syncthreads();
    auto out_of = [&](int g) {
        if (MQ) {
            const int j = g / Gq;
            return p.out + (size_t)(qbase + j) * p.out_stride + (size_t)(kvh * Gq + g - j * Gq) * HD;
        }
        return p.out + (size_t)(kvh * G + g) * HD;
    };
    // pairs of dims: one 64-bit write-through store per pair
    for (int it = tid; it < G * HD / 2; it += 256) {
        const int g = it / (HD / 2), d = 2 * (it % (HD / 2));
        const float2 a0 = *reinterpret_cast<const float2 *>(&o_s[0][g][d]);
        const float2 a1 = *reinterpret_cast<const float2 *>(&o_s[1][g][d]);
        const float2 a2 = *reinterpret_cast<const float2 *>(&o_s[2][g][d]);
        const float2 a3 = *reinterpret_cast<const float2 *>(&o_s[3][g][d]);
        const float x0 = (a0.x + a1.x) + (a2.x + a3.x), x1 = (a0.y + a1.y) + (a2.y + a3.y);
        if (nsplit == 1) {
            float *dst = out_of(g) + d;
            dst[0] = x0 / fl_s[g];
            dst[1] = x1 / fl_s[g];
        } else {
            const size_t e = (((size_t)slot * p.max_splits + split) * VG + g) * HD + d;
            const unsigned long long v = (unsigned long long)__float_as_uint(x0) |
                                         ((unsigned long long)__float_as_uint(x1) << 32);
            __hip_atomic_store(reinterpret_cast<unsigned long long *>(p.part_o + e), v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (nsplit == 1) return;
    if (tid < G) {
        const size_t e = ((size_t)slot * p.max_splits + split) * VG + tid;
        const unsigned long long v = (unsigned long long)__float_as_uint(fm_s[tid]) |
                                     ((unsigned long long)__float_as_uint(fl_s[tid]) << 32);
        __hip_atomic_store(reinterpret_cast<unsigned long long *>(p.part_ml) + e, v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (polled) {
        polled_merge<HD, VG>(p, kvh, split, G, nsplit, p.out + (size_t)kvh * G * HD);
        return;
    }
    // MQ: up to 16 virtual heads, 16 splits per round of the merge
    split_merge<HD, (GG && !MQ) ? GG : VG, decltype(out_of), VG, 256 / VG>(p, slot, G, nsplit, &last_s, out_of);
}

template <int HD, int GG, bool MQ>
__global__ void __launch_bounds__(256) attn_mfma_kernel(AttnParams p) {
    attn_mfma_body<HD, GG, MQ>(p, blockIdx.x, blockIdx.y, blockIdx.z);
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

// ZIGGY_HIP_ATTN_KERNEL=valu selects the vector-ALU kernel for every head
// size (the matrix-core kernel covers head_dim 64 and 128).
static bool attention_valu() {
    static const bool v = [] {
        const char *e = getenv("ZIGGY_HIP_ATTN_KERNEL");
        return e && strcmp(e, "valu") == 0;
    }();
    return v;
}

bool attention_poll_supported(int head_dim, int max_splits) {
    if (getenv("ZIGGY_HIP_ATTN_POLL") && getenv("ZIGGY_HIP_ATTN_POLL")[0] == '0') return false;
    return (head_dim == 64 || head_dim == 96 || head_dim == 128) && !attention_valu() && max_splits <= 64;
}

int attention_poll_min_tiles() {
    static const int t = [] {
        const char *e = getenv("ZIGGY_HIP_ATTN_MIN_TILES");
        const int v = e ? atoi(e) : 6;
        return v > 0 ? v : 6;
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

// The q/k/v epilogue of n_query tokens at positions position .. ahead of a
// multi-query attention launch: workgroup (token m, kv head) adds the biases,
// runs the per-head RMSNorm and RoPE of the group's q heads (written to
// q_out, which may be q itself) and of k, and stores k and v as binary16 at
// position + m -- the arithmetic of the fused single-query kernel, in the
// same order and thread layout.
template <int HD>
__global__ void __launch_bounds__(256) attn_prep_kernel(AttnParams p, float *q_out, RowScale rs, ZeroSpans z) {
    constexpr int QV = kMaxGroup * HD / 256;
    const int m = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int G = p.head_count / p.head_count_kv, nq = G * HD, pos = p.position + m;
    __shared__ float q_s[kMaxGroup * HD];
    __shared__ float kn_s[HD];
    __shared__ float red16[4 * QV_MAX];
    __shared__ float cs_s[HD / 2], sn_s[HD / 2];
    const float *qrow = p.q + (size_t)m * p.q_stride + (size_t)kvh * nq;
    const size_t kv_off = (size_t)m * p.kv_dim + (size_t)kvh * HD;
    const int n_rot = p.rope_dim < HD ? p.rope_dim : HD;
    // Every load first, none under a branch and none used before the last
    // is issued (an absent tensor reads a valid dummy address, q's): one
    // memory round trip where the row's sum of squares, then the biases one
    // by one, then the norm weights inside the norm took one each.
    const float ss = (rs.ss ? rs.ss : p.q)[rs.ss ? m : 0];
    const float *qbp = p.q_bias ? p.q_bias : p.q, *kbp = p.k_bias ? p.k_bias : p.q, *vbp = p.v_bias ? p.v_bias : p.q;
    const float *qn = p.q_norm ? p.q_norm : p.q, *kn = p.k_norm ? p.k_norm : p.q;
    float qraw[QV], qb[QV], qnw[QV], knw[1];
#pragma unroll
    for (int i = 0; i < QV; i++) {
        const int idx = min(tid + 256 * i, nq - 1);
        qraw[i] = qrow[idx];
        qb[i] = qbp[(size_t)kvh * nq + idx];
        qnw[i] = qn[(tid + 256 * i) % HD];
    }
    const float kraw = p.k_new[kv_off + tid % HD], vraw = p.v_new[kv_off + tid % HD];
    const float kbv = kbp[(size_t)kvh * HD + tid % HD], vbv = vbp[(size_t)kvh * HD + tid % HD];
    knw[0] = kn[tid % HD];
    const float rden_raw = rope_den_load(n_rot, p.rope_denom, p.q);
    // then the arithmetic, in the stand-alone steps' order: the deferred
    // RMSNorm of the q/k/v products' input row, the biases, the per-head
    // norm and RoPE
    const float r = rs.ss ? 1.0f / sqrtf(ss / (float)rs.n + rs.eps) : 1.0f;
    float qv[QV], kx[1];
#pragma unroll
    for (int i = 0; i < QV; i++) {
        const int idx = tid + 256 * i;
        qv[i] = 0.f;
        if (idx < nq) {
            qv[i] = r * qraw[i];
            if (p.q_bias) qv[i] += qb[i];
        }
    }
    kx[0] = r * kraw;
    float vx = r * vraw;
    if (tid < HD) {
        if (p.k_bias) kx[0] += kbv;
        if (p.v_bias) vx += vbv;
    }
    rope_table(n_rot, rope_den_finish(rden_raw, n_rot, p.rope_base, p.rope_denom), pos, cs_s, sn_s);
    norm_rope_w<HD, QV>(qv, nq, p.q_norm != nullptr, qnw, p.eps, n_rot, p.rope_style, cs_s, sn_s, q_s, red16);
    norm_rope_w<HD, 1>(kx, HD, p.k_norm != nullptr, knw, p.eps, n_rot, p.rope_style, cs_s, sn_s, kn_s, red16);
    float *qo = q_out + (size_t)m * p.q_stride + (size_t)kvh * nq;
    for (int idx = tid; idx < nq; idx += 256) qo[idx] = q_s[idx];
    if (tid < HD && pos < p.ctx) {
        const size_t idx = kv_row(p, pos) * p.kv_dim + (size_t)kvh * HD + tid;
        p.k_cache[idx] = __float2half_rn(kn_s[tid]);
        p.v_cache[idx] = __float2half_rn(vx);
    }
    // the spans the pass clears here (inputs of later accumulating products)
    const size_t nthr = (size_t)gridDim.x * gridDim.y * 256,
                 gt = ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 256 + tid;
#pragma unroll
    for (int j = 0; j < 4; j++)
        for (size_t i = gt; i < z.n[j]; i += nthr) z.p[j][i] = 0.f;
}

// The per-head norm reduces over whole wavefronts: heads of 64, 128 or 256
// values (no QK-norm for head_dim 96)
static bool norms_fit(const AttnParams &p) { return !(p.q_norm || p.k_norm) || p.head_dim % 64 == 0; }

hipError_t launch_attention_prep(const AttnParams &p, float *q_out, hipStream_t s, RowScale rs, const ZeroSpans &z) {
    for (int j = 0; j < 4; j++)
        if (z.n[j] && !z.p[j]) return hipErrorInvalidValue;
    if (rs.ss && rs.n < 1) return hipErrorInvalidValue;
    if (!p.page_table || p.page_shift != kKvPageShift) return hipErrorInvalidValue;
    if (p.head_count_kv <= 0 || p.head_count % p.head_count_kv || p.head_count / p.head_count_kv > kMaxGroup ||
        p.n_query < 1 || !p.q || !p.k_new || !p.v_new || !q_out || p.q_stride < p.head_count * p.head_dim)
        return hipErrorInvalidValue;
    if (!norms_fit(p)) return hipErrorInvalidValue;
    const dim3 grid(p.n_query, p.head_count_kv);
    switch (p.head_dim) {
    case 64: hipLaunchKernelGGL(attn_prep_kernel<64>, grid, dim3(256), 0, s, p, q_out, rs, z); break;
    case 96: hipLaunchKernelGGL(attn_prep_kernel<96>, grid, dim3(256), 0, s, p, q_out, rs, z); break;
    case 128: hipLaunchKernelGGL(attn_prep_kernel<128>, grid, dim3(256), 0, s, p, q_out, rs, z); break;
    case 256: hipLaunchKernelGGL(attn_prep_kernel<256>, grid, dim3(256), 0, s, p, q_out, rs, z); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// head_dim 96 has only the matrix-core kernel (the vector kernel's position
// lanes need a power-of-two head)
bool attention_multi_supported(int head_dim) {
    return head_dim == 96 || ((head_dim == 64 || head_dim == 128) && !attention_valu());
}

int attention_query_groups(int head_count, int head_count_kv, int n_query) {
    const int G = head_count_kv > 0 ? head_count / head_count_kv : 1;
    const int qpw = G > 0 && G <= kMaxGroup ? kMultiHeads / G : 1;
    return (n_query + qpw - 1) / qpw;
}

hipError_t launch_attention(const AttnParams &p, hipStream_t s) {
    if (p.head_count_kv <= 0 || p.head_count % p.head_count_kv || p.head_count / p.head_count_kv > kMaxGroup ||
        p.max_splits < 1 || !p.counters || !norms_fit(p))
        return hipErrorInvalidValue;
    // pages of kKvPageShift (two 32-position tiles); any window start
    if (!p.page_table || p.page_shift != kKvPageShift || p.window_start < 0 ||
        (!p.position_dev && p.window_start > p.position))
        return hipErrorInvalidValue;
    const int G = p.head_count / p.head_count_kv;
    if (p.n_query > 1) {
        // several queries: plain mode on the matrix-core kernel only
        if (p.k_new || !attention_multi_supported(p.head_dim) || p.position_dev ||
            p.q_stride < p.head_count * p.head_dim || p.out_stride < p.head_count * p.head_dim)
            return hipErrorInvalidValue;
        // the query groups multiply the workgroups: fewer splits each, about
        // the decode grid's size in all (part_o keeps its max_splits layout)
        const int groups = attention_query_groups(p.head_count, p.head_count_kv, p.n_query);
        AttnParams q = p;
        q.max_splits = attention_target_wgs() / (p.head_count_kv * groups);
        q.max_splits = q.max_splits < 1 ? 1 : q.max_splits > p.max_splits ? p.max_splits : q.max_splits;
        const dim3 grid(q.max_splits, p.head_count_kv, groups);
        auto go = [&](auto hd_tag) {
            constexpr int HD = decltype(hd_tag)::value;
            switch (G) {
            case 1: hipLaunchKernelGGL((attn_mfma_kernel<HD, 1, true>), grid, dim3(256), 0, s, q); break;
            case 2: hipLaunchKernelGGL((attn_mfma_kernel<HD, 2, true>), grid, dim3(256), 0, s, q); break;
            case 4: hipLaunchKernelGGL((attn_mfma_kernel<HD, 4, true>), grid, dim3(256), 0, s, q); break;
            case 8: hipLaunchKernelGGL((attn_mfma_kernel<HD, 8, true>), grid, dim3(256), 0, s, q); break;
            default: hipLaunchKernelGGL((attn_mfma_kernel<HD, 0, true>), grid, dim3(256), 0, s, q); break;
            }
        };
        if (p.head_dim == 64) go(std::integral_constant<int, 64>{});
        else if (p.head_dim == 96) go(std::integral_constant<int, 96>{});
        else go(std::integral_constant<int, 128>{});
        return hipGetLastError();
    }
    const dim3 grid(p.max_splits, p.head_count_kv);
    auto go = [&](auto hd_tag) {
        constexpr int HD = decltype(hd_tag)::value;
        if constexpr (HD <= 128) {
            if (!attention_valu() || HD % 64) {
                switch (G) {
                case 1: hipLaunchKernelGGL((attn_mfma_kernel<HD, 1, false>), grid, dim3(256), 0, s, p); break;
                case 2: hipLaunchKernelGGL((attn_mfma_kernel<HD, 2, false>), grid, dim3(256), 0, s, p); break;
                case 4: hipLaunchKernelGGL((attn_mfma_kernel<HD, 4, false>), grid, dim3(256), 0, s, p); break;
                case 8: hipLaunchKernelGGL((attn_mfma_kernel<HD, 8, false>), grid, dim3(256), 0, s, p); break;
                default: hipLaunchKernelGGL((attn_mfma_kernel<HD, 0, false>), grid, dim3(256), 0, s, p); break;
                }
                return;
            }
        }
        if constexpr (HD % 64 == 0) {
            switch (G) {
            case 1: hipLaunchKernelGGL((attn_kernel<HD, 1>), grid, dim3(256), 0, s, p); break;
            case 2: hipLaunchKernelGGL((attn_kernel<HD, 2>), grid, dim3(256), 0, s, p); break;
            case 4: hipLaunchKernelGGL((attn_kernel<HD, 4>), grid, dim3(256), 0, s, p); break;
            case 8: hipLaunchKernelGGL((attn_kernel<HD, 8>), grid, dim3(256), 0, s, p); break;
            default: hipLaunchKernelGGL((attn_kernel<HD, 0>), grid, dim3(256), 0, s, p); break;
            }
        }
    };
    switch (p.head_dim) {
    case 64: go(std::integral_constant<int, 64>{}); break;
    case 96: go(std::integral_constant<int, 96>{}); break;
    case 128: go(std::integral_constant<int, 128>{}); break;
    case 256: go(std::integral_constant<int, 256>{}); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}


// ---- the q/k/v projection and the attention in one launch ----
// Workgroups [0, n_qkv) run the fused RMSNorm + q/k/v matvec (teams of 64,
// device-scope stores), the rest the single-query attention (PQ: K loads
// first, then the head's q/k/v as they land).  Launch bounds of two
// workgroups per CU, so a projection and an attention workgroup share a CU;
// the projection workgroups come first in dispatch order, so no workgroup
// waits for one that is not yet resident.
template <int F1, int F2, int HD, int GG, bool VNOW>
__global__ void __launch_bounds__(256, 2) qkv_attn_kernel(MvParams pq, AttnParams pa, int n_qkv) {
    if ((int)blockIdx.x < n_qkv) {
        __shared__ float lds[36];
        mv_run<F1, F2, IN_NORM, OUT_STORE, 64, 1, MV_PUBLISH>(pq, blockIdx.x, lds, MvFuse{});
    } else {
        const int a = (int)blockIdx.x - n_qkv;
        attn_mfma_body<HD, GG, false, true, VNOW>(pa, a % pa.max_splits, a / pa.max_splits, 0);
    }
}

typedef void (*QkvAttnKernel)(MvParams, AttnParams, int);

// Q4_K q/k with a Q6_K v (a Q4_K_M layer) or Q8_0 throughout; head_dim 128
// with four query heads per kv head, or 64 with eight
template <bool VNOW> static QkvAttnKernel pick_qkv_attn_v(int f1, int f2, int hd, int g) {
    if (hd == 128 && g == 4) {
        if (f1 == Q4_K && f2 == Q6_K) return qkv_attn_kernel<Q4_K, Q6_K, 128, 4, VNOW>;
        if (f1 == Q8_0 && f2 == Q8_0) return qkv_attn_kernel<Q8_0, Q8_0, 128, 4, VNOW>;
    }
    if (hd == 64 && g == 8 && f1 == Q4_K && f2 == Q6_K) return qkv_attn_kernel<Q4_K, Q6_K, 64, 8, VNOW>;
    return nullptr;
}
static QkvAttnKernel pick_qkv_attn(int f1, int f2, int hd, int g, bool v_now = false) {
    return v_now ? pick_qkv_attn_v<true>(f1, f2, hd, g) : pick_qkv_attn_v<false>(f1, f2, hd, g);
}

// Whether the fused launch issues its V tiles right after the q/k/v wait
// (VNOW): from `position` on, each wavefront of a split holds three tiles or
// more (measured: 371 against 367 tok/s at 16k; at 4k, 1-2 tiles, it lost
// 0.8%).  ZIGGY_HIP_ATTN_V_NOW=1 / 0 forces it either way (tests).
bool qkv_attention_v_now(int position, int max_splits) {
    const char *e = getenv("ZIGGY_HIP_ATTN_V_NOW");
    if (e && e[0]) return e[0] == '1';
    // tiles per split at least 9 (every wavefront then holds three or more)
    return (long)(position + 1) >= 9L * 32 * (max_splits > 0 ? max_splits : 1);
}

bool qkv_attention_supported(int f1, int f2, int hidden, int head_dim, int group) {
    return hidden > 0 && hidden % 64 == 0 && hidden <= kMaxMatvecCols && team_width(hidden) == 64 &&
           pick_qkv_attn(f1, f2, head_dim, group) != nullptr;
}

hipError_t launch_qkv_attention(const MvParams &qkv, const AttnParams &a, hipStream_t s, bool v_now) {
    MvParams pq = qkv;
    if (pq.nseg < 1 || pq.nseg > 3 || !pq.norm_w || pq.expert || pq.pro_in || pq.x2) return hipErrorInvalidValue;
    int f1 = pq.seg[0].fmt, f2 = f1;
    for (int i = 1; i < pq.nseg; i++)
        if (pq.seg[i].fmt != f1) f2 = pq.seg[i].fmt;
    for (int i = 0; i < pq.nseg; i++)
        if (pq.seg[i].fmt != f1 && pq.seg[i].fmt != f2) return hipErrorInvalidValue;
    // the attention side: the single-query fused mode with the polled merge
    if (a.head_count_kv <= 0 || a.head_count % a.head_count_kv || a.head_count / a.head_count_kv > kMaxGroup ||
        a.max_splits < 1 || !a.counters || !norms_fit(a) || !a.page_table || a.page_shift != kKvPageShift ||
        a.window_start != 0 || a.n_query > 1 || !a.q || !a.k_new || !a.v_new || !a.out || !a.poll_merge ||
        !a.poll_err || !a.qkv_refill || !a.reset_o || !a.reset_ml ||
        !attention_poll_supported(a.head_dim, a.max_splits))
        return hipErrorInvalidValue;
    const int G = a.head_count / a.head_count_kv;
    const QkvAttnKernel k = qkv_attention_supported(f1, f2, pq.cols, a.head_dim, G)
                                ? pick_qkv_attn(f1, f2, a.head_dim, G, v_now)
                                : nullptr;
    if (!k) return hipErrorInvalidValue;
    plan_matvec(pq, matvec_target_wgs());
    if (pq.team != 64) return hipErrorInvalidValue;
    int n_qkv = 0;
    for (int i = 0; i < pq.nseg; i++) n_qkv += (pq.seg[i].rows + pq.seg[i].rows_per_wg - 1) / pq.seg[i].rows_per_wg;
    pq.route_wg = -1;
    if (n_qkv <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k, dim3(n_qkv + a.max_splits * a.head_count_kv), dim3(256), 0, s, pq, a, n_qkv);
    return hipGetLastError();
}

}  // namespace zh
