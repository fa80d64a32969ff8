// zh_mv.h -- batch-1 dequant-matvec kernel templates for gfx950 (instantiated
// by the zh_mv_*.hip files, one group of formats each, dispatched from
// zh_matvec.hip).
//
// Design (HBM-bound; the point is to keep enough weight bytes in flight):
//   * A row is processed by a "team" of T lanes (T = next power of two of
//     cols/64, at most 256); lane j owns weight slot j (64 weights) of every
//     row the team visits, so its 64 activations are loaded (and normalised /
//     SiLU-gated when fused) once per workgroup and stay in VGPRs.  A team
//     covers the whole input vector, which lets the fused RMSNorm take its
//     sum of squares from the staged slots (one pass over x).
//   * Quant blocks are read in their native GGUF layout with 16-byte loads;
//     scales are unpacked in registers (zh_quant.h).
//   * Weight loads run ring_depth() rows ahead through a ring of register buffers.
//     Every load is unconditional (rows past the team's range re-read its
//     last row), so the compiler's in-order vmcnt waits for the row being
//     consumed only, never for the rows behind it.
//   * Team sums use DPP row operations inside a wavefront (the total lands in
//     the team's last lane); teams wider than a wavefront finish through LDS
//     with one barrier per row (double-buffered slots).
//   * Epilogues: store, residual add, SwiGLU pair (silu(gate) * up from two
//     matrices sharing the staged input), greedy argmax (packed 64-bit
//     atomicMax, ties to the lowest row), expert-weighted add.
//   * Input prologues: plain, fused RMSNorm (rmsNorm order (scale * x) * w as
//     model/loader.zig:3404-3426), fused SiLU(gate) * up (the silu_down path,
//     matvec.metal:2229-2300).

#pragma once

#include "zh_internal.h"
#include "zh_quant.h"
#include "zh_route.h"

namespace zh {

constexpr int kThreads = 256;
// Rows per team in flight (ring of register buffers).  The dense formats hold
// 128 / 256 bytes per lane and row, and SwiGLU rings carry two matrices, so
// their rings are shorter.
#ifndef ZH_RING_QUANT
#define ZH_RING_QUANT 4
#endif
#ifndef ZH_RING_PAIR
#define ZH_RING_PAIR 3
#endif
template <int F, int OUT> constexpr int ring_depth() {
    return F == F32 ? 1 : F == F16 ? 2 : OUT == OUT_SWIGLU ? ZH_RING_PAIR : ZH_RING_QUANT;
}

// v + (v permuted by a DPP control); rows outside ROW_MASK add 0.
template <int CTRL, int ROW_MASK> __device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over aligned groups of T lanes (T a power of two, <= 64) of a wavefront.
// The group total is valid in the group's last lane (in every lane for T <= 16).
__device__ __forceinline__ float group_sum(float v, int T) {
    if (T >= 2) v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    if (T >= 4) v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    if (T >= 8) v = dpp_add<0x141, 0xF>(v);  // row_half_mirror
    if (T >= 16) v = dpp_add<0x140, 0xF>(v); // row_mirror
    if (T >= 32) v = dpp_add<0x142, 0xA>(v); // row_bcast:15 into rows 1 and 3
    if (T >= 64) v = dpp_add<0x143, 0xC>(v); // row_bcast:31 into rows 2 and 3
    return v;
}

// Team sum; valid in the team's last lane.  Teams wider than a wavefront use
// lds[slot*4 .. slot*4+3] and one barrier (callers alternate `slot`).
__device__ __forceinline__ float team_sum(float v, int T, float *lds, int slot) {
    if (T <= 64) return group_sum(v, T);
    v = group_sum(v, 64);
    const int tid = threadIdx.x, wave = tid >> 6;
    if ((tid & 63) == 63) lds[slot * 4 + wave] = v;
    __syncthreads();
    const int per = T >> 6, first = (wave / per) * per;
    float r = 0.f;
    for (int i = 0; i < per; i++) r += lds[slot * 4 + first + i];
    return r;
}

// Batched team sums for the fast paths (T = 64 or 256): four per-lane values
// (rows or gate/up halves) reduce together.  Two DPP transposition steps
// leave each lane one value for value index (lane & 3); row_ror and two
// swizzles finish the sums over the wavefront.  On return every lane holds
// the wavefront total of value (lane & 3).
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float reduce4_wave(float v0, float v1, float v2, float v3) {
    const int l = threadIdx.x;
    const bool b0 = l & 1, b1 = l & 2;
    const float a = (b0 ? v1 : v0) + dpp_mov<0xB1>(b0 ? v0 : v1);  // lane ^ 1
    const float b = (b0 ? v3 : v2) + dpp_mov<0xB1>(b0 ? v2 : v3);
    float c = (b1 ? b : a) + dpp_mov<0x4E>(b1 ? a : b);            // lane ^ 2
    c += dpp_mov<0x124>(c);                                       // row_ror:4
    c += dpp_mov<0x128>(c);                                       // row_ror:8
    c = xsum<16>(c);
    return xsum<32>(c);
}

__device__ __forceinline__ uint32_t ordered_bits(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The raw activations of a lane's slot (and the norm weights or the up half
// for the fused prologues), loaded before the weight ring so that waiting for
// them does not wait for the ring (vmcnt completes in order).
struct XRaw {
    float4 a[16], b[16];
};

template <int F, int IN>
// Unconditional loads (an inactive lane re-reads the last slot and
// stage_finish zeroes its values): a load under a branch makes the register
// allocator copy its destination at the join, and that copy waits for the
// load before the weight loads after it can issue.
__device__ __forceinline__ void stage_load(XRaw &r, int s, bool active, const MvParams &p, const float *x) {
    const int base = Geom<F>::x_base(active ? s : p.slots - 1);
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const int o = base + w * Geom<F>::kXStride;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            r.a[4 * w + c] = *reinterpret_cast<const float4 *>(x + o + 4 * c);
            r.b[4 * w + c] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (IN == IN_NORM) r.b[4 * w + c] = *reinterpret_cast<const float4 *>(p.norm_w + o + 4 * c);
            if (IN == IN_SILU) r.b[4 * w + c] = *reinterpret_cast<const float4 *>(p.x2 + o + 4 * c);
        }
    }
}

// Applies the input prologue to the loaded slot and converts it to the slot
// representation of format F.
template <int F, int IN>
__device__ __forceinline__ void stage_finish(XOf_t<F> &xs, const XRaw &r, const MvParams &p, int T, float *lds,
                                             bool active) {
    float v[64], aux[64];
#pragma unroll
    for (int k = 0; k < 16; k++) {
        v[4 * k] = active ? r.a[k].x : 0.f, v[4 * k + 1] = active ? r.a[k].y : 0.f;
        v[4 * k + 2] = active ? r.a[k].z : 0.f, v[4 * k + 3] = active ? r.a[k].w : 0.f;
        aux[4 * k] = r.b[k].x, aux[4 * k + 1] = r.b[k].y, aux[4 * k + 2] = r.b[k].z, aux[4 * k + 3] = r.b[k].w;
    }
    if (IN == IN_NORM) {
        // the team covers every slot of x, so the team sum of squares is the full one
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 64; i++) ss = fmaf(v[i], v[i], ss);
        ss = team_sum(ss, T, lds, 8);  // lds[32..35]: clear of the row-sum slots
        // every team holds the same total: in lane 63 of each wavefront for
        // T <= 64, in every lane for wider teams
        const float tot = T <= 64 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 63)) : ss;
        const float scale = 1.0f / sqrtf(tot / (float)p.cols + p.eps);
#pragma unroll
        for (int i = 0; i < 64; i++) v[i] = (scale * v[i]) * aux[i];
    } else if (IN == IN_SILU) {
#pragma unroll
        for (int i = 0; i < 64; i++) v[i] = (v[i] / (1.0f + expf(-v[i]))) * aux[i];
    }
    to_slot(v, xs);
}

// Stages the 64 activations of slot s (zeros for inactive lanes) with the
// input prologue applied, in the slot representation of format F.
template <int F, int IN>
__device__ __forceinline__ void stage_x(XOf_t<F> &xs, int s, bool active, const MvParams &p, const float *x, int T,
                                        float *lds) {
    XRaw r;
    stage_load<F, IN>(r, s, active, p, x);
    stage_finish<F, IN>(xs, r, p, T, lds, active);
}

// Matvec bodies inside one fused launch (moe_ffn_kernel): MV_PUBLISH stores
// its outputs with device-scope stores, for workgroups of the same launch;
// MV_POLL finds a routed segment's expert from the router logits itself and
// reads its input as another workgroup of the launch publishes it, over
// words that hold kPollEmpty until then.
enum MvMode : int { MV_PLAIN = 0, MV_PUBLISH = 1, MV_POLL = 2 };
struct MvFuse {
    int *poll_err;   // MV_POLL: set when a wait ran out (the launch's outputs are then not valid)
    float *refill;   // MV_PUBLISH: the route writer refills these words with kPollEmpty
    int refill_n;
};
constexpr long kMvPollSpin = 1L << 18;

__device__ __forceinline__ void store_published(float *y, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>(y), __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// MV_POLL staging of a plain input row (every team of the workgroup reads
// the same row): thread 0 watches the row's last word while the other
// wavefronts wait at the barrier; then the workgroup reads the row once with
// device-scope loads into LDS, again while any word still holds kPollEmpty
// (bounded: on expiry the error flag is set and the values are taken as they
// are), and every lane stages its slot from LDS.  The loads wait for the
// weight ring issued before them (vmcnt completes in order); the input is
// not there sooner anyway.
constexpr int kPollRowMax = 1024;  // values of a polled row (the generic body's rows)
template <int F>
__device__ __forceinline__ void stage_x_polled(XOf_t<F> &xs, int s, bool active, const MvParams &p,
                                               const float *x, int T, float *lds, const MvFuse &fx) {
    __shared__ __align__(16) float xrow[kPollRowMax];
    const int n = p.cols;  // a multiple of 64, at most kPollRowMax (checked by the launcher)
    if (threadIdx.x == 0) {
        const uint32_t *last = reinterpret_cast<const uint32_t *>(x) + (n - 1);
        long spin = 0;
        while (__hip_atomic_load(last, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kPollEmpty && ++spin <= kMvPollSpin)
            __builtin_amdgcn_s_sleep(2);
    }
    __syncthreads();
    const unsigned long long *x8 = reinterpret_cast<const unsigned long long *>(x);
    for (long spin = 0;; spin++) {
        int empty = 0;
        for (int i = threadIdx.x; i < n / 2; i += kThreads) {
            const unsigned long long v = __hip_atomic_load(x8 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
            empty |= lo == kPollEmpty || hi == kPollEmpty;
            xrow[2 * i] = __uint_as_float(lo);
            xrow[2 * i + 1] = __uint_as_float(hi);
        }
        if (!__syncthreads_or(empty)) break;
        if (spin > kMvPollSpin) {
            if (threadIdx.x == 0) __hip_atomic_store(fx.poll_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    stage_x<F, IN_PLAIN>(xs, s, active, p, xrow, T, lds);
}

// Workgroup-cooperative staging for teams of 64 lanes (up to 64 slots; four
// teams per workgroup share one input vector).  Thread t loads run t of x
// (x[16t .. 16t + 15], with the norm weights or the up half of the fused
// prologues) once for the whole workgroup; the workgroup applies the
// prologue and builds every slot's digits in LDS, and each lane then reads
// its own slot's.  The values, digits and run sums are those of
// stage_finish; only the RMSNorm sum of squares is added in another order.
struct XDigLds {
    uint32_t d[3][16];
    float sum[4];
    float scale;
    float pad[3];  // 56 words: 16-byte aligned rows
};
struct CoopLds {
    XDigLds slot[64];
    float run_max[256], run_sum[256];
    float red[4];
};

struct XRun {
    float4 a[4], b[4];
};

// Loads are unconditional (threads past the runs re-read the last run; their
// values are zeroed in coop_finish): a load under a branch makes the
// register allocator copy its destination at the join, and the copy waits
// for the load before anything after it (the weight loads) can issue.
template <int IN>
__device__ __forceinline__ void coop_load(XRun &r, int nruns, const MvParams &p, const float *x) {
    const int t = min((int)threadIdx.x, nruns - 1);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        r.a[c] = *reinterpret_cast<const float4 *>(x + 16 * t + 4 * c);
        r.b[c] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (IN == IN_NORM) r.b[c] = *reinterpret_cast<const float4 *>(p.norm_w + 16 * t + 4 * c);
        if (IN == IN_SILU) r.b[c] = *reinterpret_cast<const float4 *>(p.x2 + 16 * t + 4 * c);
    }
}

template <int F, int IN>
__device__ __forceinline__ void coop_finish(XDig &xs, const XRun &r, int nruns, int slots, int lane,
                                            const MvParams &p) {
    __shared__ CoopLds L;
    const int t = threadIdx.x, wave = t >> 6;
    const bool own = t < nruns;  // threads past the runs hold a re-read run: zeros
    float v[16], aux[16];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        v[4 * c] = own ? r.a[c].x : 0.f, v[4 * c + 1] = own ? r.a[c].y : 0.f;
        v[4 * c + 2] = own ? r.a[c].z : 0.f, v[4 * c + 3] = own ? r.a[c].w : 0.f;
        aux[4 * c] = r.b[c].x, aux[4 * c + 1] = r.b[c].y, aux[4 * c + 2] = r.b[c].z, aux[4 * c + 3] = r.b[c].w;
    }
    if (IN == IN_NORM) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) ss = fmaf(v[i], v[i], ss);
        ss = group_sum(ss, 64);  // wavefront total in lane 63
        if ((t & 63) == 63) L.red[wave] = ss;
        __syncthreads();
        const float tot = (L.red[0] + L.red[1]) + (L.red[2] + L.red[3]);
        const float scale = 1.0f / sqrtf(tot / (float)p.cols + p.eps);
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = (scale * v[i]) * aux[i];
    } else if (IN == IN_SILU) {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = (v[i] / (1.0f + expf(-v[i]))) * aux[i];
    }
    float m = 0.f, rs = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        m = fmaxf(m, fabsf(v[i]));
        rs += v[i];
    }
    L.run_max[t] = m;
    L.run_sum[t] = rs;
    __syncthreads();
    if (t < nruns) {
        int s, w;
        Geom<F>::run_slot(t, s, w);
        // the slot's four runs: x_base(s) + w' * stride
        const int r0 = Geom<F>::x_base(s) / 16, rstep = Geom<F>::kXStride / 16;
        const float sm = fmaxf(fmaxf(L.run_max[r0], L.run_max[r0 + rstep]),
                               fmaxf(L.run_max[r0 + 2 * rstep], L.run_max[r0 + 3 * rstep]));
        const float tot = (L.run_sum[r0] + L.run_sum[r0 + rstep]) + (L.run_sum[r0 + 2 * rstep] + L.run_sum[r0 + 3 * rstep]);
        const int k = slot_exponent(sm);
        XDigLds &o = L.slot[s];
#pragma unroll
        for (int c = 0; c < 4; c++)
            digits4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3], k, o.d[0][4 * w + c], o.d[1][4 * w + c],
                    o.d[2][4 * w + c]);
        o.sum[w] = rs;
        if (w == 0) o.scale = slot_scale(sm, tot, k);
    }
    __syncthreads();
    const XDigLds &me = L.slot[lane < slots ? lane : slots - 1];
#pragma unroll
    for (int j = 0; j < 3; j++)
#pragma unroll
        for (int c = 0; c < 16; c++) xs.d[j][c] = me.d[j][c];
#pragma unroll
    for (int w = 0; w < 4; w++) xs.sum[w] = me.sum[w];
    xs.scale = me.scale;
}

// The fused combine of the previous MoE layer (MvParams::pro_in, NORM): CPT
// float4 chunks of the row per thread, every load (hidden, the k routed rows,
// the shared row, the route's weights) in flight before any arithmetic
// (combine_load), then combine_value's operations in its order per element
// (combine_finish); the row goes to LDS (and from the writer workgroup to
// pro_out).  Loads past the row re-read its last chunk.
template <int CPT> struct CombineIn {
    float4 hv[CPT], tv[CPT][kRouteMaxK], sv[CPT];
    float w[kRouteMaxK], g;
};
template <int CPT> __device__ __forceinline__ void combine_load(CombineIn<CPT> &ci, const MvParams &p) {
    const int H = p.cols, k = (int)(p.pro_cfg & 0xF);
#pragma unroll
    for (int c = 0; c < CPT; c++) {
        const int i4 = min((int)threadIdx.x + c * kThreads, H / 4 - 1);
        ci.hv[c] = *reinterpret_cast<const float4 *>(p.x + 4 * i4);
#pragma unroll
        for (int s = 0; s < kRouteMaxK; s++)
            ci.tv[c][s] = *reinterpret_cast<const float4 *>(p.pro_in + (size_t)min(s, k - 1) * H + 4 * i4);
        ci.sv[c] = *reinterpret_cast<const float4 *>(p.pro_in + (size_t)k * H + 4 * i4);
    }
#pragma unroll
    for (int s = 0; s < kRouteMaxK; s++) ci.w[s] = __uint_as_float(p.expert[2 * min(s, k - 1) + 1]);
    ci.g = __uint_as_float(p.expert[2 * k]);
}
template <int CPT>
__device__ __forceinline__ void combine_finish(const CombineIn<CPT> &ci, const MvParams &p, float *xc, bool writer) {
    const int H = p.cols, k = (int)(p.pro_cfg & 0xF);
    const bool shared = p.pro_cfg >> 4 & 1;
    float *out = static_cast<float *>(p.pro_out);
#pragma unroll
    for (int c = 0; c < CPT; c++) {
        const int i4 = (int)threadIdx.x + c * kThreads;
        if (i4 >= H / 4) continue;
        const float hs[4] = {ci.hv[c].x, ci.hv[c].y, ci.hv[c].z, ci.hv[c].w};
        const float ss[4] = {ci.sv[c].x, ci.sv[c].y, ci.sv[c].z, ci.sv[c].w};
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            // combine_value (zh_route.h), operation for operation
            float o = 0.f;
#pragma unroll
            for (int s = 0; s < kRouteMaxK; s++) {
                if (s >= k) break;
                const float4 &t = ci.tv[c][s];
                const float d = e == 0 ? t.x : e == 1 ? t.y : e == 2 ? t.z : t.w;
                o = ci.w[s] == 1.0f ? o + d : fmaf(d, ci.w[s], o);
            }
            if (shared) o = ci.g == 1.0f ? o + ss[e] : fmaf(ss[e], ci.g, o);
            r[e] = hs[e] + o;
        }
        const float4 v = make_float4(r[0], r[1], r[2], r[3]);
        *reinterpret_cast<float4 *>(xc + 4 * i4) = v;
        if (writer) *reinterpret_cast<float4 *>(out + 4 * i4) = v;
    }
}
// The whole combine before the product (rows of more than 2048 values).
template <int CPT>
__device__ __forceinline__ void combine_prologue(const MvParams &p, float *xc, bool writer) {
    CombineIn<CPT> ci;
    combine_load<CPT>(ci, p);
    combine_finish<CPT>(ci, p, xc, writer);
}

template <int F, int IN, int OUT, int MODE = MV_PLAIN>
__device__ __forceinline__ void mv_body(const MvParams &p, const MvSeg &sg, int wg_in_seg, float *lds,
                                        const MvFuse &fx = MvFuse{}) {
    static_assert(MODE != MV_POLL || IN == IN_PLAIN, "polled inputs are plain rows");
    constexpr int D = ring_depth<F, OUT>();
    const int tid = threadIdx.x, T = p.team, teams = kThreads / T;
    const int team = tid / T, lane = tid % T;
    const bool active = lane < p.slots;
    const int sl = active ? lane : p.slots - 1;  // inactive lanes re-read a valid slot
    const bool writer = lane == T - 1;

    const uint8_t *wbase = sg.w, *wbase2 = sg.w2;
    float wscale = p.weight_scale;
    if (p.expert && sg.expert_slot >= 0) {
        const uint32_t e = p.expert[2 * sg.expert_slot];
        if (e >= (uint32_t)p.expert_limit) return;  // uniform over the segment: no rows are read
        const uint64_t off = (uint64_t)e * (uint64_t)p.rows_per_expert * sg.stride;
        wbase += off;
        if (wbase2) wbase2 += off;
        wscale = __uint_as_float(p.expert[2 * sg.expert_slot + 1]);
    }
    const int r_begin = wg_in_seg * sg.rows_per_wg;
    const int r_end = min(r_begin + sg.rows_per_wg, sg.rows);
    const int n = sg.rows_per_wg / teams;  // rows per team of this segment
    const int r0 = r_begin + team;
    // row `it` of this team, clamped to the workgroup's last row (loads only)
    auto row_of = [&](int it) { return min(r0 + it * teams, r_end - 1); };

    // Issue the first rows' weight loads before staging the input: they do not
    // depend on it, so HBM latency overlaps the staging and the norm.
    // The residual read of ADD / WADD rides in the same ring: a late load of
    // y[r] would make the in-order vmcnt wait cover the prefetched rows too.
    // kComb (the router launch with the previous layer's combine fused, rows
    // up to 2048 values): the combine's loads go first, then the ring, so the
    // combine waits only for its own loads and the ring streams meanwhile.
    constexpr bool kComb = IN == IN_NORM && OUT == OUT_STORE && F == F32;
    const bool comb = kComb && p.pro_in && p.cols <= kCombineFastCols;
    __shared__ __align__(16) float xcomb[kComb ? kCombineFastCols : 4];
    CombineIn<kComb ? 2 : 1> ci;
    if constexpr (kComb) {
        if (comb) combine_load<2>(ci, p);
        __builtin_amdgcn_sched_barrier(0);  // the combine's loads stay ahead of the ring's
    }
    constexpr bool kReadY = OUT == OUT_ADD || OUT == OUT_WADD;
    Raw<F> ra[D], rb[D];
    float ry[D];
#pragma unroll
    for (int k = 0; k < D; k++) {
        ra[k] = slot_load<F>(wbase + (uint64_t)row_of(k) * sg.stride, sl);
        if (OUT == OUT_SWIGLU) rb[k] = slot_load<F>(wbase2 + (uint64_t)row_of(k) * sg.stride, sl);
        if (kReadY) ry[k] = sg.y[row_of(k)];
    }
    XOf_t<F> xs;
    bool staged = false;
    if constexpr (kComb) {
        if (comb) {
            // the row from LDS (LDS reads: their wait does not cover the ring)
            combine_finish<2>(ci, p, xcomb, blockIdx.x == 0);
            __syncthreads();
            stage_x<F, IN>(xs, lane, active, p, xcomb, T, lds);
            staged = true;
        }
    }
    if constexpr (MODE == MV_POLL) {
        stage_x_polled<F>(xs, lane, active, p, sg.x ? sg.x : p.x, T, lds, fx);
    } else {
        if (!staged) stage_x<F, IN>(xs, lane, active, p, sg.x ? sg.x : p.x, T, lds);
    }

    float best_v = -INFINITY;
    int best_r = 0x7fffffff;
    for (int it0 = 0; it0 < n; it0 += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            const int it = it0 + k;
            if (it < n) {
                float v = slot_dot<F>(ra[k], sl, xs), v2 = 0.f;
                if (OUT == OUT_SWIGLU) v2 = slot_dot<F>(rb[k], sl, xs);
                v = active ? v : 0.f;
                v = team_sum(v, T, lds, it & 1);
                if (OUT == OUT_SWIGLU) {
                    v2 = active ? v2 : 0.f;
                    v2 = team_sum(v2, T, lds, 2 + (it & 1));
                }
                const int r = r0 + it * teams;
                if (writer && r < r_end) {
                    if (OUT == OUT_STORE) {
                        sg.y[r] = v;
                    } else if (OUT == OUT_ADD) {
                        sg.y[r] = ry[k] + v;
                    } else if (OUT == OUT_WADD) {
                        sg.y[r] = fmaf(v, wscale, ry[k]);
                    } else if (OUT == OUT_SWIGLU) {
                        const float a = (v / (1.0f + expf(-v))) * v2;  // siluInPlace then gate * up
                        if constexpr (MODE == MV_PUBLISH) store_published(&sg.y[r], a);
                        else sg.y[r] = a;
                    } else if (OUT == OUT_ARGMAX) {
                        if (sg.y) sg.y[r] = v;
                        if (v > best_v || (v == best_v && r < best_r)) {
                            best_v = v;
                            best_r = r;
                        }
                    }
                }
            }
            // refill this ring slot (unconditionally: keeps the vmcnt waits exact)
            ra[k] = slot_load<F>(wbase + (uint64_t)row_of(it + D) * sg.stride, sl);
            if (OUT == OUT_SWIGLU) rb[k] = slot_load<F>(wbase2 + (uint64_t)row_of(it + D) * sg.stride, sl);
            if (kReadY) ry[k] = sg.y[row_of(it + D)];
        }
    }
    if (OUT == OUT_ARGMAX) {
        __shared__ unsigned long long keys[kThreads];
        unsigned long long key = 0ull;
        if (writer && best_r != 0x7fffffff)
            key = ((unsigned long long)ordered_bits(best_v) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)best_r);
        if (writer) keys[team] = key;
        __syncthreads();
        if (tid == 0) {
            unsigned long long k = keys[0];
            for (int i = 1; i < teams; i++) k = keys[i] > k ? keys[i] : k;
            if (k) atomicMax(p.argmax_slot, k);
        }
    }
}

// Fast path for teams of TT = 64 lanes (one team per wavefront) or 256 lanes
// (one team per workgroup).  Values are consumed in batches of four (four
// rows, or two gate/up row pairs for SwiGLU) that reduce together.  The ring
// holds NB batches: each slot is refilled as soon as its dot is done, so NB
// batches of weight loads stay in flight.  Residuals of ADD / WADD (at most
// kMaxYB batches per team) are all loaded before the ring, so waiting for
// them never waits for weight loads (vmcnt completes in order).
constexpr int kMaxYB = 8;
template <int F, int IN, int OUT, int TT, int NB, int MODE = MV_PLAIN>
__device__ __forceinline__ void mv_body_fast(const MvParams &p, const MvSeg &sg, int wg_in_seg, float *lds) {
    static_assert(MODE != MV_POLL, "polled inputs take the generic body");
    constexpr bool kPair = OUT == OUT_SWIGLU;
    constexpr int B = kPair ? 2 : 4;  // ring slots per batch: rows (or gate/up row pairs)
    constexpr int D = NB * B;         // ring slots
    constexpr int teams = kThreads / TT;
    constexpr bool kReadY = OUT == OUT_ADD || OUT == OUT_WADD;
    const int tid = threadIdx.x, lane = tid % TT, wave = tid >> 6, l4 = tid & 3;
    const int team = __builtin_amdgcn_readfirstlane(tid / TT);
    const bool active = lane < p.slots;
    const int sl = active ? lane : p.slots - 1;  // inactive lanes re-read a valid slot

    const uint8_t *wbase = sg.w, *wbase2 = sg.w2;
    float wscale = p.weight_scale;
    if (p.expert && sg.expert_slot >= 0) {
        const uint32_t e = p.expert[2 * sg.expert_slot];
        if (e >= (uint32_t)p.expert_limit) return;  // uniform over the segment: no rows are read
        const uint64_t off = (uint64_t)e * (uint64_t)p.rows_per_expert * sg.stride;
        wbase += off;
        if (wbase2) wbase2 += off;
        wscale = __uint_as_float(p.expert[2 * sg.expert_slot + 1]);
    }
    const int r_begin = wg_in_seg * sg.rows_per_wg;
    const int r_end = min(r_begin + sg.rows_per_wg, sg.rows);
    const int n = sg.rows_per_wg / teams;  // rows per team of this segment
    const int r0 = r_begin + team;
    auto row_of = [&](int it) { return min(r0 + it * teams, r_end - 1); };

    // TT = 64: workgroup-cooperative staging (all slots in LDS); TT = 256: each
    // lane stages its own slot (one team per workgroup, nothing is shared)
    constexpr bool kCoop = TT == 64;
    const int nruns = p.slots * 4;
    XRaw xr;
    XRun xrun;
    const float *xin = sg.x ? sg.x : p.x;
    if constexpr (kCoop)
        coop_load<IN>(xrun, nruns, p, xin);
    else
        stage_load<F, IN>(xr, lane, active, p, xin);
    // residual of row (4b + l4) of the team for batch b (lane l serves value l & 3)
    float ry[kReadY ? kMaxYB : 1];
    if (kReadY) {
#pragma unroll
        for (int b = 0; b < kMaxYB; b++) ry[b] = 4 * b < n ? sg.y[row_of(4 * b + l4)] : 0.f;
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the x and residual loads ahead of the ring loads
    Raw<F> ra[D], rb[D];
#pragma unroll
    for (int k = 0; k < D; k++) {
        ra[k] = slot_load<F>(wbase + (uint64_t)row_of(k) * sg.stride, sl);
        if (kPair) rb[k] = slot_load<F>(wbase2 + (uint64_t)row_of(k) * sg.stride, sl);
        // slot by slot, in the order the loop refills them: the loop's waits
        // must hold for both issue orders, so a slot whose loads the scheduler
        // moved behind later slots would wait for those too on every pass
        __builtin_amdgcn_sched_barrier(0);
    }
    XOf_t<F> xs;
    if constexpr (kCoop)
        coop_finish<F, IN>(xs, xrun, nruns, p.slots, lane, p);
    else
        stage_finish<F, IN>(xs, xr, p, TT, lds, active);

    float best_v = -INFINITY;
    int best_r = 0x7fffffff;
    int batch = 0;  // running batch count (LDS slot parity for TT = 256)
    for (int it0 = 0; it0 < n; it0 += D) {
#pragma unroll
        for (int bt = 0; bt < NB; bt++, batch++) {
            const int ib = it0 + bt * B;  // first row index of the batch
            float v[4];
#pragma unroll
            for (int j = 0; j < B; j++) {
                const int k = bt * B + j;
                // unconditional (rows past the team's range hold a valid
                // re-read row and are dropped by the epilogue): a dot under a
                // branch lets the register allocator move the ring, and the
                // copies would wait for the loads in flight
                const float a = slot_dot<F>(ra[k], sl, xs);
                const float b = kPair ? slot_dot<F>(rb[k], sl, xs) : 0.f;
                if (kPair) {
                    v[2 * j] = active ? a : 0.f;
                    v[2 * j + 1] = active ? b : 0.f;
                } else {
                    v[j] = active ? a : 0.f;
                }
                // Refill this ring slot (unconditionally: keeps the vmcnt waits
                // exact).  The scheduling barrier keeps the loads after the dot
                // that reads the slot, so the ring stays in place across iterations.
                __builtin_amdgcn_sched_barrier(0);
                ra[k] = slot_load<F>(wbase + (uint64_t)row_of(ib + j + D) * sg.stride, sl);
                if (kPair) rb[k] = slot_load<F>(wbase2 + (uint64_t)row_of(ib + j + D) * sg.stride, sl);
            }
            float c = reduce4_wave(v[0], v[1], v[2], v[3]);
            if (TT == 256) {
                // one team per workgroup: combine the four wavefront totals
                const int slot = batch & 1;
                if ((tid & 63) < 4) lds[slot * 16 + wave * 4 + l4] = c;
                __syncthreads();
                c = (lds[slot * 16 + l4] + lds[slot * 16 + 4 + l4]) + (lds[slot * 16 + 8 + l4] + lds[slot * 16 + 12 + l4]);
            }
            // value (lane & 3) of the batch: row ib + l4 (single) or half l4 & 1 of row ib + l4 / 2 (pair)
            if (kPair) {
                const float up = dpp_mov<0xF5>(c);  // quad_perm [1,1,3,3]: the up half next to its gate
                const int k = l4 >> 1;
                const int r = r0 + (ib + k) * teams;
                if (lane < 4 && !(l4 & 1) && ib + k < n && r < r_end) {
                    const float a = (c / (1.0f + expf(-c))) * up;
                    if constexpr (MODE == MV_PUBLISH) store_published(&sg.y[r], a);
                    else sg.y[r] = a;
                }
            } else {
                const int r = r0 + (ib + l4) * teams;
                if (lane < 4 && ib + l4 < n && r < r_end) {
                    if (OUT == OUT_STORE) {
                        if constexpr (MODE == MV_PUBLISH) store_published(&sg.y[r], c);
                        else sg.y[r] = c;
                    } else if (OUT == OUT_ADD) {
                        sg.y[r] = ry[0] + c;
                    } else if (OUT == OUT_WADD) {
                        sg.y[r] = fmaf(c, wscale, ry[0]);
                    } else if (OUT == OUT_ARGMAX) {
                        if (sg.y) sg.y[r] = c;
                        if (c > best_v || (c == best_v && r < best_r)) {
                            best_v = c;
                            best_r = r;
                        }
                    }
                }
                if (kReadY) {
#pragma unroll
                    for (int b = 0; b + 1 < kMaxYB; b++) ry[b] = ry[b + 1];
                }
            }
        }
    }
    if (OUT == OUT_ARGMAX) {
        __shared__ unsigned long long keys[16];
        unsigned long long key = 0ull;
        if (best_r != 0x7fffffff)
            key = ((unsigned long long)ordered_bits(best_v) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)best_r);
        if ((tid & 63) < 4) keys[wave * 4 + l4] = TT == 64 || wave == 0 ? key : 0ull;
        __syncthreads();
        if (tid == 0) {
            unsigned long long k = 0ull;
            for (int i = 0; i < 16; i++) k = keys[i] > k ? keys[i] : k;
            if (k) atomicMax(p.argmax_slot, k);
        }
    }
}

template <int F, int IN, int OUT, int TT, int NB, int MODE = MV_PLAIN>
__device__ __forceinline__ void mv_dispatch(const MvParams &p, const MvSeg &sg, int wg_in_seg, float *lds,
                                            const MvFuse &fx) {
    if constexpr (TT != 0)
        mv_body_fast<F, IN, OUT, TT, NB, MODE>(p, sg, wg_in_seg, lds);
    else
        mv_body<F, IN, OUT, MODE>(p, sg, wg_in_seg, lds, fx);
}

// TT: compile-time team width (64 or 256) of the fast path, 0 for any width;
// NB: batches of four values in the fast path's load ring.  wg: the
// workgroup's index in this matvec's grid.
template <int F1, int F2, int IN, int OUT, int TT, int NB, int MODE = MV_PLAIN>
__device__ __forceinline__ void mv_run(const MvParams &p, int wg, float *lds, const MvFuse &fx) {
    touch_params(p);  // the segment search, the segment's fields, the inputs' addresses
    // only the output head is gated (prompt steps skip it): the other
    // kernels do not wait for the flag's loads before issuing their own
    if (OUT == OUT_ARGMAX && p.gate_flag && *p.gate_flag == 0) return;
    int si = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeg; i++)
        if (i < p.nseg && wg >= p.seg[i].wg_begin) si = i;
    // a copy: every field of the segment is read in one batch of scalar
    // loads, not one dependent round trip per use
    MvSeg sg = p.seg[si];
    if constexpr (OUT == OUT_SWIGLU || MODE == MV_POLL) {
        if (p.pro_in) {  // uniform over the workgroup
            const uint32_t c = p.pro_cfg;
            const int E = (int)(c & 0xFFFF), gating = (int)(c >> 20 & 0xF);
            if (OUT == OUT_SWIGLU && wg == p.route_wg) {
                // the route writer (a workgroup of its own, no rows): the
                // whole route, weights and shared gate included, to pro_out
                if (threadIdx.x < 64) {
                    uint32_t *out = static_cast<uint32_t *>(p.pro_out);
                    route_wave(p.pro_in, E, (int)(c >> 16 & 0xF), gating, (int)(c >> 24 & 1), p.pro_scale,
                               (int)(c >> 25 & 1), [&](int i, uint32_t v) { out[i] = v; });
                }
                if constexpr (MODE == MV_PUBLISH) {
                    // the other set of published words, for the next launch (its
                    // start orders these stores before its loads)
                    for (int i = threadIdx.x; i < fx.refill_n; i += kThreads) fx.refill[i] = __uint_as_float(kPollEmpty);
                }
                return;
            }
            if (sg.expert_slot >= 0) {
                // every wavefront finds this segment's expert itself: the
                // softmax and the top-k up to its slot (no barrier, no weights)
                const uint32_t e = route_id(p.pro_in, E, gating, sg.expert_slot);
                if (e >= (uint32_t)p.expert_limit) return;  // uniform over the segment: no rows are read
                const uint64_t off = (uint64_t)e * (uint64_t)p.rows_per_expert * sg.stride;
                sg.w += off;
                if (sg.w2) sg.w2 += off;
                sg.expert_slot = -1;
            }
        }
    }
    if constexpr (IN == IN_NORM && OUT == OUT_STORE && F1 == F32 && F2 == F32) {
        // the previous MoE layer's combine, then the norm as usual: rows up
        // to kCombineFastCols inside the product (its loads ahead of the
        // weights'), wider rows here
        if (p.pro_in && p.cols > kCombineFastCols) {
            __shared__ __align__(16) float xc[kCombineMaxCols];
            combine_prologue<kCombineMaxCols / (4 * kThreads)>(p, xc, wg == 0);
            __syncthreads();
            sg.x = xc;
        }
    }
    if (F1 == F2 || sg.fmt == F1)
        mv_dispatch<F1, IN, OUT, TT, NB, MODE>(p, sg, wg - sg.wg_begin, lds, fx);
    else
        mv_dispatch<F2, IN, OUT, TT, NB, MODE>(p, sg, wg - sg.wg_begin, lds, fx);
}

template <int F1, int F2, int IN, int OUT, int TT, int NB>
__global__ void __launch_bounds__(kThreads) mv_kernel(MvParams p) {
    __shared__ float lds[36];
    mv_run<F1, F2, IN, OUT, TT, NB>(p, blockIdx.x, lds, MvFuse{});
}

// An MoE layer's routed and shared expert FFNs in one launch: workgroups
// [0, n_gu) run the gate/up product (fused RMSNorm, routing, SwiGLU;
// MV_PUBLISH: its act rows with device-scope stores), the rest the down
// products (MV_POLL: each routed wavefront finds its expert, issues its
// weight loads, then reads its act row as the gate/up workgroups publish
// it).  The gate/up workgroups come first in dispatch order, so no
// workgroup waits for one that is not yet resident.
template <int F1, int F2, int TTG>
__global__ void __launch_bounds__(kThreads) moe_ffn_kernel(MvParams pg, MvParams pd, int n_gu, MvFuse fx) {
    __shared__ float lds[36];
    if ((int)blockIdx.x < n_gu)
        mv_run<F1, F2, IN_NORM, OUT_SWIGLU, TTG, 1, MV_PUBLISH>(pg, blockIdx.x, lds, fx);
    else
        mv_run<F1, F2, IN_PLAIN, OUT_STORE, 0, 1, MV_POLL>(pd, (int)blockIdx.x - n_gu, lds, fx);
}

// Team width of a row of `cols` values: next power of two of the slot count,
// at most one workgroup.
// Rows of 1024 .. 4032 values take a whole wavefront (16 .. 63 active lanes):
// the fast path serves teams of 64 and 256 lanes only.
inline int team_width(int cols) {
    int t = 1;
    while (t < cols / 64) t <<= 1;
    if (cols >= 1024 && t < 64) t = 64;
    return t > kThreads ? kThreads : t;
}

typedef void (*MvKernel)(MvParams);

template <int F1, int F2, int TT, int NB> MvKernel pick_io(int in, int out) {
    if (in == IN_PLAIN && out == OUT_STORE) return mv_kernel<F1, F2, IN_PLAIN, OUT_STORE, TT, NB>;
    if (in == IN_PLAIN && out == OUT_ADD) return mv_kernel<F1, F2, IN_PLAIN, OUT_ADD, TT, NB>;
    if (in == IN_NORM && out == OUT_STORE) return mv_kernel<F1, F2, IN_NORM, OUT_STORE, TT, NB>;
    if (in == IN_NORM && out == OUT_SWIGLU) return mv_kernel<F1, F2, IN_NORM, OUT_SWIGLU, TT, NB>;
    if (in == IN_PLAIN && out == OUT_SWIGLU) return mv_kernel<F1, F2, IN_PLAIN, OUT_SWIGLU, TT, NB>;
    if (in == IN_PLAIN && out == OUT_ARGMAX) return mv_kernel<F1, F2, IN_PLAIN, OUT_ARGMAX, TT, NB>;
    if (in == IN_NORM && out == OUT_ARGMAX) return mv_kernel<F1, F2, IN_NORM, OUT_ARGMAX, TT, NB>;
    if (in == IN_SILU && out == OUT_ADD) return mv_kernel<F1, F2, IN_SILU, OUT_ADD, TT, NB>;
    if (in == IN_PLAIN && out == OUT_WADD) return mv_kernel<F1, F2, IN_PLAIN, OUT_WADD, TT, NB>;
    return nullptr;
}

// Ring batches of the fast path; ZIGGY_HIP_MATVEC_NB forces 1, 2 or 3 (a tuning knob).
int forced_nb();

// The fast path serves teams of 64 or 256 lanes, with at most kMaxYB residual
// batches per team for ADD / WADD; its ring holds enough batches for all of a
// team's rows, up to two (three when forced).
template <int F1, int F2, bool kFast> MvKernel pick(int in, int out, int cols, int rows_per_team) {
    if constexpr (kFast) {
        const int T = team_width(cols);
        const bool read_y = out == OUT_ADD || out == OUT_WADD;
        if ((T == 64 || T == 256) && !(read_y && rows_per_team > 4 * kMaxYB)) {
            const int per_batch = out == OUT_SWIGLU ? 2 : 4;
            // one batch in flight measured fastest on MI355X for every decode
            // shape (deeper rings slowed q/k/v, o_proj, gate/up and down)
            int nb = forced_nb();
            if (!nb) nb = 1;
            (void)per_batch;
            if (T == 64)
                return nb == 1 ? pick_io<F1, F2, 64, 1>(in, out)
                               : nb == 2 ? pick_io<F1, F2, 64, 2>(in, out) : pick_io<F1, F2, 64, 3>(in, out);
            return nb == 1 ? pick_io<F1, F2, 256, 1>(in, out)
                           : nb == 2 ? pick_io<F1, F2, 256, 2>(in, out) : pick_io<F1, F2, 256, 3>(in, out);
        }
    }
    return pick_io<F1, F2, 0, 1>(in, out);
}

// The q/k/v launch of a Q4_K_M layer mixes Q4_K and Q6_K segments (fused
// RMSNorm, plain store); only that combination is instantiated.
template <int F1, int F2> MvKernel pick_mixed(int cols, int rows_per_team) {
    const int T = team_width(cols);
    int nb = forced_nb();
    if (!nb) nb = 1;
    if (T == 64)
        return nb == 1 ? mv_kernel<F1, F2, IN_NORM, OUT_STORE, 64, 1>
                       : nb == 2 ? mv_kernel<F1, F2, IN_NORM, OUT_STORE, 64, 2> : mv_kernel<F1, F2, IN_NORM, OUT_STORE, 64, 3>;
    if (T == 256)
        return nb == 1 ? mv_kernel<F1, F2, IN_NORM, OUT_STORE, 256, 1>
                       : nb == 2 ? mv_kernel<F1, F2, IN_NORM, OUT_STORE, 256, 2> : mv_kernel<F1, F2, IN_NORM, OUT_STORE, 256, 3>;
    return mv_kernel<F1, F2, IN_NORM, OUT_STORE, 0, 1>;
}

// Two formats in one launch for a fixed prologue / epilogue (the q/k/v launch
// of a Q4_K_M layer; the routed + shared experts of an MoE layer).
template <int F1, int F2, int IN, int OUT> MvKernel pick_two(int cols) {
    const int T = team_width(cols);
    if (T == 64) return mv_kernel<F1, F2, IN, OUT, 64, 1>;
    if (T == 256) return mv_kernel<F1, F2, IN, OUT, 256, 1>;
    return mv_kernel<F1, F2, IN, OUT, 0, 1>;
}

// Kernel pickers, one per group of formats (zh_mv_*.hip).
MvKernel pick_mv_q4k(int in, int out, int cols, int rows_per_team);
MvKernel pick_mv_q6k(int in, int out, int cols, int rows_per_team);
MvKernel pick_mv_q8_0(int in, int out, int cols, int rows_per_team);
MvKernel pick_mv_other(int fmt, int in, int out, int cols, int rows_per_team);
MvKernel pick_mv_mixed(int f1, int f2, int cols, int rows_per_team);
MvKernel pick_mv_moe(int f1, int f2, int in, int out, int cols);
typedef void (*MoeFfnKernel)(MvParams, MvParams, int, MvFuse);
MoeFfnKernel pick_moe_ffn(int f1, int f2, int gate_cols, int down_cols);

}  // namespace zh
