// zh_route.h -- the routing of one token's MoE layer by one wavefront (up to
// 256 experts, four per lane): softmax over all experts (expert_gating_func
// 1, 2; softmaxInPlace, model/loader.zig:4160-4170), top-k with ties to the
// lower index (selectTopK, :3953-3975), normalizePositiveWeights
// (:3977-3990) when expert_weights_norm, x expert_weights_scale, and the
// sigmoid of the shared expert's gate logit (sigmoidScalar, :4022-4029).
// Lane 0 hands out the route through put(i, value): entries i = 2 r (expert
// id) and 2 r + 1 (weight bits) for r < k, then i = 2 k (shared scale bits).
// Used by the routing kernel and by the MoE gate/up matvec's prologue, so
// both compute the same bits.
#pragma once

#include "zh_internal.h"

namespace zh {

constexpr int kRouteMaxK = 8;           // experts per token at most
constexpr int kRouteWaveExperts = 256;  // experts one wavefront routes

__device__ __forceinline__ uint32_t route_ordered_bits(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The wavefront sum of `for (o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o)`,
// operand for operand, without LDS-path bpermutes: lane swaps for 32 and 16,
// row_ror:8 for 8, row_shl:4 / row_shr:4 by lane for 4, quad permutations
// for 2 and 1 (each step adds the partner lane's value, as the shuffle does).
__device__ __forceinline__ float wave_sum_xor(float v) {
    auto mov = [](float x, auto ctrl) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, false));
    };
    v = xsum<32>(v);
    v = xsum<16>(v);
    v += mov(v, std::integral_constant<int, 0x128>{});  // row_ror:8 = lane ^ 8
    const float up = mov(v, std::integral_constant<int, 0x104>{}), dn = mov(v, std::integral_constant<int, 0x114>{});
    v += (threadIdx.x & 4) ? dn : up;                   // row_shr:4 / row_shl:4 = lane ^ 4
    v += mov(v, std::integral_constant<int, 0x4E>{});   // lane ^ 2
    v += mov(v, std::integral_constant<int, 0xB1>{});   // lane ^ 1
    return v;
}

// The wavefront maximum of a 32-bit unsigned value, valid in every lane: DPP
// within each 16-lane row, then the two lane swaps across rows (as
// wave_max_key does for 64 bits).  Every lane must be active.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    auto mov = [](uint32_t x, auto ctrl) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, decltype(ctrl)::value, 0xF, 0xF, false);
    };
    v = max(v, mov(v, std::integral_constant<int, 0xB1>{}));
    v = max(v, mov(v, std::integral_constant<int, 0x4E>{}));
    v = max(v, mov(v, std::integral_constant<int, 0x141>{}));
    v = max(v, mov(v, std::integral_constant<int, 0x140>{}));
    uint32_t a, b;
    lane_pair<16>(v, a, b);
    v = max(a, b);
    lane_pair<32>(v, a, b);
    return max(a, b);
}

// The softmax (gating 1, 2) of the E router logits, four entries per lane
// (entry l + 64 i in pr[i]; -INFINITY past E).
__device__ __forceinline__ void route_probs(const float *__restrict__ logits, int E, int gating, float (&pr)[4]) {
    const int l = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 4; i++) pr[i] = l + 64 * i < E ? logits[l + 64 * i] : -INFINITY;
    if (gating == 1 || gating == 2) {
        // softmaxInPlace (model/loader.zig:4160-4170): max, exp(v - max), / sum
        float m = fmaxf(fmaxf(pr[0], pr[1]), fmaxf(pr[2], pr[3]));
        m = wave_max_f32(m);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pr[i] = l + 64 * i < E ? expf(pr[i] - m) : 0.f;
            s += pr[i];
        }
        s = wave_sum_xor(s);
#pragma unroll
        for (int i = 0; i < 4; i++) pr[i] = l + 64 * i < E ? pr[i] / s : -INFINITY;
    }
}

// The first k selections (k <= kRouteMaxK) of the top-k over pr: ids in
// sel[r] and probabilities in w[r] (uniform over the wavefront).
__device__ __forceinline__ void route_topk(const float (&pr)[4], int E, int k, uint32_t (&sel)[kRouteMaxK],
                                           float (&w)[kRouteMaxK]) {
    const int l = threadIdx.x & 63;
    // k rounds: the largest value not yet taken (in the total order of
    // route_ordered_bits), then, among the entries holding it, the lowest
    // index (ballots: entry l + 64 i, i first, then the lane).  The round's
    // value is the selected probability itself, so no lane read follows.
    // Keys: live entries at least 1, entries out of range or taken 0, so a
    // round is maxima and selects only (no flags, no branch per lane); a
    // best key of 0 means no live entry is left (index -1, as before).
    uint32_t key[4];
#pragma unroll
    for (int i = 0; i < 4; i++) key[i] = l + 64 * i < E ? max(route_ordered_bits(pr[i]), 1u) : 0u;
    // (loops over r run to the compile-time bound kRouteMaxK with a uniform
    // r < k guard: sel and w stay in scalar registers, indexed statically)
#pragma unroll
    for (int r = 0; r < kRouteMaxK; r++) sel[r] = 0u, w[r] = 0.f;
#pragma unroll
    for (int r = 0; r < kRouteMaxK; r++) {
        if (r < k) {
            const uint32_t best = (uint32_t)__builtin_amdgcn_readfirstlane(
                (int)wave_max_u32(max(max(key[0], key[1]), max(key[2], key[3]))));
            const unsigned long long b0 = __ballot(key[0] == best), b1 = __ballot(key[1] == best),
                                     b2 = __ballot(key[2] == best), b3 = __ballot(key[3] == best);
            // the first set bit of the 256-entry mask b3:b2:b1:b0 (scalar
            // minima, no branches: an empty mask gives 64 past its block)
            int idx = min(min(__builtin_ctzg(b0, 256), 64 + __builtin_ctzg(b1, 192)),
                          min(128 + __builtin_ctzg(b2, 128), 192 + __builtin_ctzg(b3, 64)));
            if (best == 0u) idx = -1;
            sel[r] = (uint32_t)idx;
            w[r] = __uint_as_float((best & 0x80000000u) ? (best & 0x7FFFFFFFu) : ~best);
            const bool mine = idx >= 0 && (idx & 63) == l;
#pragma unroll
            for (int i = 0; i < 4; i++) key[i] = (mine && (idx >> 6) == i) ? 0u : key[i];
        }
    }
}

// Expert id of selection `slot` (< kRouteMaxK): the softmax and the first
// slot + 1 rounds of the top-k, no weights (every wavefront of a workgroup
// can run it for itself).
__device__ __forceinline__ uint32_t route_id(const float *__restrict__ logits, int E, int gating, int slot) {
    float pr[4];
    route_probs(logits, E, gating, pr);
    uint32_t sel[kRouteMaxK];
    float w[kRouteMaxK];
    route_topk(pr, E, slot + 1, sel, w);
    uint32_t e = 0u;
#pragma unroll
    for (int r = 0; r < kRouteMaxK; r++) e = r == slot ? sel[r] : e;
    return e;
}

template <class Put>
__device__ __forceinline__ void route_wave(const float *__restrict__ logits, int E, int k, int gating,
                                           int weights_norm, float weights_scale, int has_shared_gate, Put put) {
    const int l = threadIdx.x & 63;
    float pr[4];
    route_probs(logits, E, gating, pr);
    // the shared expert's gate logit, loaded with the others (not after the top-k)
    const float gate_logit = has_shared_gate ? logits[E] : 0.f;
    uint32_t sel[kRouteMaxK];
    float w[kRouteMaxK];
    route_topk(pr, E, k, sel, w);
    if (l == 0) {
        if (weights_norm) {
            float sum = 0.f;
#pragma unroll
            for (int r = 0; r < kRouteMaxK; r++)
                if (r < k && isfinite(w[r]) && w[r] > 0.f) sum += w[r];
            const float inv = sum > 0.f ? 1.0f / sum : 0.f;
#pragma unroll
            for (int r = 0; r < kRouteMaxK; r++) w[r] = (sum > 0.f && isfinite(w[r]) && w[r] > 0.f) ? w[r] * inv : 0.f;
        }
        if (weights_scale != 1.0f) {
#pragma unroll
            for (int r = 0; r < kRouteMaxK; r++) w[r] *= weights_scale;
        }
#pragma unroll
        for (int r = 0; r < kRouteMaxK; r++) {
            if (r >= k) continue;
            put(2 * r, sel[r]);
            put(2 * r + 1, __float_as_uint(w[r]));
        }
        float g = 1.0f;
        if (has_shared_gate) {
            const float v = gate_logit;
            if (v >= 0.f) {
                g = 1.0f / (1.0f + expf(-v));
            } else {
                const float e = expf(v);
                g = e / (1.0f + e);
            }
        }
        put(2 * k, __float_as_uint(g));
    }
}

// One element of the MoE combine: out = sum over slots of w_s * down_s in slot
// order (addScaledInPlace: an exact weight of 1 adds without a product),
// + g * shared, then hidden + out (addInPlace) -- the reference's order.
// Used by the combine kernel and by the fused combine of the next layer's
// router launch.
__device__ __forceinline__ float combine_value(const float *hidden, const float *tmp, const uint32_t *route, int H,
                                               int k, bool has_shared, const float *sh, int r) {
    float out = 0.f;
    for (int s = 0; s < k; s++) {
        const float w = __uint_as_float(route[2 * s + 1]), d = tmp[(size_t)s * H + r];
        out = w == 1.0f ? out + d : fmaf(d, w, out);
    }
    if (has_shared) {
        const float g = __uint_as_float(route[2 * k]), d = sh[r];
        out = g == 1.0f ? out + d : fmaf(d, g, out);
    }
    return hidden[r] + out;
}

constexpr int kCombineMaxCols = 4096;   // hidden size of the fused combine at most
constexpr int kCombineFastCols = 2048;  // rows combined inside the product (two float4 per thread)

}  // namespace zh
