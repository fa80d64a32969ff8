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

template <class Put>
__device__ __forceinline__ void route_wave(const float *__restrict__ logits, int E, int k, int gating,
                                           int weights_norm, float weights_scale, int has_shared_gate, Put put) {
    const int l = threadIdx.x & 63;
    float pr[4];
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
    // k rounds of a wavefront argmax over the values not yet taken (the
    // largest value first; equal values: the lower index first)
    uint32_t sel[kRouteMaxK];
    unsigned taken = 0;  // bit i: expert l + 64 i taken
    for (int r = 0; r < k; r++) {
        unsigned long long best = 0ull;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int idx = l + 64 * i;
            if (idx >= E || (taken >> i & 1)) continue;
            const unsigned long long key =
                ((unsigned long long)route_ordered_bits(pr[i]) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
            best = key > best ? key : best;
        }
        best = wave_max_key(best);
        const uint32_t idx = 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull);
        sel[r] = idx;
        if ((int)(idx & 63) == l) taken |= 1u << (idx >> 6);
    }
    // the selected probabilities: from the lane that holds each
    float w[kRouteMaxK];
    for (int r = 0; r < k; r++) {
        const int e = __builtin_amdgcn_readfirstlane((int)sel[r]), src = e & 63, i = e >> 6;
        const float mine = i == 0 ? pr[0] : i == 1 ? pr[1] : i == 2 ? pr[2] : pr[3];
        w[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), src));
    }
    if (l == 0) {
        if (weights_norm) {
            float sum = 0.f;
            for (int r = 0; r < k; r++)
                if (isfinite(w[r]) && w[r] > 0.f) sum += w[r];
            if (sum <= 0.f) {
                for (int r = 0; r < k; r++) w[r] = 0.f;
            } else {
                const float inv = 1.0f / sum;
                for (int r = 0; r < k; r++) w[r] = (isfinite(w[r]) && w[r] > 0.f) ? w[r] * inv : 0.f;
            }
        }
        if (weights_scale != 1.0f)
            for (int r = 0; r < k; r++) w[r] *= weights_scale;
        for (int r = 0; r < k; r++) {
            put(2 * r, sel[r]);
            put(2 * r + 1, __float_as_uint(w[r]));
        }
        float g = 1.0f;
        if (has_shared_gate) {
            const float v = logits[E];
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

constexpr int kCombineMaxCols = 4096;  // hidden size of the fused combine at most

}  // namespace zh
