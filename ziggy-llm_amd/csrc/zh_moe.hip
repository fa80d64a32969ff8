// zh_moe.hip -- the MoE FFN block of a layer on the decode path (batch 1), and
// a stack of such blocks: the MI355X counterpart of computeMoeFfn
// (model/loader.zig:1718-1749) as the reference's Metal session runs it
// (runMoeFfnBlock, runtime/gpu/session.zig:515-613).
//
// One layer is four launches (five above 256 experts), captured once into a
// HIP graph for the stack:
//   router   fused RMSNorm (ffn_norm) + router matvec, and the shared
//            expert's gate row when present, into logits[E (+1)]
//   route    (in the gate/up launch's prologue up to 256 experts, see
//            zh_route.h; a launch of its own above that)
//            softmax over all experts (expert_gating_func 1, 2), top-k with
//            ties to the lower index (selectTopK, :3953-3975),
//            normalizePositiveWeights (:3977-3990) when expert_weights_norm,
//            x expert_weights_scale; sigmoid of the shared gate
//            (sigmoidScalar, :4022-4029)
//   gate/up  fused RMSNorm + gate/up + SiLU(gate) * up of the k routed
//            experts (rows offset by the routed expert id, one launch segment
//            each) and of the shared expert (computeExpertFfn :1699-1716,
//            computeSharedFfn :1679-1697)
//   down     the k + 1 down projections, each of its own activation row
//   combine  out = sum over slots of w_s * down_s in slot order
//            (addScaledInPlace), + g * shared, then hidden += out
//            (addInPlace) -- the reference's summation order per element.
#include <new>
#include <vector>

#include "zh_internal.h"
#include "zh_quant.h"
#include "zh_route.h"

namespace zh {

constexpr int kMoeMaxK = 8;
constexpr int kMoeMaxExperts = 1024;

__device__ __forceinline__ uint32_t ordered_bits_moe(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// route: [2k] {u32 id, f32 weight} entries, then the shared expert's scale.
__global__ void __launch_bounds__(256) moe_route_kernel(const float *__restrict__ logits, int E, int k, int gating,
                                                        int weights_norm, float weights_scale, int has_shared_gate,
                                                        uint32_t *__restrict__ route, int logits_stride) {
    // one workgroup per token
    logits += (size_t)blockIdx.x * logits_stride;
    route += (size_t)blockIdx.x * (2 * k + 2);
    __shared__ float pr[kMoeMaxExperts];
    __shared__ float red[4];
    __shared__ unsigned long long keys[4];
    __shared__ unsigned char taken[kMoeMaxExperts];
    __shared__ uint32_t sel[kMoeMaxK];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    for (int i = t; i < E; i += 256) {
        pr[i] = logits[i];
        taken[i] = 0;
    }
    __syncthreads();
    if (gating == 1 || gating == 2) {
        // softmaxInPlace (model/loader.zig:4160-4170): max, exp(v - max), / sum
        float m = -INFINITY;
        for (int i = t; i < E; i += 256) m = fmaxf(m, pr[i]);
        m = wave_max_f32(m);
        if (lane == 0) red[wave] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        float s = 0.f;
        for (int i = t; i < E; i += 256) {
            pr[i] = expf(pr[i] - m);
            s += pr[i];
        }
        for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
        if (lane == 0) red[wave] = s;
        __syncthreads();
        s = (red[0] + red[1]) + (red[2] + red[3]);
        for (int i = t; i < E; i += 256) pr[i] = pr[i] / s;
        __syncthreads();
    }
    // k rounds of a workgroup argmax over the values not yet taken (the
    // largest value first; equal values: the lower index first)
    for (int r = 0; r < k; r++) {
        unsigned long long best = 0ull;
        for (int i = t; i < E; i += 256) {
            if (taken[i]) continue;
            const unsigned long long key =
                ((unsigned long long)ordered_bits_moe(pr[i]) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
            best = key > best ? key : best;
        }
        best = wave_max_key(best);
        if (lane == 0) keys[wave] = best;
        __syncthreads();
        if (t == 0) {
            unsigned long long b = keys[0];
            for (int w = 1; w < 4; w++) b = keys[w] > b ? keys[w] : b;
            const uint32_t idx = 0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull);
            sel[r] = idx;
            taken[idx] = 1;
        }
        __syncthreads();
    }
    if (t == 0) {
        float w[kMoeMaxK];
        for (int r = 0; r < k; r++) w[r] = pr[sel[r]];
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
            route[2 * r] = sel[r];
            route[2 * r + 1] = __float_as_uint(w[r]);
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
        route[2 * k] = __float_as_uint(g);
    }
}

// One wavefront, up to 256 experts (four per lane): the same routing as
// moe_route_kernel with wavefront reductions only (no barriers).
__global__ void __launch_bounds__(64) moe_route_wave_kernel(const float *__restrict__ logits, int E, int k,
                                                           int gating, int weights_norm, float weights_scale,
                                                           int has_shared_gate, uint32_t *__restrict__ route,
                                                           int logits_stride) {
    logits += (size_t)blockIdx.x * logits_stride;
    route += (size_t)blockIdx.x * (2 * k + 2);
    route_wave(logits, E, k, gating, weights_norm, weights_scale, has_shared_gate,
               [&](int i, uint32_t v) { route[i] = v; });
}

__global__ void moe_combine_kernel(float *__restrict__ hidden, const float *__restrict__ tmp,
                                   const uint32_t *__restrict__ route, int H, int k, int has_shared,
                                   const float *__restrict__ sh_tmp) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= H) return;
    // token blockIdx.y: its k routed rows, its route row, its hidden row
    const int t = blockIdx.y;
    hidden += (size_t)t * H;
    route += (size_t)t * (2 * k + 2);
    tmp += (size_t)t * k * H;
    const float *sh = sh_tmp ? sh_tmp + (size_t)t * H : tmp + (size_t)k * H;
    hidden[r] = combine_value(hidden, tmp, route, H, k, has_shared != 0, sh, r);
}

hipError_t launch_moe_route(const float *logits, int E, int k, int gating, int weights_norm, float weights_scale,
                            int has_shared_gate, uint32_t *route, hipStream_t s, int tokens, int logits_stride) {
    if (E < 1 || E > kMoeMaxExperts || k < 1 || k > kMoeMaxK || k > E || tokens < 1) return hipErrorInvalidValue;
    if (E <= 256)
        hipLaunchKernelGGL(moe_route_wave_kernel, dim3(tokens), dim3(64), 0, s, logits, E, k, gating, weights_norm,
                           weights_scale, has_shared_gate, route, logits_stride);
    else
        hipLaunchKernelGGL(moe_route_kernel, dim3(tokens), dim3(256), 0, s, logits, E, k, gating, weights_norm,
                           weights_scale, has_shared_gate, route, logits_stride);
    return hipGetLastError();
}

hipError_t launch_moe_combine(float *hidden, const float *tmp, const uint32_t *route, int H, int k, int has_shared,
                              hipStream_t s, int tokens, const float *sh_tmp) {
    if (tokens < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((H + 255) / 256, tokens), dim3(256), 0, s, hidden, tmp, route, H, k,
                       has_shared, sh_tmp);
    return hipGetLastError();
}

}  // namespace zh
