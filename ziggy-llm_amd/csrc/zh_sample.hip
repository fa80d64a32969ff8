// zh_sample.hip -- the output shortlist of stochastic decoding: the top-k
// logits (k <= 64), highest first, ties to the lower token id, as the
// reference's GPU session hands them to its CPU sampler
// (Session.runOutputShortlist, runtime/gpu/session.zig:789-828; topk_f32,
// matvec.metal:1568-1651; sampleShortlist, sampling.zig:31-45).
//
// Two launches over packed keys (ordered value bits << 32 | ~id, so the
// largest key is the largest value and, among equal values, the lowest id):
//   partial  workgroup b takes logits [4096 b, 4096 b + 4096): each
//            wavefront's 1024 values (16 per lane) give their top k by k
//            rounds of a wavefront max, the workgroup's 4k candidates their
//            top k the same way; k keys per workgroup;
//   final    one wavefront, every workgroup's k keys: the top k, as entries.
#include "zh_internal.h"

namespace zh {

constexpr int kSlice = 4096;         // logits per partial workgroup
constexpr int kShortMax = 64;        // longest shortlist (max_shortlist_len, runtime/gpu/types.zig:119)
constexpr int kFinalPerLane = 64;    // keys per lane of the final wavefront: 64 x 64 = 4096 partial keys

__device__ __forceinline__ unsigned long long short_key(float v, uint32_t id) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(0xFFFFFFFFu - id);
}

// The top k of the N keys each lane holds (k rounds; a taken key becomes 0,
// which no real key equals); round r's winner goes to out(r) from lane 0.
template <int N, class Out>
__device__ __forceinline__ void wave_topk(unsigned long long (&key)[N], int k, Out out) {
    const int lane = threadIdx.x & 63;
    for (int r = 0; r < k; r++) {
        unsigned long long best = 0ull;
#pragma unroll
        for (int i = 0; i < N; i++) best = key[i] > best ? key[i] : best;
        best = wave_max_key(best);
#pragma unroll
        for (int i = 0; i < N; i++)
            if (key[i] == best) key[i] = 0ull;
        if (lane == 0) out(r, best);
    }
}

__global__ void __launch_bounds__(256) shortlist_partial_kernel(const float *__restrict__ x, int n, int k,
                                                                unsigned long long *__restrict__ keys) {
    __shared__ unsigned long long cand[4 * kShortMax];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int base = blockIdx.x * kSlice + wave * 1024 + lane;
    unsigned long long key[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int idx = base + 64 * i;
        key[i] = idx < n ? short_key(x[idx], (uint32_t)idx) : 0ull;
    }
    wave_topk<16>(key, k, [&](int r, unsigned long long v) { cand[wave * kShortMax + r] = v; });
    __syncthreads();
    if (wave == 0) {
        unsigned long long c[4];
#pragma unroll
        for (int i = 0; i < 4; i++) c[i] = lane < k ? cand[i * kShortMax + lane] : 0ull;
        unsigned long long *dst = keys + (size_t)blockIdx.x * k;
        wave_topk<4>(c, k, [&](int r, unsigned long long v) { dst[r] = v; });
    }
}

__global__ void __launch_bounds__(64) shortlist_final_kernel(const unsigned long long *__restrict__ keys, int nkeys,
                                                             int k, uint32_t *__restrict__ entries) {
    const int lane = threadIdx.x;
    unsigned long long key[kFinalPerLane];
#pragma unroll
    for (int i = 0; i < kFinalPerLane; i++) {
        const int j = lane + 64 * i;
        key[i] = j < nkeys ? keys[j] : 0ull;
    }
    wave_topk<kFinalPerLane>(key, k, [&](int r, unsigned long long v) {
        // entry r: {u32 token id, f32 logit} (ShortlistEntry, runtime/gpu/types.zig:114-117)
        const uint32_t o = (uint32_t)(v >> 32);
        const uint32_t bits = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
        entries[2 * r] = 0xFFFFFFFFu - (uint32_t)(v & 0xFFFFFFFFull);
        entries[2 * r + 1] = bits;
    });
}

size_t shortlist_scratch_keys(int n) { return (size_t)((n + kSlice - 1) / kSlice) * kShortMax; }

hipError_t launch_shortlist(const float *x, int n, int k, unsigned long long *keys, uint32_t *entries,
                            hipStream_t s) {
    const int blocks = (n + kSlice - 1) / kSlice;
    if (n < 1 || k < 1 || k > kShortMax || k > n || (size_t)blocks * k > (size_t)64 * kFinalPerLane)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(shortlist_partial_kernel, dim3(blocks), dim3(256), 0, s, x, n, k, keys);
    hipLaunchKernelGGL(shortlist_final_kernel, dim3(1), dim3(64), 0, s, keys, blocks * k, k, entries);
    return hipGetLastError();
}

}  // namespace zh
