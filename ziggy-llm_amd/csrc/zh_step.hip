// zh_step.hip -- per-step kernels of the decode session: device-resident
// token/position state, embedding gather, and the fused q/k/v epilogue
// (bias, per-head QK RMSNorm, RoPE, binary16 KV store).
//
// The token and the position of a step live in device memory (StepState), so
// one captured graph replays every decode step and a whole greedy generation
// runs without host round trips: step_begin takes the next token either from
// the prompt or from the previous step's packed argmax.
#include "zh_internal.h"
#include "zh_quant.h"
#include "zh_step.h"

namespace zh {

// Device-side embedding lookup: hidden = dequant(token_embd[token])
// (embeddingLookup, model/loader.zig:3391-3402); bit-exact decode.
template <int F> __device__ void embed_row(const uint8_t *row, int cols, float *out) {
    constexpr int V = Geom<F>::kValues, B = Geom<F>::kBytes;
    for (int i = threadIdx.x; i < cols; i += blockDim.x) out[i] = dequant_value<F>(row + (size_t)(i / V) * B, i % V);
}

__global__ void step_begin_kernel(StepState *st, const uint32_t *prompt, uint32_t *history, const uint8_t *embd,
                                  uint64_t embd_stride, int embd_rows, int embd_type, int cols, float *hidden) {
    __shared__ uint32_t tok;
    if (threadIdx.x == 0) {
        uint32_t t = st->token;
        if (st->mode == 1) {
            const int i = st->step;
            if (i < st->n_prompt) {
                t = prompt[i];
            } else {
                const unsigned long long k = st->argmax;
                t = 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull);
                if (i - st->n_prompt < st->n_gen) history[i - st->n_prompt] = t;
            }
            st->pos = st->base_pos + i;
            st->out_flag = (i >= st->n_prompt - 1) ? 1 : 0;
            st->step = i + 1;
        }
        if (t >= (uint32_t)embd_rows) {
            st->error = 1;  // out-of-vocabulary token: embed row 0 and flag it for the host
            t = 0;
        }
        st->token = t;
        st->argmax = 0ull;
        tok = t;
    }
    __syncthreads();
    const uint8_t *row = embd + (uint64_t)tok * embd_stride;
    switch (embd_type) {
    case Q4_K: embed_row<Q4_K>(row, cols, hidden); break;
    case Q6_K: embed_row<Q6_K>(row, cols, hidden); break;
    case Q8_0: embed_row<Q8_0>(row, cols, hidden); break;
    case Q3_K: embed_row<Q3_K>(row, cols, hidden); break;
    case IQ4_XS: embed_row<IQ4_XS>(row, cols, hidden); break;
    case F16:
        for (int i = threadIdx.x; i < cols; i += blockDim.x) hidden[i] = h2f(ld2(row + 2 * i));
        break;
    default:
        for (int i = threadIdx.x; i < cols; i += blockDim.x) hidden[i] = __uint_as_float(ld4(row + 4 * i));
        break;
    }
}

// One workgroup per q head, k head and v head (in that order).  q/k: + bias,
// optional per-head RMSNorm (rmsNormPerHeadWithOffset, model/loader.zig:1777-1812),
// RoPE (applyRoPE, :3827-3866); k and v are stored to the cache as binary16
// (store_kv_half, matvec.metal:246-255) at the step's position.
__global__ void rope_kv_kernel(RopeKvParams p) {
    __shared__ float hv[256];
    __shared__ float red[4];
    const int b = blockIdx.x, t = threadIdx.x, hd = p.hd;
    const int pos = p.pos_dev ? *p.pos_dev : p.pos;
    int kind, head;
    if (b < p.heads) {
        kind = 0;
        head = b;
    } else if (b < p.heads + p.kv_heads) {
        kind = 1;
        head = b - p.heads;
    } else {
        kind = 2;
        head = b - p.heads - p.kv_heads;
    }
    float *src = kind == 0 ? p.q + (size_t)head * hd : (kind == 1 ? p.k + (size_t)head * hd : p.v + (size_t)head * hd);
    const float *bias = kind == 0 ? p.q_bias : (kind == 1 ? p.k_bias : p.v_bias);
    float x = 0.f;
    if (t < hd) {
        x = src[t];
        if (bias) x += bias[(size_t)head * hd + t];
    }
    const float *nw = kind == 0 ? p.q_norm : (kind == 1 ? p.k_norm : nullptr);
    if (nw) {
        float ss = t < hd ? x * x : 0.f;
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if ((t & 63) == 0) red[t >> 6] = ss;
        __syncthreads();
        float tot = 0.f;
        for (int i = 0; i < (hd + 63) / 64; i++) tot += red[i];
        const float scale = 1.0f / sqrtf(tot / (float)hd + p.eps);
        if (t < hd) x = (scale * x) * nw[t];
    }
    if (t < hd) hv[t] = x;
    __syncthreads();
    if (kind < 2) {
        const int n_rot = p.rope_dim < hd ? p.rope_dim : hd, half = n_rot / 2;
        if (t < half) {
            const int a = p.style == 0 ? 2 * t : t, c = p.style == 0 ? 2 * t + 1 : t + half;
            const float e = (float)(2 * t) / (float)n_rot;
            const float theta = (float)pos / powf(p.base, e);
            const float cs = cosf(theta), sn = sinf(theta);
            const float x0 = hv[a], x1 = hv[c];
            hv[a] = fmaf(x0, cs, -x1 * sn);
            hv[c] = fmaf(x0, sn, x1 * cs);
        }
        __syncthreads();
    }
    if (t >= hd) return;
    const float y = hv[t];
    if (kind == 0) {
        src[t] = y;
    } else if (pos < p.ctx) {
        __half *cache = kind == 1 ? p.k_cache : p.v_cache;
        const size_t idx = (size_t)pos * (size_t)(p.kv_heads * hd) + (size_t)head * hd + t;
        cache[idx] = __float2half_rn(y);
        if (kind == 1) src[t] = y;
    }
}

hipError_t launch_step_begin(StepState *st, const uint32_t *prompt, uint32_t *history, const uint8_t *embd,
                             uint64_t embd_stride, int embd_rows, int embd_type, int cols, float *hidden,
                             hipStream_t s) {
    hipLaunchKernelGGL(step_begin_kernel, dim3(1), dim3(256), 0, s, st, prompt, history, embd, embd_stride,
                       embd_rows, embd_type, cols, hidden);
    return hipGetLastError();
}

hipError_t launch_rope_kv(const RopeKvParams &p, hipStream_t s) {
    if (p.hd > 256 || p.hd % 2) return hipErrorInvalidValue;
    const int threads = p.hd <= 64 ? 64 : (p.hd <= 128 ? 128 : 256);
    hipLaunchKernelGGL(rope_kv_kernel, dim3(p.heads + 2 * p.kv_heads), dim3(threads), 0, s, p);
    return hipGetLastError();
}

}  // namespace zh
