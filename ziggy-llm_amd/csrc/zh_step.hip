// zh_step.hip -- per-step kernel of the decode session: device-resident
// token/position state and the embedding gather.  (The q/k/v epilogue --
// bias, per-head QK RMSNorm, RoPE, binary16 KV store -- runs inside the
// attention kernel, zh_attn.hip.)
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
// U values per thread per round, their loads issued before any store (the
// row and the output do not alias, so the loads need not wait for the stores
// of the round before: one memory round trip per round, not per value).
template <int F> __device__ void embed_row(const uint8_t *__restrict__ row, int cols, float *__restrict__ out) {
    constexpr int V = Geom<F>::kValues, B = Geom<F>::kBytes, U = 8;
    for (int i0 = threadIdx.x; i0 < cols; i0 += blockDim.x * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = min(i0 + u * (int)blockDim.x, cols - 1);  // past the row: re-read its last value
            v[u] = dequant_value<F>(row + (size_t)(i / V) * B, i % V);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * (int)blockDim.x;
            if (i < cols) out[i] = v[u];
        }
    }
}

// One workgroup of 1024 threads: the embedding row's loads (up to 8192
// values) all in flight in one round after the token is known.
__global__ void __launch_bounds__(1024) step_begin_kernel(StepState *st, const uint32_t *prompt, uint32_t *history, const uint8_t *embd,
                                  uint64_t embd_stride, int embd_rows, int embd_type, int cols, float *hidden) {
    __shared__ uint32_t tok;
    if (threadIdx.x == 0) {
        // every field in one batch of loads (not one round trip per branch)
        const StepState s = *st;
        uint32_t t = s.token;
        if (s.mode == 1) {
            const int i = s.step;
            if (i < s.n_prompt) {
                t = prompt[i];
            } else {
                t = 0xFFFFFFFFu - (uint32_t)(s.argmax & 0xFFFFFFFFull);
                if (i - s.n_prompt < s.n_gen) history[i - s.n_prompt] = t;
            }
            st->pos = s.base_pos + i;
            st->out_flag = (i >= s.n_prompt - 1) ? 1 : 0;
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

// Embedding rows of `count` tokens (the batched verify / prefill input):
// hidden[m] = dequant(token_embd[tokens[m]]), one workgroup per token;
// out-of-range ids embed row 0 (the host checks them first).
__global__ void embed_rows_kernel(const uint32_t *tokens, const uint8_t *embd, uint64_t embd_stride, int embd_rows,
                                  int embd_type, int cols, float *hidden) {
    uint32_t t = tokens[blockIdx.x];
    if (t >= (uint32_t)embd_rows) t = 0;
    const uint8_t *row = embd + (uint64_t)t * embd_stride;
    float *out = hidden + (size_t)blockIdx.x * cols;
    switch (embd_type) {
    case Q4_K: embed_row<Q4_K>(row, cols, out); break;
    case Q6_K: embed_row<Q6_K>(row, cols, out); break;
    case Q8_0: embed_row<Q8_0>(row, cols, out); break;
    case Q3_K: embed_row<Q3_K>(row, cols, out); break;
    case IQ4_XS: embed_row<IQ4_XS>(row, cols, out); break;
    case F16:
        for (int i = threadIdx.x; i < cols; i += blockDim.x) out[i] = h2f(ld2(row + 2 * i));
        break;
    default:
        for (int i = threadIdx.x; i < cols; i += blockDim.x) out[i] = __uint_as_float(ld4(row + 4 * i));
        break;
    }
}

hipError_t launch_embed_rows(const uint32_t *tokens, int count, const uint8_t *embd, uint64_t embd_stride,
                             int embd_rows, int embd_type, int cols, float *hidden, hipStream_t s) {
    if (count < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_rows_kernel, dim3(count), dim3(256), 0, s, tokens, embd, embd_stride, embd_rows,
                       embd_type, cols, hidden);
    return hipGetLastError();
}

hipError_t launch_step_begin(StepState *st, const uint32_t *prompt, uint32_t *history, const uint8_t *embd,
                             uint64_t embd_stride, int embd_rows, int embd_type, int cols, float *hidden,
                             hipStream_t s) {
    hipLaunchKernelGGL(step_begin_kernel, dim3(1), dim3(1024), 0, s, st, prompt, history, embd, embd_stride,
                       embd_rows, embd_type, cols, hidden);
    return hipGetLastError();
}


}  // namespace zh
