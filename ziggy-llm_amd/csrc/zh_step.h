// zh_step.h -- device-resident step state and the step-begin kernel launcher.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zh {

// Lives in device memory; read and written by the step kernels.
struct StepState {
    unsigned long long argmax;  // packed (ordered logit << 32 | ~token) of the last output head
    int mode;                   // 0: token/pos/out_flag set by the host; 1: device-driven generation
    int pos;                    // position of the token being processed
    int out_flag;               // run the output head this step
    uint32_t token;             // token being processed
    int step;                   // generation: steps done
    int base_pos;               // generation: position of prompt[0]
    int n_prompt, n_gen;
    int error;                  // set when a token is out of range
    int pad[5];
};


hipError_t launch_embed_rows(const uint32_t *tokens, int count, const uint8_t *embd, uint64_t embd_stride,
                             int embd_rows, int embd_type, int cols, float *hidden, hipStream_t s);

hipError_t launch_step_begin(StepState *st, const uint32_t *prompt, uint32_t *history, const uint8_t *embd,
                             uint64_t embd_stride, int embd_rows, int embd_type, int cols, float *hidden,
                             hipStream_t s);

}  // namespace zh
