/*
 * ziggy_hip.h -- C ABI of libziggy_hip, the MI355X (gfx950) decode backend for
 * ziggy-llm.
 *
 * This is the HIP counterpart of the reference's Metal bridge
 * (src/runtime/metal/bridge.h).  Conventions carried over unchanged so the
 * Zig wrapper pattern of src/runtime/metal_backend.zig applies as-is:
 *   - opaque context / buffer handles (bridge.h:9-10);
 *   - every call returns an int status from the enum below (bridge.h:25-32)
 *     and takes a trailing (char *error_message, size_t error_message_len)
 *     pair that receives a NUL-terminated, truncated message
 *     (bridge.m:95-101, metal_backend.zig:2027-2047);
 *   - ops enqueue while a sequence is open and run synchronously otherwise
 *     (bridge.m:350-384, 448-485);
 *   - rows = output dimension, cols = reduction dimension; quant matrices are
 *     raw GGUF rows, row-major, row_stride = cols / QK * block_bytes;
 *   - the KV cache is [layer][pos][kv_dim] binary16 with
 *     layer_base = layer * context_length * kv_dim (gpu/session.zig:382-383).
 * Differences, each deliberate:
 *   - buffers live in HBM (hipMalloc), not shared memory: reads and writes
 *     are explicit copies;
 *   - kernels come from the library's own gfx950 code object, not source
 *     compiled at run time, so there is no shader-source argument;
 *   - dense f32/f16 projections use GGUF's row-major rows (the Metal path
 *     re-lays them column-major on the host, tensor_store.zig:208-225);
 *   - status 6 (INVALID_ARGUMENT) reports shape/offset errors that the Zig
 *     wrapper checks before calling Metal (metal_backend.zig:266-327).
 * A context is not thread-safe; use one context per host thread.
 */
#ifndef ZIGGY_HIP_H
#define ZIGGY_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ZiggyHipContext ZiggyHipContext;
typedef struct ZiggyHipBuffer ZiggyHipBuffer;
typedef struct ZiggyHipSession ZiggyHipSession;

/* Replaces ZiggyMetalDeviceInfo (bridge.h:12-17). */
typedef struct {
    char name[128];
    char arch[64];                 /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    uint64_t total_memory;         /* HBM bytes */
    uint32_t compute_units;
    uint32_t wavefront_size;
    uint32_t clock_khz;
    uint32_t l2_bytes;
} ZiggyHipDeviceInfo;

/* Replaces ZiggyMetalCommitStats (bridge.h:19-23). */
typedef struct {
    uint64_t cpu_wait_ns;
    uint64_t gpu_elapsed_ns;
    bool gpu_timestamps_valid;
} ZiggyHipCommitStats;

/* Status codes (bridge.h:25-32), plus INVALID_ARGUMENT. */
enum {
    ZIGGY_HIP_OK = 0,
    ZIGGY_HIP_UNAVAILABLE = 1,
    ZIGGY_HIP_INITIALIZATION_FAILED = 2,
    ZIGGY_HIP_COMPILATION_FAILED = 3,
    ZIGGY_HIP_BUFFER_FAILED = 4,
    ZIGGY_HIP_EXECUTION_FAILED = 5,
    ZIGGY_HIP_INVALID_ARGUMENT = 6,
};

/* GGUF tensor type ids accepted by the matvec family (model/loader.zig:119-153). */
enum {
    ZIGGY_HIP_TYPE_F32 = 0,
    ZIGGY_HIP_TYPE_F16 = 1,
    ZIGGY_HIP_TYPE_Q8_0 = 8,
    ZIGGY_HIP_TYPE_Q3_K = 11,
    ZIGGY_HIP_TYPE_Q4_K = 12,
    ZIGGY_HIP_TYPE_Q6_K = 14,
    ZIGGY_HIP_TYPE_IQ4_XS = 23,
};

/* ---- context (replaces ziggy_metal_create_context / destroy, bridge.h:34-42) ---- */
int ziggy_hip_create_context(int device_index, ZiggyHipContext **out_ctx, ZiggyHipDeviceInfo *out_info,
                             char *error_message, size_t error_message_len);
void ziggy_hip_destroy_context(ZiggyHipContext *ctx);

/* ---- buffers (replace bridge.h:44-77) ---- */
int ziggy_hip_create_buffer(ZiggyHipContext *ctx, const void *bytes, size_t length, ZiggyHipBuffer **out_buffer,
                            char *error_message, size_t error_message_len);
int ziggy_hip_create_empty_buffer(ZiggyHipContext *ctx, size_t length, ZiggyHipBuffer **out_buffer,
                                  char *error_message, size_t error_message_len);
void ziggy_hip_destroy_buffer(ZiggyHipBuffer *buffer);
size_t ziggy_hip_buffer_length(const ZiggyHipBuffer *buffer);
int ziggy_hip_write_buffer(ZiggyHipBuffer *buffer, const void *bytes, size_t length, size_t offset,
                           char *error_message, size_t error_message_len);
int ziggy_hip_read_buffer(const ZiggyHipBuffer *buffer, void *out_bytes, size_t length, size_t offset,
                          char *error_message, size_t error_message_len);
/* replaces ziggy_metal_copy_buffer_region (bridge.h:396-405) */
int ziggy_hip_copy_buffer_region(ZiggyHipContext *ctx, const ZiggyHipBuffer *src, size_t src_offset,
                                 ZiggyHipBuffer *dst, size_t dst_offset, size_t length, char *error_message,
                                 size_t error_message_len);

/* ---- sequences (replace bridge.h:497-514) ---- */
int ziggy_hip_begin_sequence(ZiggyHipContext *ctx, char *error_message, size_t error_message_len);
int ziggy_hip_commit_sequence(ZiggyHipContext *ctx, char *error_message, size_t error_message_len);
int ziggy_hip_commit_sequence_timed(ZiggyHipContext *ctx, ZiggyHipCommitStats *out_stats, char *error_message,
                                    size_t error_message_len);

/* ---- dequant-matvec (replaces the ziggy_metal_run_matvec_{f32,q4k,q6k,q8_0,q3k}_f32
 * {,_to_dst,_add} family, bridge.h:79-292).  One typed entry point:
 *   output[output_offset_bytes/4 + r] (=|+=) dot(row r of matrix, input[0..cols))
 * matrix rows start at matrix_offset bytes; add != 0 selects the _add variant.
 * cols: a multiple of 64 (and of the format's block), at most 65536; rows
 * longer than 16384 values run as column windows whose sums add in turn. ---- */
int ziggy_hip_run_matvec(ZiggyHipContext *ctx, uint32_t tensor_type, const ZiggyHipBuffer *matrix,
                         size_t matrix_offset, const ZiggyHipBuffer *input, ZiggyHipBuffer *output,
                         size_t output_offset_bytes, uint32_t rows, uint32_t cols, int add, char *error_message,
                         size_t error_message_len);
/* Named per-type wrappers with the reference's exact shapes (bridge.h:113-292). */
#define ZIGGY_HIP_DECLARE_MATVEC(sfx)                                                                              \
    int ziggy_hip_run_matvec_##sfx##_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix,                        \
                                         const ZiggyHipBuffer *input, ZiggyHipBuffer *output, uint32_t rows,         \
                                         uint32_t cols, char *error_message, size_t error_message_len);              \
    int ziggy_hip_run_matvec_##sfx##_f32_to_dst(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix,                 \
                                                const ZiggyHipBuffer *input, ZiggyHipBuffer *output,                 \
                                                size_t output_offset_bytes, uint32_t rows, uint32_t cols,            \
                                                char *error_message, size_t error_message_len);                      \
    int ziggy_hip_run_matvec_##sfx##_add_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix,                    \
                                             const ZiggyHipBuffer *input, ZiggyHipBuffer *output, uint32_t rows,     \
                                             uint32_t cols, char *error_message, size_t error_message_len);
ZIGGY_HIP_DECLARE_MATVEC(q4k)
ZIGGY_HIP_DECLARE_MATVEC(q6k)
ZIGGY_HIP_DECLARE_MATVEC(q8_0)
ZIGGY_HIP_DECLARE_MATVEC(q3k)
ZIGGY_HIP_DECLARE_MATVEC(f16)
ZIGGY_HIP_DECLARE_MATVEC(dense)

/* Fused SwiGLU + down projection + residual (replaces
 * ziggy_metal_run_matvec_q4k_silu_down_add_f32, bridge.h:372-382; any type):
 *   output[r] += dot(row r, silu(gate) * up). */
int ziggy_hip_run_matvec_silu_down_add(ZiggyHipContext *ctx, uint32_t tensor_type, const ZiggyHipBuffer *matrix,
                                       const ZiggyHipBuffer *gate, const ZiggyHipBuffer *up,
                                       ZiggyHipBuffer *output, uint32_t rows, uint32_t cols, char *error_message,
                                       size_t error_message_len);
int ziggy_hip_run_matvec_q4k_silu_down_add_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix,
                                               const ZiggyHipBuffer *gate, const ZiggyHipBuffer *up,
                                               ZiggyHipBuffer *output, uint32_t rows, uint32_t cols,
                                               char *error_message, size_t error_message_len);

/* Fused matvec + greedy argmax (replaces ziggy_metal_run_matvec_q6k_argmax_f32,
 * bridge.h:215-224).  output_state is 2 x u32: {ordered logit bits, token};
 * initialise it to {0, 0xFFFFFFFF} (the reference's convention); ties resolve
 * to the lowest token. */
int ziggy_hip_run_matvec_argmax(ZiggyHipContext *ctx, uint32_t tensor_type, const ZiggyHipBuffer *matrix,
                                const ZiggyHipBuffer *input, ZiggyHipBuffer *output_state, uint32_t rows,
                                uint32_t cols, char *error_message, size_t error_message_len);
int ziggy_hip_run_matvec_q6k_argmax_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix,
                                        const ZiggyHipBuffer *input, ZiggyHipBuffer *output_state, uint32_t rows,
                                        uint32_t cols, char *error_message, size_t error_message_len);

/* Times the matvec kernel (no counterpart in the reference): `iterations`
 * launches of ziggy_hip_run_matvec's kernel, launch i reading copy
 * (i % copies) of the matrix, copies laid out copy_stride bytes apart in
 * `matrices`, so a copy set larger than the 256 MB Infinity Cache streams
 * from HBM.  The launches run back to back between one pair of HIP events;
 * *avg_ns is the elapsed time divided by `iterations`. */
int ziggy_hip_time_matvec(ZiggyHipContext *ctx, uint32_t tensor_type, const ZiggyHipBuffer *matrices,
                          uint32_t copies, size_t copy_stride, const ZiggyHipBuffer *input, ZiggyHipBuffer *output,
                          uint32_t rows, uint32_t cols, uint32_t iterations, uint64_t *avg_ns,
                          char *error_message, size_t error_message_len);

/* Bit-exact block decode of `rows` rows to f32 (debug/parity entry; the
 * reference's counterpart is the CPU dequantizeRow, model/loader.zig:3428-3459). */
int ziggy_hip_dequantize_rows(ZiggyHipContext *ctx, uint32_t tensor_type, const ZiggyHipBuffer *matrix,
                              size_t matrix_offset, ZiggyHipBuffer *output, uint32_t rows, uint32_t cols,
                              char *error_message, size_t error_message_len);

/* ---- dense path for M >= 8 tokens on the matrix cores (the batched matvecs of the
 * reference's speculative verify, ziggy_metal_batch_matvec_*_f32, bridge.h:622-700, which
 * run one token per dispatch):
 *   output[t][r] (=|+=) dot(row r of matrix, input[t][0..cols)),  t < tokens,
 * input [tokens][cols] and output [tokens][rows] row-major f32. ---- */
int ziggy_hip_run_gemm(ZiggyHipContext *ctx, uint32_t tensor_type, const ZiggyHipBuffer *matrix,
                       const ZiggyHipBuffer *input, ZiggyHipBuffer *output, uint32_t tokens, uint32_t rows,
                       uint32_t cols, int add, char *error_message, size_t error_message_len);

/* ---- expert-indexed matvec (replace bridge.h:294-336, 701-757).  The expert id
 * is entries[slot_idx].token_id of a ShortlistEntry{u32, f32} array; rows
 * are offset by expert_id * rows_per_expert. ---- */
int ziggy_hip_indexed_matvec(ZiggyHipContext *ctx, uint32_t tensor_type, const ZiggyHipBuffer *matrix,
                             const ZiggyHipBuffer *input, ZiggyHipBuffer *output, uint32_t rows, uint32_t cols,
                             const ZiggyHipBuffer *entries, uint32_t slot_idx, uint32_t rows_per_expert,
                             int add_weighted, char *error_message, size_t error_message_len);
int ziggy_hip_dual_indexed_matvec(ZiggyHipContext *ctx, uint32_t tensor_type, const ZiggyHipBuffer *matrix_a,
                                  const ZiggyHipBuffer *matrix_b, const ZiggyHipBuffer *input,
                                  ZiggyHipBuffer *output_a, ZiggyHipBuffer *output_b, uint32_t rows, uint32_t cols,
                                  const ZiggyHipBuffer *entries, uint32_t slot_idx, uint32_t rows_per_expert,
                                  char *error_message, size_t error_message_len);
int ziggy_hip_indexed_matvec_iq4_xs_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix,
                                        const ZiggyHipBuffer *input, ZiggyHipBuffer *output, uint32_t rows,
                                        uint32_t cols, const ZiggyHipBuffer *entries, uint32_t slot_idx,
                                        uint32_t rows_per_expert, char *error_message, size_t error_message_len);
int ziggy_hip_indexed_matvec_iq4_xs_add_weighted_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix,
                                                     const ZiggyHipBuffer *input, ZiggyHipBuffer *output,
                                                     uint32_t rows, uint32_t cols, const ZiggyHipBuffer *entries,
                                                     uint32_t slot_idx, uint32_t rows_per_expert,
                                                     char *error_message, size_t error_message_len);
int ziggy_hip_indexed_matvec_q3k_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix,
                                     const ZiggyHipBuffer *input, ZiggyHipBuffer *output, uint32_t rows,
                                     uint32_t cols, const ZiggyHipBuffer *entries, uint32_t slot_idx,
                                     uint32_t rows_per_expert, char *error_message, size_t error_message_len);
int ziggy_hip_dual_indexed_matvec_q3k_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix_a,
                                          const ZiggyHipBuffer *matrix_b, const ZiggyHipBuffer *input,
                                          ZiggyHipBuffer *output_a, ZiggyHipBuffer *output_b, uint32_t rows,
                                          uint32_t cols, const ZiggyHipBuffer *entries, uint32_t slot_idx,
                                          uint32_t rows_per_expert, char *error_message,
                                          size_t error_message_len);
int ziggy_hip_indexed_matvec_q3k_add_weighted_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *matrix,
                                                  const ZiggyHipBuffer *input, ZiggyHipBuffer *output,
                                                  uint32_t rows, uint32_t cols, const ZiggyHipBuffer *entries,
                                                  uint32_t slot_idx, uint32_t rows_per_expert,
                                                  char *error_message, size_t error_message_len);

/* ---- elementwise / attention (replace bridge.h:407-620) ---- */
int ziggy_hip_apply_rope_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *vector, uint32_t head_count, uint32_t head_dim,
                             uint32_t rope_dim, uint32_t position, float freq_base, uint32_t rope_style,
                             char *error_message, size_t error_message_len);
int ziggy_hip_apply_rope_at_offset_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *vector, size_t vector_offset_bytes,
                                       uint32_t head_count, uint32_t head_dim, uint32_t rope_dim, uint32_t position,
                                       float freq_base, uint32_t rope_style, char *error_message,
                                       size_t error_message_len);
int ziggy_hip_apply_rope_to_dst_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *src, ZiggyHipBuffer *dst,
                                    size_t dst_offset_bytes, uint32_t head_count, uint32_t head_dim,
                                    uint32_t rope_dim, uint32_t position, float freq_base, uint32_t rope_style,
                                    char *error_message, size_t error_message_len);
int ziggy_hip_store_kv_half(ZiggyHipContext *ctx, const ZiggyHipBuffer *src, ZiggyHipBuffer *dst,
                            size_t dst_offset_elements, uint32_t count, char *error_message,
                            size_t error_message_len);
/* GQA decode attention over the binary16 cache; split-K flash decoding whose
 * last split to finish merges the others (replaces
 * ziggy_metal_attention_fused_f32, bridge.h:459-477).  q is the roped query;
 * the cache already holds the current position.  Positions
 * [window_start, position] are attended (any window_start <= position: the
 * reference's sliding-window layers pass position + 1 - sliding_window,
 * model/loader.zig:1440-1444).  head_dim 64, 96, 128 or 256; softcap must be
 * 0 (softcapping belongs to Gemma, outside this path). */
int ziggy_hip_attention_fused_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *q, const ZiggyHipBuffer *k_cache,
                                  const ZiggyHipBuffer *v_cache, ZiggyHipBuffer *output, uint32_t head_count,
                                  uint32_t head_count_kv, uint32_t head_dim, uint32_t kv_dim,
                                  uint32_t context_length, uint32_t position, uint32_t layer_base,
                                  uint32_t window_start, float scale, float softcap, char *error_message,
                                  size_t error_message_len);
/* The same attention, allocating nothing.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid it).  Its split partials and arrival
 * counters live in a fixed per-device static array of 4 MiB (4 KiB of
 * counters, the rest partials) instead of the context's scratch; calls whose
 * partials (kv heads x splits x 8 x (head_dim + 2) floats) exceed it fail with
 * ZIGGY_HIP_INVALID_ARGUMENT.  Calls on one device share the array, so calls
 * that overlap on one device race; each call clears the counters it uses. */
int ziggy_hip_attention_fused_f32_noalloc(ZiggyHipContext *ctx, const ZiggyHipBuffer *q,
                                          const ZiggyHipBuffer *k_cache, const ZiggyHipBuffer *v_cache,
                                          ZiggyHipBuffer *output, uint32_t head_count, uint32_t head_count_kv,
                                          uint32_t head_dim, uint32_t kv_dim, uint32_t context_length,
                                          uint32_t position, uint32_t layer_base, uint32_t window_start, float scale,
                                          float softcap, char *error_message, size_t error_message_len);
int ziggy_hip_silu_mul_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *gate, const ZiggyHipBuffer *up, uint32_t count,
                           char *error_message, size_t error_message_len);
int ziggy_hip_add_in_place_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *dst, const ZiggyHipBuffer *src,
                               uint32_t count, char *error_message, size_t error_message_len);
int ziggy_hip_add_bias_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *dst, const ZiggyHipBuffer *bias, uint32_t count,
                           char *error_message, size_t error_message_len);
int ziggy_hip_rms_norm_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *input, const ZiggyHipBuffer *weights,
                           ZiggyHipBuffer *output, uint32_t count, float eps, float weight_offset,
                           char *error_message, size_t error_message_len);
int ziggy_hip_rms_norm_per_head_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *input,
                                    const ZiggyHipBuffer *weights, ZiggyHipBuffer *output, uint32_t head_count,
                                    uint32_t head_dim, float eps, float weight_offset, char *error_message,
                                    size_t error_message_len);
int ziggy_hip_argmax_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *input, ZiggyHipBuffer *output_token,
                         uint32_t count, char *error_message, size_t error_message_len);
/* Top-k (k <= 64) as ShortlistEntry{u32 id, f32 score}, descending, ties to the
 * lower index (replaces ziggy_metal_topk_f32, bridge.h:568-576). */
int ziggy_hip_topk_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *input, ZiggyHipBuffer *output_entries,
                       uint32_t count, uint32_t top_k, char *error_message, size_t error_message_len);
int ziggy_hip_normalize_topk_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *entries, uint32_t top_k,
                                 bool apply_softmax, bool normalize_weights, float scale, char *error_message,
                                 size_t error_message_len);
int ziggy_hip_weighted_sum_topk_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *dst, const ZiggyHipBuffer *src,
                                    const ZiggyHipBuffer *entries, uint32_t count, uint32_t slot_idx,
                                    char *error_message, size_t error_message_len);
int ziggy_hip_sigmoid_scale_add_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *dst, const ZiggyHipBuffer *src,
                                    const ZiggyHipBuffer *scalar, uint32_t count, char *error_message,
                                    size_t error_message_len);

/* ---- decode session (replaces the Zig gpu.Session, runtime/gpu/session.zig:27-651,
 * which drives the entry points above one dispatch at a time).  The session
 * uploads the weights once (DenseTensorStore.prewarm,
 * runtime/gpu/metal/tensor_store.zig:112-144), owns the binary16 KV cache and
 * runs one decode step as a single captured HIP graph of fused kernels. ---- */

/* One tensor as the loader sees it (gpu/types.zig:22-27): raw GGUF bytes on the
 * host, row length (dims[0]) and row count. */
typedef struct {
    const void *data;   /* NULL = absent */
    uint64_t rows;
    uint64_t cols;
    uint32_t tensor_type;
    uint32_t reserved;
} ZiggyHipTensorDesc;

/* Per-layer tensors (gpu/types.zig:48-67; the Gemma/Qwen3.5-only fields are omitted). */
typedef struct {
    ZiggyHipTensorDesc attn_norm, attn_q, attn_k, attn_v, attn_output;
    ZiggyHipTensorDesc attn_q_bias, attn_k_bias, attn_v_bias, attn_q_norm, attn_k_norm;
    ZiggyHipTensorDesc ffn_norm, ffn_gate, ffn_up, ffn_down;
} ZiggyHipLayerDesc;

/* Model hyperparameters (gpu/types.zig:69-112, subset on this path). */
typedef struct {
    uint32_t embedding_length, block_count, context_length, feed_forward_length;
    uint32_t head_count, head_count_kv, head_dim, rope_dim;
    uint32_t vocab_size, rope_style; /* 0 = interleaved pairs, 1 = NeoX halves */
    float rms_norm_eps, rope_freq_base;
} ZiggyHipModelDesc;

typedef struct {
    uint64_t steps;
    uint64_t gpu_elapsed_ns;   /* HIP events around the decode steps */
    uint64_t wall_ns;          /* host clock around the decode steps */
    uint32_t next_token;       /* greedy token of the last step (not emitted) */
    uint32_t reserved;
    uint64_t prompt_ns;        /* host clock around the prompt (batched passes and its last step) */
} ZiggyHipGenerateStats;

/* ---- measurement probes (no counterpart in the reference: they time the
 * hardware under the decode step's launch structure; python -m zhip.microbench
 * --chain / --sync / --row-load) ---- */
typedef struct {
    uint64_t bytes;         /* bytes streamed (each entry rounded down to whole 16-byte words) */
    uint32_t kernels;       /* entries of the plan */
    uint32_t workgroups;    /* grid of every launch: the CU count */
    double one_kernel_ms;   /* all the bytes as one streaming kernel */
    double chain_ms;        /* one streaming kernel per entry, captured in a HIP graph */
    double empty_chain_ms;  /* as many empty kernels in a graph */
} ZiggyHipChainProbe;
/* Streams a byte plan (bytes[i]: what launch i of a decode step reads) three
 * ways; best of `reps` runs after one warm-up. */
int ziggy_hip_probe_chain(ZiggyHipContext *ctx, const uint64_t *bytes, uint32_t count, uint32_t reps,
                          ZiggyHipChainProbe *out, char *error_message, size_t error_message_len);
typedef struct {
    uint32_t workgroups;        /* the barriers' grid: the CU count */
    int32_t timed_out;          /* a wait ran out of its bound: the figures are not valid */
    double handoff_relaxed_us;  /* one-way hand-off between two CUs, relaxed device-scope store / load */
    double handoff_acqrel_us;   /* the same with release store / acquire load */
    double barrier_flags_us;    /* barrier of the grid: arrival words polled by one wavefront */
    double barrier_counter_us;  /* barrier of the grid: one arrival counter */
} ZiggyHipSyncProbe;
/* Latencies of in-launch dependencies between workgroups, averaged over `rounds`. */
int ziggy_hip_probe_sync(ZiggyHipContext *ctx, uint32_t rounds, ZiggyHipSyncProbe *out, char *error_message,
                         size_t error_message_len);
typedef struct {
    uint32_t workgroups;     /* two per CU, 256 lanes each */
    uint32_t values;         /* floats per row (4096) */
    double slot_us[2];       /* every lane loads its own 256-byte slot: [0] the row, [1] with a second row */
    double coalesced_us[2];  /* coalesced 16-byte loads of the same bytes per wavefront */
    double lds_us[2];        /* loaded once per workgroup into LDS, slots read there */
} ZiggyHipRowLoadProbe;
/* Median time per workgroup to bring a row written by the previous launch
 * into every lane (python -m zhip.microbench --row-load), median of `reps`. */
int ziggy_hip_probe_row_load(ZiggyHipContext *ctx, uint32_t reps, ZiggyHipRowLoadProbe *out, char *error_message,
                             size_t error_message_len);

/* Kernels of one decode step, for ziggy_hip_session_time_kernel. */
enum {
    ZIGGY_HIP_KERNEL_QKV = 0,      /* fused RMSNorm + q/k/v projections */
    ZIGGY_HIP_KERNEL_ROPE_KV = 1,  /* folded into ATTENTION: launches nothing (id kept stable) */
    ZIGGY_HIP_KERNEL_ATTENTION = 2,/* q/k bias, QK-norm, RoPE, binary16 K/V store, split-K
                                      attention with the merge in the last split */
    ZIGGY_HIP_KERNEL_O_PROJ = 3,   /* output projection + residual */
    ZIGGY_HIP_KERNEL_GATE_UP = 4,  /* fused RMSNorm + gate/up + SiLU(gate) * up */
    ZIGGY_HIP_KERNEL_DOWN = 5,     /* down projection + residual */
    ZIGGY_HIP_KERNEL_OUTPUT = 6,   /* fused RMSNorm + output head + argmax */
    ZIGGY_HIP_KERNEL_QKV_ATTENTION = 7, /* QKV and ATTENTION in one launch, as a whole step runs them
                                           where the session serves it (no reference counterpart: its
                                           step encodes them as separate dispatches) */
};

int ziggy_hip_session_create(ZiggyHipContext *ctx, const ZiggyHipModelDesc *model,
                             const ZiggyHipTensorDesc *token_embd, const ZiggyHipTensorDesc *output_norm,
                             const ZiggyHipTensorDesc *output, const ZiggyHipLayerDesc *layers,
                             ZiggyHipSession **out_session, char *error_message, size_t error_message_len);
void ziggy_hip_session_destroy(ZiggyHipSession *session);
/* Clears the cache and the position (ReusableSession.reset, model/loader.zig:857-868). */
int ziggy_hip_session_reset(ZiggyHipSession *session, char *error_message, size_t error_message_len);
uint32_t ziggy_hip_session_position(const ZiggyHipSession *session);
/* Moves the position back to `position` (<= the current one), keeping the
 * cache rows before it: the reuse of a cached prompt prefix
 * (generateLoadedStreamingCached, model/loader.zig:2281-2336, which resumes at
 * the common-prefix length).  Rows at and past `position` are overwritten by
 * the steps that follow. */
int ziggy_hip_session_rewind(ZiggyHipSession *session, uint32_t position, char *error_message,
                             size_t error_message_len);

/* Per-layer contract of gpu.Session (session.zig:258-261, 339-513, 615-651): the
 * host computes the embedding and drives the layers one call at a time. */
int ziggy_hip_session_begin_token(ZiggyHipSession *session, const float *hidden, char *error_message,
                                  size_t error_message_len);
int ziggy_hip_session_run_attention_block(ZiggyHipSession *session, uint32_t layer_index, uint32_t position,
                                          char *error_message, size_t error_message_len);
int ziggy_hip_session_run_ffn_block(ZiggyHipSession *session, uint32_t layer_index, char *error_message,
                                    size_t error_message_len);
int ziggy_hip_session_run_output(ZiggyHipSession *session, float *logits, char *error_message,
                                 size_t error_message_len);
int ziggy_hip_session_run_output_argmax(ZiggyHipSession *session, uint32_t *out_token, char *error_message,
                                        size_t error_message_len);
int ziggy_hip_session_read_hidden(ZiggyHipSession *session, float *out, char *error_message,
                                  size_t error_message_len);
int ziggy_hip_session_write_hidden(ZiggyHipSession *session, const float *values, char *error_message,
                                   size_t error_message_len);
/* Reads back K and V of one cache row (binary16 widened to f32). */
int ziggy_hip_session_read_kv(ZiggyHipSession *session, uint32_t layer, uint32_t position, float *k_out,
                              float *v_out, char *error_message, size_t error_message_len);

/* One whole greedy step (Session.stepGreedy, model/loader.zig:1080-1099) as one
 * graph launch: embedding gather on the device, every layer, final norm,
 * output projection fused with argmax.  Advances the position by one. */
int ziggy_hip_session_step_greedy(ZiggyHipSession *session, uint32_t token, uint32_t *out_next,
                                  char *error_message, size_t error_message_len);
/* Session.stepNoOutput (model/loader.zig:1100-1109): a step without the output head. */
int ziggy_hip_session_step_no_output(ZiggyHipSession *session, uint32_t token, char *error_message,
                                     size_t error_message_len);
/* Device-resident greedy generation (generateLoadedStreaming's greedy loop,
 * model/loader.zig:2065-2279): every prompt token but the last runs in
 * batched passes of up to 256 tokens on the matrix cores (the reference's
 * runPrompt, model/loader.zig:1016-1036, steps them one by one; head sizes
 * without the multi-query attention, or ZIGGY_HIP_PREFILL=steps, step them
 * too), the last one through the decode step for its logits, then
 * `steps` tokens are generated with every token fed back on the device;
 * replays of one step graph are queued back to back.  out_tokens receives
 * the generated ids.  EOS is not checked (the benchmark configurations
 * disable it). */
int ziggy_hip_session_generate(ZiggyHipSession *session, const uint32_t *prompt, uint32_t prompt_len,
                               uint32_t steps, uint32_t *out_tokens, ZiggyHipGenerateStats *stats,
                               char *error_message, size_t error_message_len);
/* Speculative verify in one batched pass (the reference's
 * verifyDraftTokensBatchGpu / gpu.Session.runBatchSpeculativeDecode,
 * model/loader.zig:1153-1190, runtime/gpu/session.zig:1525-1650, with the
 * acceptance of verifyDraftTokensSequential, model/loader.zig:1131-1151):
 * current_token and the draft_count (<= 15) drafts run at positions
 * position .. position + draft_count on the matrix cores (GEMMs of M =
 * draft_count + 1 tokens), writing their K/V rows.  out_predicted[i]
 * (draft_count + 1 entries) is the greedy token after input i;
 * *out_count = the predictions emitted: up to and including the first that
 * differs from its draft, or all of them.  The position advances by
 * *out_count (later steps overwrite the K/V of rejected drafts). */
int ziggy_hip_session_verify(ZiggyHipSession *session, uint32_t current_token, const uint32_t *drafts,
                             uint32_t draft_count, uint32_t *out_predicted, uint32_t *out_count,
                             char *error_message, size_t error_message_len);
/* Prompt prefill reusing the cached prefix (replaces the prefix reuse of
 * generateLoadedStreamingCached, model/loader.zig:2281-2336).  The session
 * records the token of every K/V row its token steps wrote.  The longest
 * common prefix of those and `prompt` is kept (the position moves back to it;
 * the reference instead resets unless all of its cache is a prefix of the
 * prompt), then the rest of the prompt is fed; the last prompt token is always
 * fed again, for its logits.  *out_reused: commonPrefixLen of the cached
 * tokens and the prompt, the count the reference reports as
 * reused_prompt_token_count (model/loader.zig:2310-2313; when the prompt
 * equals the cached tokens, one more than the rows kept, since the last
 * prompt row is recomputed); *out_next: the greedy token after the prompt.
 * Rows written by the block-level calls (run_attention_block) or by
 * session_fill_kv_pattern are not reused. */
int ziggy_hip_session_prefill_cached(ZiggyHipSession *session, const uint32_t *prompt, uint32_t prompt_len,
                                     uint32_t *out_reused, uint32_t *out_next, char *error_message,
                                     size_t error_message_len);
/* Paged KV cache.  The session's binary16 cache is a pool of pages of
 * ZIGGY_HIP_KV_PAGE_POSITIONS consecutive positions per layer; a block table
 * maps each logical page (positions 64 p .. 64 p + 63) to a pool page, shared
 * by every layer.  The reference keeps one contiguous [layer][pos][kv_dim]
 * cache (runtime/gpu/session.zig:106-111, 382-383); a paged table lets a
 * cache manager place pages (and is what the bridge-level attention's
 * layer_base addressing becomes per page).  Pages start in order.
 * set_block_table replaces the table (a permutation of the session's
 * kv_pages pages) on an empty cache (position 0). */
#define ZIGGY_HIP_KV_PAGE_POSITIONS 64
uint32_t ziggy_hip_session_kv_pages(const ZiggyHipSession *session);
int ziggy_hip_session_set_block_table(ZiggyHipSession *session, const uint32_t *table, uint32_t count,
                                      char *error_message, size_t error_message_len);
/* Test and benchmark hook (no counterpart in the reference's runtime; it
 * mirrors the CPU oracle's fill): writes a deterministic binary16-exact
 * pattern into the K/V rows [0, position) of every layer and moves the
 * position there, so one long-context step can be compared with a CPU session
 * filled the same way, or timed, without a prefill.  x = seed *
 * 0x9E3779B97F4A7C15 + 1, then per layer, position and dimension one
 * xorshift64 step (13, 7, 17) and v = ((x >> 40 & 0x7FF) - 1024) / 1024;
 * K = v, V = -v.  The rows are not reusable by prefill_cached. */
int ziggy_hip_session_fill_kv_pattern(ZiggyHipSession *session, uint32_t position, uint64_t seed,
                                      char *error_message, size_t error_message_len);
/* Logits of the most recent step that ran the output head (f32, vocab_size). */
int ziggy_hip_session_read_logits(ZiggyHipSession *session, float *out, char *error_message,
                                  size_t error_message_len);

/* ---- stochastic decoding: device shortlist, host sampler ---- */

/* ShortlistEntry (runtime/gpu/types.zig:114-117). */
typedef struct {
    uint32_t token_id;
    float logit;
} ZiggyHipShortlistEntry;
/* The sampling fields of GenerationOptions (runtime/types.zig:171-185). */
typedef struct {
    float temperature;
    float repeat_penalty;
    uint32_t top_k; /* 0: no limit */
    float top_p;
    float min_p;
} ZiggyHipSamplingOptions;
/* One decode step of `token` whose output is the top-`count` shortlist of the
 * logits: count <= 64 (max_shortlist_len, runtime/gpu/types.zig:119), the
 * highest logit first, ties to the lower token id (replaces
 * Session.runOutputShortlist, runtime/gpu/session.zig:789-828, which
 * model/loader.zig:1047 calls for the shortlist sampler).  The logits stay
 * readable with session_read_logits; the position advances by one. */
int ziggy_hip_session_step_shortlist(ZiggyHipSession *session, uint32_t token, uint32_t count,
                                     ZiggyHipShortlistEntry *out, char *error_message, size_t error_message_len);
/* shortlistLenFor (sampling.zig:47-52): the shortlist a step should return. */
uint32_t ziggy_hip_shortlist_len(const ZiggyHipSamplingOptions *options, uint32_t vocab_size);
/* The reference's CPU sampler, on the host: sampleShortlist
 * (sampling.zig:31-45, policy :54-110) over a shortlist, and sampleToken
 * (sampling.zig:11-29) over full logits.  recent: the tokens so far (repeat
 * penalty); uniform: the value random.float(f64) gives the reference, in
 * [0, 1).  Host code only: no device work. */
int ziggy_hip_sample_shortlist(const ZiggyHipShortlistEntry *entries, uint32_t count, const uint32_t *recent,
                               uint32_t recent_count, const ZiggyHipSamplingOptions *options, double uniform,
                               uint32_t *out_token);
int ziggy_hip_sample_logits(const float *logits, uint32_t count, const uint32_t *recent, uint32_t recent_count,
                            const ZiggyHipSamplingOptions *options, double uniform, uint32_t *out_token);

/* Times one kernel of the decode step (no counterpart in the reference; its
 * Metal profiler times host-side encode, runtime/metal_profile.zig:80-315):
 * one warm-up launch, then `iterations` back-to-back launches at the
 * session's current position, rotating over the layers so successive launches
 * read distinct weights from HBM, between one pair of HIP events on the
 * session stream.  Reports the mean launch duration and the algorithmic bytes
 * one launch streams (weights + binary16 KV; activations excluded).  Leaves
 * the position as it was; overwrites the hidden state and (ATTENTION,
 * QKV_ATTENTION) the cache row of the current position, which the next step
 * writes anyway.  QKV_ATTENTION fails with ZIGGY_HIP_INVALID_ARGUMENT where the
 * session runs the two separately; its launches go through whole passes over
 * the layers (`iterations` rounded up), as a step's do. */
int ziggy_hip_session_time_kernel(ZiggyHipSession *session, uint32_t kernel, uint32_t iterations,
                                  uint64_t *avg_ns, uint64_t *bytes_per_launch, char *error_message,
                                  size_t error_message_len);

/* ---- decode profiler (runtime/metal_profile.zig) ----
 * Record kinds: the reference's Category values (metal_profile.zig:3-27), in
 * its order, then the profiler calls that are not categories. */
enum {
    ZIGGY_HIP_PROFILE_PROJECTIONS = 0,
    ZIGGY_HIP_PROFILE_ATTENTION = 1,
    ZIGGY_HIP_PROFILE_KV_WRITES = 2,
    ZIGGY_HIP_PROFILE_NORMALIZATION = 3,
    ZIGGY_HIP_PROFILE_ELEMENTWISE_OPS = 4,
    ZIGGY_HIP_PROFILE_OUTPUT_REDUCE = 5,
    ZIGGY_HIP_PROFILE_COMMIT_WAIT = 6,
    ZIGGY_HIP_PROFILE_HOST_READBACK = 7,
    ZIGGY_HIP_PROFILE_CPU_SAMPLING = 8,
    ZIGGY_HIP_PROFILE_COMMIT_WAIT_GPU = 16, /* recordCommitWaitGpu (:193-197) */
    ZIGGY_HIP_PROFILE_MOON_QUANT = 17,      /* recordMoonQuantProjection (:171-191); this backend emits none */
    ZIGGY_HIP_PROFILE_TOKEN_BEGIN = 32,     /* beginDecodeToken (:120-126) */
    ZIGGY_HIP_PROFILE_TOKEN_END = 33,       /* endDecodeToken (:128-137) */
};
typedef struct {
    uint32_t kind;        /* ZIGGY_HIP_PROFILE_* */
    uint32_t has_shape;   /* 1: recordWithShape (:146-169), 0: record (:139-144) */
    uint64_t ns;
    uint64_t rows, cols, depth, extra; /* ShapeDesc (:35-41) */
    uint32_t tensor_type, reserved;
} ZiggyHipProfileRecord; /* 56 bytes */
/* Folds a record stream as the reference's Profiler does and writes its
 * renderSummary text (metal_profile.zig:201-316): the same keys in the same
 * order.  out_length receives the text's length; the call fails with
 * ZIGGY_HIP_INVALID_ARGUMENT when capacity is below out_length + 1 (the text
 * is then not written) or a record kind is unknown.  Host code only. */
int ziggy_hip_profile_render(const ZiggyHipProfileRecord *records, size_t count, char *out, size_t capacity,
                             size_t *out_length);
/* `steps` greedy decode steps from `token` (Session.stepGreedy, as
 * generateLoaded drives them with the profiler on: model/loader.zig:2137-2159)
 * with every kernel launched directly and a HIP event after each, on the
 * session stream.  Per token it emits TOKEN_BEGIN, one record per launch with
 * the launch's device time (hipEventElapsedTime of the events around it) under
 * the category of the reference's op (the step begin's embedding gather:
 * elementwise_ops; q/k/v, o, gate/up and down: projections, each with its
 * RMSNorm / SwiGLU fused; attention, with the q/k norms, RoPE and the K/V
 * store fused: attention, shaped as session.zig:445-450; where a layer's
 * q/k/v projection and attention run as one launch, that launch is one
 * attention record; the output head
 * fused with argmax: output_reduce, shaped as session.zig:633-645), then
 * COMMIT_WAIT (host time blocked in the stream synchronization),
 * COMMIT_WAIT_GPU (device time from the first event to the last),
 * HOST_READBACK (the token's device-to-host copy) and TOKEN_END.  out_tokens
 * receives the `steps` greedy tokens; the position advances by `steps`.
 * *out_count receives the records written, or, when `capacity` is too small
 * (the call then fails before any work), the count needed. */
int ziggy_hip_session_profile_decode(ZiggyHipSession *session, uint32_t token, uint32_t steps, uint32_t *out_tokens,
                                     ZiggyHipProfileRecord *records, size_t capacity, size_t *out_count,
                                     char *error_message, size_t error_message_len);

/* ---- MoE FFN layer stack (batch-1 decode) ----
 * The MoE FFN block of a layer, hidden += computeMoeFfn(rmsNorm(hidden,
 * ffn_norm)) (model/loader.zig:1262-1285, 1718-1749), as the Metal session
 * runs it (runMoeFfnBlock, runtime/gpu/session.zig:515-613), for a stack of
 * layers: router, softmax / top-k / normalise routing, the k routed experts'
 * SwiGLU FFNs (expert rows offset by the routed id) and the shared expert
 * scaled by sigmoid of its gate row (computeSharedFfn, :1679-1697).  The
 * reference's session keeps these tensors in gpu/types.zig:48-67 (the moe
 * fields); this stack uploads them once and runs every layer as one
 * captured HIP graph. */
typedef struct ZiggyHipMoeStack ZiggyHipMoeStack;

typedef struct {
    ZiggyHipTensorDesc ffn_norm;        /* f32, [1][hidden] */
    ZiggyHipTensorDesc router;          /* ffn_gate_inp: [expert_count][hidden] */
    ZiggyHipTensorDesc gate_exps;       /* ffn_gate_exps: [expert_count * expert_ff][hidden] */
    ZiggyHipTensorDesc up_exps;         /* ffn_up_exps: same shape and type */
    ZiggyHipTensorDesc down_exps;       /* ffn_down_exps: [expert_count * hidden][expert_ff] */
    ZiggyHipTensorDesc gate_shexp;      /* optional: [shared_ff][hidden] */
    ZiggyHipTensorDesc up_shexp;        /* optional: same */
    ZiggyHipTensorDesc down_shexp;      /* optional: [hidden][shared_ff] */
    ZiggyHipTensorDesc gate_inp_shexp;  /* optional: [1][hidden], same type as router */
} ZiggyHipMoeLayerDesc;

typedef struct {
    uint32_t hidden, expert_count, expert_used_count, expert_ff_length, shared_ff_length;
    uint32_t gating_func;    /* 0: raw logits, 1 / 2: softmax over all experts */
    uint32_t weights_norm;   /* normalizePositiveWeights over the selected weights */
    float weights_scale, rms_norm_eps;
} ZiggyHipMoeDesc;

int ziggy_hip_moe_stack_create(ZiggyHipContext *ctx, const ZiggyHipMoeDesc *desc, const ZiggyHipMoeLayerDesc *layers,
                               uint32_t layer_count, ZiggyHipMoeStack **out_stack, char *error_message,
                               size_t error_message_len);
void ziggy_hip_moe_stack_destroy(ZiggyHipMoeStack *stack);
/* Runs one token's hidden state (f32, [hidden]) through every layer; selected
 * (optional, [layer_count][expert_used_count] u32) and weights (optional,
 * same shape, f32) receive each layer's routing. */
int ziggy_hip_moe_stack_forward(ZiggyHipMoeStack *stack, const float *hidden_in, float *hidden_out,
                                uint32_t *selected, float *weights, char *error_message, size_t error_message_len);
/* Mean time of one pass through the stack: `iterations` graph replays back to
 * back between one pair of HIP events (no counterpart in the reference). */
int ziggy_hip_moe_stack_time(ZiggyHipMoeStack *stack, uint32_t iterations, uint64_t *avg_ns, char *error_message,
                             size_t error_message_len);
/* Prefill: `tokens` independent hidden rows (f32, [tokens][hidden]) through
 * every layer, each row exactly as ziggy_hip_moe_stack_forward would take it,
 * with the routed experts run grouped by expert on the matrix cores.
 * selected / weights (optional) are [tokens][layer_count][expert_used_count].
 * The reference prefills token by token (runPrompt, model/loader.zig:1016-1036,
 * each token through computeMoeFfn :1718-1749); rows are taken in batches of
 * up to 4096 / expert_used_count (at most 512). */
int ziggy_hip_moe_stack_prefill(ZiggyHipMoeStack *stack, const float *hidden_in, uint32_t tokens, float *hidden_out,
                                uint32_t *selected, float *weights, char *error_message, size_t error_message_len);
/* Mean time of one prefill of the first `tokens` rows of the last prefill's
 * input (tokens <= one batch), `iterations` passes between one pair of HIP
 * events (no counterpart in the reference). */
int ziggy_hip_moe_stack_time_prefill(ZiggyHipMoeStack *stack, uint32_t tokens, uint32_t iterations, uint64_t *avg_ns,
                                     char *error_message, size_t error_message_len);

/* Library build tag, for logs. */
const char *ziggy_hip_version(void);

#ifdef __cplusplus
}
#endif
#endif
