/*
 * zo.h -- CPU oracle for the batch-1 GGUF decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is a plain-C restatement of the
 * reference's CPU decode path (ziggy-llm, Zig 0.15.2).  It exists to check the
 * HIP product path and to time the reference algorithm on host cores.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * nothing in the product links or calls it.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the reference's src/ directory.
 *
 * Floating-point rules (reference: Zig strict float mode, no @setFloatMode
 * anywhere): products and sums are separately rounded binary32 operations;
 * fusion happens only where the reference writes @mulAdd, restated here as
 * fmaf().  The library is compiled with -ffp-contract=off so the C compiler
 * cannot fuse on its own.  Zig's @reduce(.Add) over an 8-lane f32 vector is
 * restated as a sequential left-to-right sum (the reference does not pin the
 * order; results agree with it to tolerance, not to the last ulp).
 *
 * Parity unpinned (no reference-held vector, closed form or brute force can
 * fix these without running the Zig binary):
 *   - the summation order of the matvec dots (zo_dot_*, zo_matvec): pinned
 *     only to a float64 dot of the dequantized row, not to the last ulp;
 *   - the ulps of pow / sin / cos inside zo_apply_rope (Zig std.math vs
 *     glibc): pinned by closed forms (position 0, partial rotary) and
 *     tolerance only.
 * Everything else is pinned by the reference's known-answer tests, its
 * fixture blocks and golden text, closed forms and brute-force layouts
 * (tests/test_oracle_pins.py, tests/test_golden.py); zo_round_f16 (the
 * binary16 K/V store) against numpy's IEEE conversion at every exponent,
 * tie, subnormal and overflow boundary (tests/test_round_f16_pin.py).  The MoE composition
 * (zo_moe_ffn: router, gating, top-k, normalisation, scale, expert row
 * offsets, SwiGLU, slot-order combine, sigmoid-gated shared expert) is pinned
 * against an independent float64 composition over the dequantized weights,
 * with planted misreadings shown to fail (tests/test_moe_oracle_pin.py).
 */
#ifndef ZIGGY_ORACLE_H
#define ZIGGY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (model/loader.zig:119-153). */
enum {
    ZO_F32 = 0,
    ZO_F16 = 1,
    ZO_Q8_0 = 8,
    ZO_Q3_K = 11,
    ZO_Q4_K = 12,
    ZO_Q5_K = 13,
    ZO_Q6_K = 14,
    ZO_IQ4_XS = 23,
};

/* Status codes. */
enum {
    ZO_OK = 0,
    ZO_ERR_INVALID = 1,      /* InvalidTensorMetadata / InvalidMetadataValue */
    ZO_ERR_UNSUPPORTED = 2,  /* UnsupportedTensorType / UnsupportedArchitecture */
    ZO_ERR_MISSING = 3,      /* MissingRequiredMetadata / MissingRequiredTensor */
    ZO_ERR_TRUNCATED = 4,    /* TruncatedFile */
    ZO_ERR_CONTEXT = 5,      /* ContextOverflow */
    ZO_ERR_NOMEM = 6,
    ZO_ERR_MAGIC = 7,        /* InvalidMagic / UnsupportedVersion */
    ZO_ERR_PROMPT = 8,       /* InvalidPrompt (token id out of range) */
};

/* ---- format primitives (model/loader.zig, model/quant_extra.zig) ---- */
float zo_f16_to_f32(uint16_t h);
/* f32 -> binary16 -> f32 as the f16 KV cache stores it (Metal store_kv_half,
 * runtime/metal/matvec.metal:246-255): round to nearest even. */
float zo_round_f16(float f);
/* Bytes per row for a tensor type (model/loader.zig:3325-3389, correct rows only). */
int zo_row_bytes(int type, size_t row_len, size_t *out_bytes);
/* getScaleMinK4 (model/loader.zig:3814-3825): out[0]=scale, out[1]=min. */
void zo_scale_min_k4(int index, const uint8_t *scale_bytes, uint8_t *out);
/* dequantizeRow (model/loader.zig:3428-3459). */
int zo_dequantize_row(int type, const uint8_t *row, size_t row_len, float *out);
/* dotRow (model/loader.zig:3499-3513). */
int zo_dot_row(int type, const uint8_t *row, size_t row_len, const float *x, float *out);

/* ---- elementwise (model/loader.zig) ---- */
float zo_dot_simd(const float *a, const float *b, size_t n);                 /* :4133-4145 */
void zo_rms_norm(float *out, const float *x, const float *w, size_t n,
                 float eps, float weight_offset);                             /* :3404-3426 */
void zo_rms_norm_per_head(float *out, const float *x, const float *w, size_t head_count,
                          size_t head_dim, float eps, float weight_offset);   /* :1773-1813 */
void zo_apply_rope(float *v, size_t head_count, size_t head_dim, size_t rope_dim,
                   size_t position, float freq_base, int style);              /* :3827-3866 */
void zo_softmax(float *v, size_t n);                                          /* :4160-4170 */
uint32_t zo_argmax(const float *v, size_t n);                                 /* :3910-3920 */
void zo_silu_in_place(float *v, size_t n);                                    /* :4004-4020 */
float zo_sigmoid(float x);                                                    /* :4022-4029 */
void zo_select_topk(const float *probs, size_t n, uint32_t *idx, float *w, size_t k); /* :3953-3975 */
void zo_normalize_positive(float *w, size_t k);                               /* :3977-3990 */

/* computeAttention (model/loader.zig:1397-1438) for one layer, one position.
 * k_cache / v_cache are f32 [ctx][kv_dim] for this layer. */
void zo_attention(float *out, const float *q, const float *k_cache, const float *v_cache,
                  size_t head_count, size_t head_count_kv, size_t head_dim, size_t kv_dim,
                  size_t position, size_t window_start, float *scores_scratch);

/* Row-parallel matvec with the reference's worker policy (model/loader.zig:1596-1634,
 * 1943-2052): rows split across 1 caller + helpers when rows >= 2048 and
 * rows*cols >= 4e6.  threads <= 0 selects 1 + min(11, ncpu-1). */
int zo_matvec(int type, const uint8_t *bytes, size_t rows, size_t cols, const float *x,
              float *y, int threads);

/* ---- model + session (model/loader.zig:830-1440, 2525-2785) ---- */
typedef struct zo_model zo_model;
typedef struct zo_session zo_session;

typedef struct {
    uint32_t block_count, embedding_length, feed_forward_length, context_length;
    uint32_t head_count, head_count_kv, key_head_dim, value_head_dim, rope_dim;
    uint32_t vocab_size, rope_style, expert_count, expert_used_count, expert_ff_length;
    uint32_t expert_gating_func, expert_weights_norm, has_qk_norm, eos_token_id;
    float rms_norm_eps, rope_freq_base, expert_weights_scale;
    uint64_t data_offset;
} zo_model_info;

/* Parses a GGUF image held in memory (not copied; must outlive the model). */
int zo_model_open(const uint8_t *bytes, size_t len, zo_model **out);
void zo_model_close(zo_model *m);
int zo_model_get_info(const zo_model *m, zo_model_info *info);
/* Looks up a tensor: returns type, dims and byte offset from the start of the image. */
int zo_model_tensor(const zo_model *m, const char *name, uint32_t *type, uint64_t *row_len,
                    uint64_t *row_count, uint64_t *file_offset);

/* kv_f16 != 0 rounds K/V to binary16 at store (the reference's GPU cache semantics,
 * runtime/metal/matvec.metal:246-255); 0 keeps the CPU path's f32 cache. */
int zo_session_create(const zo_model *m, uint32_t context_length, int kv_f16, int threads,
                      zo_session **out);
void zo_session_destroy(zo_session *s);
void zo_session_reset(zo_session *s);
uint32_t zo_session_position(const zo_session *s);
int zo_session_set_position(zo_session *s, uint32_t position);
/* Session.step: runTokenCore + computeOutputCpu (model/loader.zig:1192-1209). */
int zo_session_step(zo_session *s, uint32_t token, float *logits_out);
/* Session.stepGreedy on the CPU path: argmax of the logits (:1080-1099). */
int zo_session_step_greedy(zo_session *s, uint32_t token, uint32_t *next);
/* Session.stepNoOutput (:1100-1109). */
int zo_session_step_no_output(zo_session *s, uint32_t token);
/* Copies of the running hidden state and per-layer caches, for tests. */
int zo_session_hidden(const zo_session *s, float *out);
int zo_session_kv(const zo_session *s, uint32_t layer, uint32_t position, float *k_out, float *v_out);
/* Fills the K/V cache of every layer for positions [0, position) with a
 * deterministic pattern and sets the position: to time decode at a long
 * context without running the prefill (decode cost does not depend on the
 * cached values), and to compare one long-context step with the HIP session
 * filled the same way.  x = seed * 0x9E3779B97F4A7C15 + 1, then for each
 * layer, position and dimension in that order one xorshift64 step (x ^= x<<13,
 * x ^= x>>7, x ^= x<<17) and v = ((x >> 40 & 0x7FF) - 1024) / 1024 (exact in
 * binary16); K = v, V = -v. */
int zo_session_fill_kv_pattern(zo_session *s, uint32_t position, uint64_t seed);

/* Greedy generation as generateLoadedStreaming runs it on the CPU path
 * (model/loader.zig:2065-2279): prompt token-by-token, then `steps` greedy
 * tokens (EOS ignored when ignore_eos != 0).  decode_ns brackets the decode
 * loop exactly as the reference's decode_ns does (:2135-2257). */
int zo_generate(zo_session *s, const uint32_t *prompt, size_t n_prompt, size_t steps,
                int ignore_eos, uint32_t *out_tokens, size_t *out_count, uint64_t *decode_ns);

/* MoE FFN for one layer on a normed input (computeMoeFfn, model/loader.zig:1718-1749).
 * out must be zeroed by the callee semantics of attn_tmp (it is overwritten). */
typedef struct {
    int router_type; const uint8_t *router;          /* [expert_count][hidden] */
    int exps_type; const uint8_t *gate_exps, *up_exps, *down_exps;
    int shared_type; const uint8_t *gate_sh, *up_sh, *down_sh;
    int shared_gate_type; const uint8_t *shared_gate; /* optional [1][hidden] */
    uint32_t hidden, expert_ff, shared_ff, expert_count, top_k;
    uint32_t gating_func, weights_norm;
    float weights_scale;
} zo_moe_desc;
int zo_moe_ffn(const zo_moe_desc *d, const float *normed, float *out, uint32_t *sel_experts,
               float *sel_weights, int threads);

#ifdef __cplusplus
}
#endif
#endif
