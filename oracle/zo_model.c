/*
 * zo_model.c -- CPU oracle: GGUF model parse, per-token graph, greedy decode, MoE FFN.
 *
 * TEST INFRASTRUCTURE ONLY (see zo.h).  Restates model/loader.zig of the
 * reference: loadModel (:2525-2785), Session (:871-1440), matVec/matVecRows
 * (:1596-1667), the MoE FFN (:1679-1749) and the decode loop (:2065-2279) on
 * the CPU path (backend == null).  Architectures outside the north-star path
 * (Gemma's softcap/GELU/sliding window, Qwen3.5 linear attention) are rejected.
 */
#include "zo.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define MAX_LAYERS 256

typedef struct {
    int present;
    uint32_t type;
    uint64_t row_len, rows, offset; /* offset relative to the data section */
} tref;

typedef struct {
    tref attn_norm, attn_q, attn_k, attn_v, attn_output, attn_q_bias, attn_k_bias, attn_v_bias;
    tref attn_q_norm, attn_k_norm, ffn_norm, ffn_gate, ffn_up, ffn_down;
} layer_refs;

typedef struct {
    char *name;
    tref t;
} named_tensor;

struct zo_model {
    const uint8_t *bytes;
    size_t len;
    uint64_t data_offset;
    uint32_t alignment;
    zo_model_info info;
    int rope_style;
    named_tensor *tensors;
    size_t n_tensors;
    tref token_embd, output, output_norm;
    layer_refs *layers;
};

struct zo_session {
    const zo_model *m;
    uint32_t ctx;
    int kv_f16, threads;
    uint32_t position;
    float *hidden, *normed, *q, *k, *v, *attn_out, *attn_tmp, *gate, *up, *logits, *scores, *kc, *vc;
    float *norm_w; /* scratch: an f32 norm weight vector */
};

/* ---------------- GGUF parsing (model/loader.zig:2525-2600, 3021-3272) ---------------- */

typedef struct {
    const uint8_t *b;
    size_t len, pos;
    int err;
} parser;

static int need(parser *p, size_t n) {
    if (p->err || p->pos + n > p->len || p->pos + n < p->pos) {
        p->err = ZO_ERR_TRUNCATED;
        return 0;
    }
    return 1;
}
static uint64_t rd_u(parser *p, int n) {
    if (!need(p, (size_t)n)) return 0;
    uint64_t v = 0;
    for (int i = 0; i < n; i++) v |= (uint64_t)p->b[p->pos + i] << (8 * i);
    p->pos += (size_t)n;
    return v;
}
static float rd_f(parser *p) {
    uint32_t u = (uint32_t)rd_u(p, 4);
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static const char *rd_str(parser *p, uint64_t *len) {
    *len = rd_u(p, 8);
    if (!need(p, (size_t)*len)) return NULL;
    const char *s = (const char *)p->b + p->pos;
    p->pos += (size_t)*len;
    return s;
}

/* Size of a scalar metadata value type (loader ValueType :98-113). */
static int scalar_size(uint32_t t) {
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return -1;
    }
}

static void skip_value(parser *p, uint32_t t) {
    if (t == 8) {
        uint64_t l;
        rd_str(p, &l);
        return;
    }
    if (t == 9) {
        uint32_t et = (uint32_t)rd_u(p, 4);
        uint64_t n = rd_u(p, 8);
        for (uint64_t i = 0; i < n && !p->err; i++) skip_value(p, et);
        return;
    }
    int s = scalar_size(t);
    if (s < 0) {
        p->err = ZO_ERR_INVALID;
        return;
    }
    if (need(p, (size_t)s)) p->pos += (size_t)s;
}

static uint64_t read_uint(parser *p, uint32_t t) {
    switch (t) {
    case 0: return rd_u(p, 1);
    case 2: return rd_u(p, 2);
    case 4: return rd_u(p, 4);
    case 10: return rd_u(p, 8);
    case 1: return (uint64_t)(int64_t)(int8_t)rd_u(p, 1);
    case 3: return (uint64_t)(int64_t)(int16_t)rd_u(p, 2);
    case 5: return (uint64_t)(int64_t)(int32_t)rd_u(p, 4);
    case 11: return rd_u(p, 8);
    default: p->err = ZO_ERR_INVALID; return 0;
    }
}
static double read_float(parser *p, uint32_t t) {
    if (t == 6) return rd_f(p);
    if (t == 12) {
        uint64_t u = rd_u(p, 8);
        double d;
        memcpy(&d, &u, 8);
        return d;
    }
    p->err = ZO_ERR_INVALID;
    return 0;
}

static int ends_with(const char *k, size_t kl, const char *suf) {
    size_t sl = strlen(suf);
    return kl >= sl && memcmp(k + kl - sl, suf, sl) == 0;
}
static int key_is(const char *k, size_t kl, const char *s) { return kl == strlen(s) && memcmp(k, s, kl) == 0; }

typedef struct {
    char arch[64];
    int has_arch;
    uint32_t alignment;
    int64_t block_count, embedding_length, context_length, feed_forward_length, head_count, head_count_kv;
    int64_t key_length, value_length, rope_dim, expert_count, expert_used, expert_ff, expert_gating, eos;
    int expert_weights_norm;
    double eps, rope_base, rope_scale, expert_weights_scale, partial_rotary;
    int has_eps, has_base, has_ews, has_partial;
    int64_t vocab;
    int has_tokenizer_model;
    int64_t sliding_window;
    int has_softcap;
} meta;

static void parse_kv(parser *p, meta *md) {
    uint64_t kl;
    const char *k = rd_str(p, &kl);
    uint32_t t = (uint32_t)rd_u(p, 4);
    if (p->err) return;
    if (key_is(k, kl, "general.architecture") && t == 8) {
        uint64_t l;
        const char *s = rd_str(p, &l);
        if (!s || l >= sizeof(md->arch)) {
            p->err = ZO_ERR_INVALID;
            return;
        }
        memcpy(md->arch, s, (size_t)l);
        md->arch[l] = 0;
        md->has_arch = 1;
        return;
    }
    if (key_is(k, kl, "general.alignment")) { md->alignment = (uint32_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".context_length")) { md->context_length = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".embedding_length")) { md->embedding_length = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".block_count")) { md->block_count = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".expert_feed_forward_length")) { md->expert_ff = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".expert_shared_feed_forward_length")) { read_uint(p, t); return; }
    if (ends_with(k, kl, ".feed_forward_length")) { md->feed_forward_length = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".expert_count")) { md->expert_count = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".expert_used_count")) { md->expert_used = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".expert_weights_scale")) { md->expert_weights_scale = read_float(p, t); md->has_ews = 1; return; }
    if (ends_with(k, kl, ".expert_weights_norm")) { md->expert_weights_norm = (int)rd_u(p, 1); return; }
    if (ends_with(k, kl, ".expert_gating_func")) { md->expert_gating = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".rope.dimension_count")) { md->rope_dim = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".attention.head_count")) { md->head_count = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".attention.head_count_kv")) { md->head_count_kv = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".attention.key_length")) { md->key_length = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".attention.value_length")) { md->value_length = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".attention.layer_norm_rms_epsilon") || ends_with(k, kl, ".attention.layer_norm_epsilon")) {
        md->eps = read_float(p, t);
        md->has_eps = 1;
        return;
    }
    if (ends_with(k, kl, ".rope.freq_base")) { md->rope_base = read_float(p, t); md->has_base = 1; return; }
    if (ends_with(k, kl, ".rope.scaling.factor")) { md->rope_scale = read_float(p, t); return; }
    if (ends_with(k, kl, ".attention.sliding_window")) { md->sliding_window = (int64_t)read_uint(p, t); return; }
    if (ends_with(k, kl, ".attn_logit_softcapping") || ends_with(k, kl, ".final_logit_softcapping")) {
        md->has_softcap = 1;
        skip_value(p, t);
        return;
    }
    if (key_is(k, kl, "partial_rotary_factor") || ends_with(k, kl, ".partial_rotary_factor")) {
        md->partial_rotary = read_float(p, t);
        md->has_partial = 1;
        return;
    }
    if (key_is(k, kl, "tokenizer.ggml.model")) { md->has_tokenizer_model = 1; skip_value(p, t); return; }
    if (key_is(k, kl, "tokenizer.ggml.tokens") && t == 9) {
        uint32_t et = (uint32_t)rd_u(p, 4);
        uint64_t n = rd_u(p, 8);
        md->vocab = (int64_t)n;
        for (uint64_t i = 0; i < n && !p->err; i++) skip_value(p, et);
        return;
    }
    if (key_is(k, kl, "tokenizer.ggml.eos_token_id")) { md->eos = (int64_t)read_uint(p, t); return; }
    skip_value(p, t);
}

static tref *find_tensor(zo_model *m, const char *name) {
    for (size_t i = 0; i < m->n_tensors; i++)
        if (strcmp(m->tensors[i].name, name) == 0) return &m->tensors[i].t;
    return NULL;
}

static int take(zo_model *m, const char *name, tref *out, int required) {
    tref *t = find_tensor(m, name);
    if (!t) {
        memset(out, 0, sizeof(*out));
        return required ? ZO_ERR_MISSING : ZO_OK;
    }
    *out = *t;
    return ZO_OK;
}

static int take_layer(zo_model *m, size_t layer, const char *suffix, tref *out, int required) {
    char name[96];
    snprintf(name, sizeof(name), "blk.%zu.%s", layer, suffix);
    return take(m, name, out, required);
}

int zo_model_open(const uint8_t *bytes, size_t len, zo_model **out) {
    *out = NULL;
    parser p = {bytes, len, 0, 0};
    if (!need(&p, 4) || memcmp(bytes, "GGUF", 4) != 0) return ZO_ERR_MAGIC;
    p.pos = 4;
    uint32_t version = (uint32_t)rd_u(&p, 4);
    if (version != 2 && version != 3) return ZO_ERR_MAGIC;
    uint64_t n_tensors = rd_u(&p, 8), n_kv = rd_u(&p, 8);
    if (p.err) return p.err;
    meta md;
    memset(&md, 0, sizeof(md));
    md.alignment = 32;
    md.block_count = md.embedding_length = md.context_length = md.feed_forward_length = -1;
    md.head_count = md.head_count_kv = md.key_length = md.value_length = md.rope_dim = -1;
    md.eos = -1;
    md.expert_weights_norm = -1;
    md.expert_gating = -1;
    for (uint64_t i = 0; i < n_kv && !p.err; i++) parse_kv(&p, &md);
    if (p.err) return p.err;
    if (!md.has_arch) return ZO_ERR_MISSING;
    int is_qwen = strncmp(md.arch, "qwen", 4) == 0;
    int is_mistral = strncmp(md.arch, "mistral", 7) == 0;
    int is_llama = strncmp(md.arch, "llama", 5) == 0;
    if (strcmp(md.arch, "qwen35") == 0 || strcmp(md.arch, "qwen3_5_text") == 0 || strcmp(md.arch, "qwen35moe") == 0)
        return ZO_ERR_UNSUPPORTED;
    if (!is_llama && !is_qwen && !is_mistral) return ZO_ERR_UNSUPPORTED;
    if (!md.has_tokenizer_model && !is_qwen) return ZO_ERR_MISSING;
    if (md.has_softcap || md.sliding_window > 0) return ZO_ERR_UNSUPPORTED;

    zo_model *m = (zo_model *)calloc(1, sizeof(zo_model));
    if (!m) return ZO_ERR_NOMEM;
    m->bytes = bytes;
    m->len = len;
    m->alignment = md.alignment ? md.alignment : 32;
    m->tensors = (named_tensor *)calloc(n_tensors ? n_tensors : 1, sizeof(named_tensor));
    int st = ZO_OK;
    for (uint64_t i = 0; i < n_tensors && !p.err; i++) {
        uint64_t nl;
        const char *name = rd_str(&p, &nl);
        uint32_t nd = (uint32_t)rd_u(&p, 4);
        if (p.err) break;
        if (nd == 0 || nd > 4) {
            st = ZO_ERR_INVALID;
            break;
        }
        uint64_t dims[4] = {1, 1, 1, 1};
        for (uint32_t d = 0; d < nd; d++) {
            dims[d] = rd_u(&p, 8);
            if (dims[d] == 0) st = ZO_ERR_INVALID;
        }
        uint32_t type = (uint32_t)rd_u(&p, 4);
        uint64_t off = rd_u(&p, 8);
        if (p.err || st) break;
        if (off % m->alignment) {
            st = ZO_ERR_INVALID;
            break;
        }
        named_tensor *nt = &m->tensors[m->n_tensors++];
        nt->name = (char *)malloc((size_t)nl + 1);
        memcpy(nt->name, name, (size_t)nl);
        nt->name[nl] = 0;
        nt->t.present = 1;
        nt->t.type = type;
        nt->t.row_len = dims[0];
        nt->t.rows = dims[1] * dims[2] * dims[3];
        nt->t.offset = off;
    }
    if (!st && p.err) st = p.err;
    if (st) {
        zo_model_close(m);
        return st;
    }
    m->data_offset = ((uint64_t)p.pos + m->alignment - 1) / m->alignment * m->alignment;
    if (m->data_offset > len) {
        zo_model_close(m);
        return ZO_ERR_TRUNCATED;
    }
    if (md.block_count < 0 || md.embedding_length < 0 || md.context_length < 0 || md.head_count < 0 ||
        md.head_count_kv < 0 || md.feed_forward_length < 0) {
        zo_model_close(m);
        return ZO_ERR_MISSING;
    }
    zo_model_info *in = &m->info;
    in->block_count = (uint32_t)md.block_count;
    in->embedding_length = (uint32_t)md.embedding_length;
    in->context_length = (uint32_t)md.context_length;
    in->feed_forward_length = (uint32_t)md.feed_forward_length;
    in->head_count = (uint32_t)md.head_count;
    in->head_count_kv = (uint32_t)md.head_count_kv;
    if (in->head_count == 0 || in->head_count_kv == 0 || in->embedding_length % in->head_count) {
        zo_model_close(m);
        return ZO_ERR_INVALID;
    }
    uint32_t head_dim = in->embedding_length / in->head_count;
    in->key_head_dim = md.key_length >= 0 ? (uint32_t)md.key_length : head_dim;
    in->value_head_dim = md.value_length >= 0 ? (uint32_t)md.value_length : in->key_head_dim;
    in->rope_dim = md.rope_dim >= 0 ? (uint32_t)md.rope_dim : in->key_head_dim;
    if (in->key_head_dim == 0 || in->rope_dim > in->key_head_dim || md.block_count > MAX_LAYERS) {
        zo_model_close(m);
        return ZO_ERR_INVALID;
    }
    float partial = md.has_partial ? (float)md.partial_rotary : 1.0f;
    in->rope_dim = (uint32_t)((float)in->rope_dim * partial);
    in->rms_norm_eps = md.has_eps ? (float)md.eps : 1e-6f;
    float base = md.has_base ? (float)md.rope_base : 10000.0f;
    if (md.rope_scale > 0 && base > 0) base = base / (float)md.rope_scale;
    in->rope_freq_base = base;
    in->rope_style = (is_qwen || is_mistral) ? 1 : 0; /* model/loader.zig:2571-2576 */
    in->expert_count = md.expert_count > 0 ? (uint32_t)md.expert_count : 0;
    in->expert_used_count = md.expert_used > 0 ? (uint32_t)md.expert_used : 0;
    in->expert_ff_length = md.expert_ff > 0 ? (uint32_t)md.expert_ff : 0;
    in->expert_gating_func = md.expert_gating >= 0 ? (uint32_t)md.expert_gating : 0;
    in->expert_weights_norm = md.expert_weights_norm >= 0 ? (uint32_t)md.expert_weights_norm : 0;
    in->expert_weights_scale = md.has_ews ? (float)md.expert_weights_scale : 1.0f;
    in->eos_token_id = md.eos >= 0 ? (uint32_t)md.eos : 0xFFFFFFFFu;
    in->data_offset = m->data_offset;
    m->rope_style = (int)in->rope_style;

    st = take(m, "token_embd.weight", &m->token_embd, 1);
    if (!st) {
        if (take(m, "output.weight", &m->output, 0) == ZO_OK && !m->output.present) m->output = m->token_embd;
        st = take(m, "output_norm.weight", &m->output_norm, 1);
    }
    in->vocab_size = md.vocab > 0 ? (uint32_t)md.vocab : (uint32_t)m->output.rows;
    m->layers = (layer_refs *)calloc(in->block_count ? in->block_count : 1, sizeof(layer_refs));
    for (uint32_t l = 0; l < in->block_count && !st; l++) {
        layer_refs *L = &m->layers[l];
        st = take_layer(m, l, "attn_norm.weight", &L->attn_norm, 1);
        if (!st) st = take_layer(m, l, "attn_q.weight", &L->attn_q, 1);
        if (!st) st = take_layer(m, l, "attn_k.weight", &L->attn_k, 1);
        if (!st) st = take_layer(m, l, "attn_v.weight", &L->attn_v, 1);
        if (!st) st = take_layer(m, l, "attn_output.weight", &L->attn_output, 1);
        if (!st) st = take_layer(m, l, "attn_q.bias", &L->attn_q_bias, 0);
        if (!st) st = take_layer(m, l, "attn_k.bias", &L->attn_k_bias, 0);
        if (!st) st = take_layer(m, l, "attn_v.bias", &L->attn_v_bias, 0);
        if (!st) st = take_layer(m, l, "attn_q_norm.weight", &L->attn_q_norm, 0);
        if (!st) st = take_layer(m, l, "attn_k_norm.weight", &L->attn_k_norm, 0);
        if (!st) st = take_layer(m, l, "ffn_norm.weight", &L->ffn_norm, 1);
        if (!st) st = take_layer(m, l, "ffn_gate.weight", &L->ffn_gate, 1);
        if (!st) st = take_layer(m, l, "ffn_up.weight", &L->ffn_up, 1);
        if (!st) st = take_layer(m, l, "ffn_down.weight", &L->ffn_down, 1);
        if (!st && L->attn_q_norm.present) in->has_qk_norm = 1;
    }
    if (st) {
        zo_model_close(m);
        return st;
    }
    *out = m;
    return ZO_OK;
}

void zo_model_close(zo_model *m) {
    if (!m) return;
    for (size_t i = 0; i < m->n_tensors; i++) free(m->tensors[i].name);
    free(m->tensors);
    free(m->layers);
    free(m);
}

int zo_model_get_info(const zo_model *m, zo_model_info *info) {
    *info = m->info;
    return ZO_OK;
}

int zo_model_tensor(const zo_model *m, const char *name, uint32_t *type, uint64_t *row_len, uint64_t *rows,
                    uint64_t *file_offset) {
    tref *t = find_tensor((zo_model *)m, name);
    if (!t) return ZO_ERR_MISSING;
    *type = t->type;
    *row_len = t->row_len;
    *rows = t->rows;
    *file_offset = m->data_offset + t->offset;
    return ZO_OK;
}

/* tensorBytes (model/loader.zig:3314-3323). */
static int tensor_bytes(const zo_model *m, const tref *t, const uint8_t **out) {
    size_t rb;
    int st = zo_row_bytes((int)t->type, (size_t)t->row_len, &rb);
    if (st) return st;
    uint64_t start = m->data_offset + t->offset, total = (uint64_t)rb * t->rows;
    if (start + total > m->len) return ZO_ERR_TRUNCATED;
    *out = m->bytes + start;
    return ZO_OK;
}

/* ---------------- session ---------------- */

int zo_session_create(const zo_model *m, uint32_t ctx, int kv_f16, int threads, zo_session **out) {
    const zo_model_info *in = &m->info;
    zo_session *s = (zo_session *)calloc(1, sizeof(zo_session));
    if (!s) return ZO_ERR_NOMEM;
    s->m = m;
    s->ctx = ctx ? ctx : in->context_length;
    s->kv_f16 = kv_f16;
    s->threads = threads;
    size_t H = in->embedding_length, qs = (size_t)in->head_count * in->key_head_dim;
    size_t kvs = (size_t)in->head_count_kv * in->key_head_dim, F = in->feed_forward_length;
    size_t gcap = F > qs ? F : qs, ucap = F > 2 * qs ? F : 2 * qs;
    size_t cache = (size_t)in->block_count * s->ctx * kvs;
    size_t nw = H > in->key_head_dim ? H : in->key_head_dim;
    s->hidden = calloc(H, 4);
    s->normed = calloc(H, 4);
    s->q = calloc(qs, 4);
    s->k = calloc(kvs, 4);
    s->v = calloc(kvs, 4);
    s->attn_out = calloc(qs, 4);
    s->attn_tmp = calloc(H, 4);
    s->gate = calloc(gcap, 4);
    s->up = calloc(ucap, 4);
    s->logits = calloc(in->vocab_size, 4);
    s->scores = calloc(s->ctx, 4);
    s->kc = calloc(cache ? cache : 1, 4);
    s->vc = calloc(cache ? cache : 1, 4);
    s->norm_w = calloc(nw, 4);
    if (!s->hidden || !s->normed || !s->q || !s->k || !s->v || !s->attn_out || !s->attn_tmp || !s->gate || !s->up ||
        !s->logits || !s->scores || !s->kc || !s->vc || !s->norm_w) {
        zo_session_destroy(s);
        return ZO_ERR_NOMEM;
    }
    *out = s;
    return ZO_OK;
}

void zo_session_destroy(zo_session *s) {
    if (!s) return;
    free(s->hidden); free(s->normed); free(s->q); free(s->k); free(s->v); free(s->attn_out);
    free(s->attn_tmp); free(s->gate); free(s->up); free(s->logits); free(s->scores); free(s->kc);
    free(s->vc); free(s->norm_w);
    free(s);
}

void zo_session_reset(zo_session *s) {
    const zo_model_info *in = &s->m->info;
    size_t cache = (size_t)in->block_count * s->ctx * in->head_count_kv * in->key_head_dim;
    memset(s->kc, 0, cache * 4);
    memset(s->vc, 0, cache * 4);
    s->position = 0;
}

uint32_t zo_session_position(const zo_session *s) { return s->position; }

int zo_session_set_position(zo_session *s, uint32_t pos) {
    if (pos > s->ctx) return ZO_ERR_CONTEXT;
    s->position = pos;
    return ZO_OK;
}

/* f32 -> binary16 (round to nearest even) -> f32, for the f16 KV cache mode:
 * Metal's store_kv_half writes half(src[i]) (runtime/metal/matvec.metal:246-255),
 * a round-to-nearest-even conversion with gradual underflow and overflow to
 * infinity from 65520 on. */
float zo_round_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = x & 0x80000000u, ax = x & 0x7fffffffu;
    uint16_t h;
    if (ax >= 0x7f800000u) {
        h = (uint16_t)((sign >> 16) | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    } else if (ax >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        h = (uint16_t)((sign >> 16) | 0x7c00u);
    } else if (ax < 0x38800000u) { /* below the smallest normal half: subnormal or zero */
        float a;
        memcpy(&a, &ax, 4);
        float scaled = a * 0x1p24f; /* exact */
        float r = nearbyintf(scaled); /* current mode: round-to-nearest-even */
        h = (uint16_t)((sign >> 16) | (uint16_t)r);
    } else {
        uint32_t mant = ax & 0x7fffffu, exp = (ax >> 23) - 112u;
        uint32_t hm = mant >> 13, rem = mant & 0x1fffu;
        uint32_t hv = (exp << 10) | hm;
        if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) hv++;
        h = (uint16_t)((sign >> 16) | hv);
    }
    return zo_f16_to_f32(h);
}

static int norm_weights(zo_session *s, const tref *t, size_t n, const float **w) {
    const uint8_t *b;
    if (t->type != ZO_F32) return ZO_ERR_UNSUPPORTED;
    if (t->row_len != n) return ZO_ERR_INVALID;
    int st = tensor_bytes(s->m, t, &b);
    if (st) return st;
    memcpy(s->norm_w, b, n * 4);
    *w = s->norm_w;
    return ZO_OK;
}

static int rms_norm_t(zo_session *s, float *out, const float *x, const tref *t) {
    const float *w;
    size_t n = s->m->info.embedding_length;
    int st = norm_weights(s, t, n, &w);
    if (st) return st;
    zo_rms_norm(out, x, w, n, s->m->info.rms_norm_eps, 0.0f);
    return ZO_OK;
}

/* Session.matVec (model/loader.zig:1596-1634). */
static int matvec_t(zo_session *s, float *out, const tref *t, const float *x, size_t in_len, size_t out_len) {
    if (t->row_len != in_len || t->rows != out_len) return ZO_ERR_INVALID;
    const uint8_t *b;
    int st = tensor_bytes(s->m, t, &b);
    if (st) return st;
    return zo_matvec((int)t->type, b, (size_t)t->rows, (size_t)t->row_len, x, out, s->threads);
}

/* addBiasCpu (model/loader.zig:1757-1770). */
static int add_bias(zo_session *s, float *out, const tref *t, size_t n) {
    if (!t->present) return ZO_OK;
    const uint8_t *b;
    int st = tensor_bytes(s->m, t, &b);
    if (st) return st;
    if (t->row_len != n) return ZO_ERR_INVALID;
    for (size_t i = 0; i < n; i++) {
        float v;
        if (t->type == ZO_F32) memcpy(&v, b + 4 * i, 4);
        else if (t->type == ZO_F16) v = zo_f16_to_f32((uint16_t)(b[2 * i] | (b[2 * i + 1] << 8)));
        else return ZO_ERR_UNSUPPORTED;
        out[i] += v;
    }
    return ZO_OK;
}

/* runTokenCore + runCpuAttentionBlock on the CPU path (model/loader.zig:1211-1343). */
static int run_token_core(zo_session *s, uint32_t token) {
    const zo_model *m = s->m;
    const zo_model_info *in = &m->info;
    if (s->position >= s->ctx) return ZO_ERR_CONTEXT;
    size_t H = in->embedding_length, hd = in->key_head_dim, hc = in->head_count, hkv = in->head_count_kv;
    size_t qs = hc * hd, kvs = hkv * hd, F = in->feed_forward_length;
    /* embeddingLookup (:3391-3402) */
    if (token >= m->token_embd.rows) return ZO_ERR_PROMPT;
    if (m->token_embd.row_len != H) return ZO_ERR_INVALID;
    const uint8_t *eb;
    int st = tensor_bytes(m, &m->token_embd, &eb);
    if (st) return st;
    size_t rb;
    zo_row_bytes((int)m->token_embd.type, H, &rb);
    st = zo_dequantize_row((int)m->token_embd.type, eb + (size_t)token * rb, H, s->hidden);
    if (st) return st;

    for (uint32_t l = 0; l < in->block_count; l++) {
        const layer_refs *L = &m->layers[l];
        if ((st = rms_norm_t(s, s->normed, s->hidden, &L->attn_norm))) return st;
        if ((st = matvec_t(s, s->q, &L->attn_q, s->normed, H, qs))) return st;
        if ((st = add_bias(s, s->q, &L->attn_q_bias, qs))) return st;
        if (L->attn_q_norm.present) {
            const float *w;
            if ((st = norm_weights(s, &L->attn_q_norm, hd, &w))) return st;
            zo_rms_norm_per_head(s->q, s->q, w, hc, hd, in->rms_norm_eps, 0.0f);
        }
        if ((st = matvec_t(s, s->k, &L->attn_k, s->normed, H, kvs))) return st;
        if ((st = add_bias(s, s->k, &L->attn_k_bias, kvs))) return st;
        if (L->attn_k_norm.present) {
            const float *w;
            if ((st = norm_weights(s, &L->attn_k_norm, hd, &w))) return st;
            zo_rms_norm_per_head(s->k, s->k, w, hkv, hd, in->rms_norm_eps, 0.0f);
        }
        if ((st = matvec_t(s, s->v, &L->attn_v, s->normed, H, kvs))) return st;
        if ((st = add_bias(s, s->v, &L->attn_v_bias, kvs))) return st;
        zo_apply_rope(s->q, hc, hd, in->rope_dim, s->position, in->rope_freq_base, m->rope_style);
        zo_apply_rope(s->k, hkv, hd, in->rope_dim, s->position, in->rope_freq_base, m->rope_style);
        /* storeKv (:1390-1395) */
        size_t base = (size_t)l * s->ctx * kvs + (size_t)s->position * kvs;
        for (size_t i = 0; i < kvs; i++) {
            s->kc[base + i] = s->kv_f16 ? zo_round_f16(s->k[i]) : s->k[i];
            s->vc[base + i] = s->kv_f16 ? zo_round_f16(s->v[i]) : s->v[i];
        }
        size_t lb = (size_t)l * s->ctx * kvs;
        zo_attention(s->attn_out, s->q, s->kc + lb, s->vc + lb, hc, hkv, hd, kvs, s->position, 0, s->scores);
        if ((st = matvec_t(s, s->attn_tmp, &L->attn_output, s->attn_out, qs, H))) return st;
        /* addInPlace(hidden, attn_tmp) (:3922-3933) */
        for (size_t i = 0; i < H; i++) s->hidden[i] = s->hidden[i] + s->attn_tmp[i];
        if ((st = rms_norm_t(s, s->normed, s->hidden, &L->ffn_norm))) return st;
        if ((st = matvec_t(s, s->gate, &L->ffn_gate, s->normed, H, F))) return st;
        if ((st = matvec_t(s, s->up, &L->ffn_up, s->normed, H, F))) return st;
        zo_silu_in_place(s->gate, F);
        for (size_t i = 0; i < F; i++) s->gate[i] *= s->up[i];
        if ((st = matvec_t(s, s->attn_tmp, &L->ffn_down, s->gate, F, H))) return st;
        for (size_t i = 0; i < H; i++) s->hidden[i] = s->hidden[i] + s->attn_tmp[i];
    }
    return ZO_OK;
}

/* computeOutputCpu (model/loader.zig:1357-1361). */
static int compute_output(zo_session *s) {
    const zo_model_info *in = &s->m->info;
    int st = rms_norm_t(s, s->normed, s->hidden, &s->m->output_norm);
    if (st) return st;
    return matvec_t(s, s->logits, &s->m->output, s->normed, in->embedding_length, in->vocab_size);
}

int zo_session_step(zo_session *s, uint32_t token, float *logits_out) {
    int st = run_token_core(s, token);
    if (!st) st = compute_output(s);
    if (st) return st;
    if (logits_out) memcpy(logits_out, s->logits, (size_t)s->m->info.vocab_size * 4);
    s->position++; /* finishToken (:1363-1366) */
    return ZO_OK;
}

int zo_session_step_greedy(zo_session *s, uint32_t token, uint32_t *next) {
    int st = zo_session_step(s, token, NULL);
    if (st) return st;
    *next = zo_argmax(s->logits, s->m->info.vocab_size);
    return ZO_OK;
}

int zo_session_step_no_output(zo_session *s, uint32_t token) {
    int st = run_token_core(s, token);
    if (st) return st;
    s->position++;
    return ZO_OK;
}

int zo_session_hidden(const zo_session *s, float *out) {
    memcpy(out, s->hidden, (size_t)s->m->info.embedding_length * 4);
    return ZO_OK;
}

int zo_session_kv(const zo_session *s, uint32_t layer, uint32_t pos, float *k_out, float *v_out) {
    const zo_model_info *in = &s->m->info;
    if (layer >= in->block_count || pos >= s->ctx) return ZO_ERR_INVALID;
    size_t kvs = (size_t)in->head_count_kv * in->key_head_dim;
    size_t base = (size_t)layer * s->ctx * kvs + (size_t)pos * kvs;
    memcpy(k_out, s->kc + base, kvs * 4);
    memcpy(v_out, s->vc + base, kvs * 4);
    return ZO_OK;
}

int zo_session_fill_kv_pattern(zo_session *s, uint32_t pos, uint64_t seed) {
    const zo_model_info *in = &s->m->info;
    if (pos > s->ctx) return ZO_ERR_CONTEXT;
    size_t kvs = (size_t)in->head_count_kv * in->key_head_dim;
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + 1;
    for (uint32_t l = 0; l < in->block_count; l++)
        for (size_t i = 0; i < (size_t)pos * kvs; i++) {
            x ^= x << 13;
            x ^= x >> 7;
            x ^= x << 17;
            /* multiples of 2^-10 in [-1, 1): exact in binary16, so both cache modes hold the same values */
            float v = (float)((int)(x >> 40 & 0x7FF) - 1024) * (1.0f / 1024.0f);
            size_t idx = (size_t)l * s->ctx * kvs + i;
            s->kc[idx] = v;
            s->vc[idx] = -v;
        }
    s->position = pos;
    return ZO_OK;
}

static uint64_t now_ns(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

/* generateLoadedStreaming on the CPU path, greedy (model/loader.zig:2065-2279):
 * runPrompt steps every prompt token (the last one with logits), then the
 * decode loop takes the argmax, stops on EOS, records it and steps it. */
int zo_generate(zo_session *s, const uint32_t *prompt, size_t n_prompt, size_t steps, int ignore_eos,
                uint32_t *out_tokens, size_t *out_count, uint64_t *decode_ns) {
    const zo_model_info *in = &s->m->info;
    if (n_prompt == 0) return ZO_ERR_PROMPT;
    int st = ZO_OK;
    for (size_t i = 0; i + 1 < n_prompt && !st; i++) st = zo_session_step_no_output(s, prompt[i]);
    if (!st) st = zo_session_step(s, prompt[n_prompt - 1], NULL);
    if (st) return st;
    size_t n = 0;
    uint64_t t0 = now_ns();
    while (n < steps) {
        uint32_t next = zo_argmax(s->logits, in->vocab_size);
        if (!ignore_eos && next == in->eos_token_id) break;
        out_tokens[n++] = next;
        st = zo_session_step(s, next, NULL);
        if (st) break;
    }
    uint64_t t1 = now_ns();
    if (out_count) *out_count = n;
    if (decode_ns) *decode_ns = t1 - t0;
    return st;
}

/* ---------------- MoE FFN (model/loader.zig:1679-1749) ---------------- */

/* matVecRows (model/loader.zig:1636-1667): a row window of a (possibly 3-D) tensor. */
static int matvec_rows(int type, const uint8_t *bytes, size_t cols, size_t row_offset, size_t n, const float *x,
                       float *y, int threads) {
    size_t rb;
    int st = zo_row_bytes(type, cols, &rb);
    if (st) return st;
    return zo_matvec(type, bytes + row_offset * rb, n, cols, x, y, threads);
}

int zo_moe_ffn(const zo_moe_desc *d, const float *normed, float *out, uint32_t *sel, float *selw, int threads) {
    size_t H = d->hidden, E = d->expert_count, K = d->top_k, FF = d->expert_ff, SF = d->shared_ff;
    if (E == 0 || K == 0 || FF == 0) return ZO_ERR_INVALID;
    size_t cap = FF > SF ? FF : SF;
    if (H > cap) cap = H;
    float *logits = calloc(E, 4), *g = calloc(cap, 4), *u = calloc(cap, 4);
    int st = ZO_OK;
    if (!logits || !g || !u) {
        st = ZO_ERR_NOMEM;
        goto done;
    }
    if ((st = zo_matvec(d->router_type, d->router, E, H, normed, logits, threads))) goto done;
    if (d->gating_func == 1 || d->gating_func == 2) zo_softmax(logits, E);
    else if (d->gating_func != 0) {
        st = ZO_ERR_INVALID;
        goto done;
    }
    zo_select_topk(logits, E, sel, selw, K);
    if (d->weights_norm) zo_normalize_positive(selw, K);
    if (d->weights_scale != 1.0f)
        for (size_t i = 0; i < K; i++) selw[i] *= d->weights_scale;
    memset(out, 0, H * 4);
    for (size_t s = 0; s < K; s++) {
        /* computeExpertFfn (:1699-1716) */
        size_t e = sel[s];
        if ((st = matvec_rows(d->exps_type, d->gate_exps, H, e * FF, FF, normed, g, threads))) goto done;
        if ((st = matvec_rows(d->exps_type, d->up_exps, H, e * FF, FF, normed, u, threads))) goto done;
        zo_silu_in_place(g, FF);
        for (size_t i = 0; i < FF; i++) g[i] *= u[i];
        if ((st = matvec_rows(d->exps_type, d->down_exps, FF, e * H, H, g, u, threads))) goto done;
        /* addScaledInPlace (:3935-3951) */
        if (selw[s] == 1.0f)
            for (size_t i = 0; i < H; i++) out[i] = out[i] + u[i];
        else
            for (size_t i = 0; i < H; i++) out[i] = fmaf(u[i], selw[s], out[i]);
    }
    /* computeSharedFfn (:1679-1697) scaled by sigmoid(shared gate) (:1742-1746) */
    float scale = 1.0f;
    if (d->shared_gate) {
        float dot;
        if ((st = zo_dot_row(d->shared_gate_type, d->shared_gate, H, normed, &dot))) goto done;
        scale = zo_sigmoid(dot);
    }
    if (SF > 0 && d->gate_sh) {
        if ((st = zo_matvec(d->shared_type, d->gate_sh, SF, H, normed, g, threads))) goto done;
        if ((st = zo_matvec(d->shared_type, d->up_sh, SF, H, normed, u, threads))) goto done;
        zo_silu_in_place(g, SF);
        for (size_t i = 0; i < SF; i++) g[i] *= u[i];
        if ((st = zo_matvec(d->shared_type, d->down_sh, H, SF, g, u, threads))) goto done;
        if (scale == 1.0f)
            for (size_t i = 0; i < H; i++) out[i] = out[i] + u[i];
        else
            for (size_t i = 0; i < H; i++) out[i] = fmaf(u[i], scale, out[i]);
    }
done:
    free(logits);
    free(g);
    free(u);
    return st;
}
