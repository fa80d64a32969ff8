// zh_session.cpp -- the HIP decode session: the MI355X counterpart of the Zig
// gpu.Session (runtime/gpu/session.zig:27-651) plus a device-resident step.
//
// Weights are uploaded once into one HBM arena (raw GGUF bytes; f32 norm
// vectors as-is), the binary16 KV cache is [layer][pos][kv_dim]
// (session.zig:108-111, 382-383), and one decode step is:
//   step_begin   token (host, prompt or previous argmax) -> embedding row
//   per layer:   qkv       fused RMSNorm + q/k/v matvec (one launch, mixed formats)
//                rope_kv   bias, QK-norm, RoPE, binary16 K/V store
//                attention split-K partials + merge
//                o_proj    matvec + residual add
//                gate_up   fused RMSNorm + gate/up matvec + SiLU(gate) * up
//                down      matvec + residual add
//   output:      fused RMSNorm + output matvec + argmax (skipped on prompt steps)
// The step is captured once into a HIP graph; position and token live in
// device memory, so the same graph replays every step.
#include <algorithm>
#include <chrono>
#include <new>
#include <vector>

#include "zh_arena.h"
#include "zh_internal.h"
#include "zh_quant.h"
#include "zh_step.h"

using namespace zh;

namespace {

struct LayerW {
    DT attn_norm, q, k, v, o, q_bias, k_bias, v_bias, q_norm, k_norm, ffn_norm, gate, up, down;
};

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

}  // namespace

struct ZiggyHipSession {
    ZiggyHipContext *ctx = nullptr;
    ZiggyHipModelDesc md{};
    uint8_t *arena = nullptr;
    size_t arena_len = 0;
    DT embd, out_norm, out;
    std::vector<LayerW> layers;
    int q_size = 0, kv_size = 0, max_splits = 0;
    float *hidden = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *act = nullptr;
    float *logits = nullptr, *part_o = nullptr, *part_ml = nullptr;
    float *rope_denom = nullptr;  // [rope_dim / 2] RoPE denominators from the host's powf
    unsigned *counters = nullptr;  // attention arrival counters (zero between launches)
    // polled attention merge: two partials sets (part_o/part_ml and part_o2/part_ml2, each all
    // kPollEmpty until used); a launch uses the set the previous one did not and refills that
    // one.  attn_set: the set of the last launch enqueued; graph_set0 / graph_set1: the sets of
    // the step graph's first and last attention launch.
    bool attn_poll = false;
    float *part_o2 = nullptr, *part_ml2 = nullptr;
    int *poll_err = nullptr;
    int attn_set = 1, graph_set0 = 0, graph_set1 = 1;
    size_t attn_scratch = 0;
    // qkv_fuse: each decode step's q/k/v projection and attention run as one
    // launch (launch_qkv_attention).  Their q/k/v words come in qkv_sets sets
    // of [q][k][v], layer l using set l % qkv_sets, every word kPollEmpty
    // until used; layer l's launch refills the set of layer l + 1 (of layer 0
    // after the last), which is never its own: qkv_sets is the smallest n >= 2
    // with (layers - 1) % n != 0.  Only whole steps (layers in order) use them.
    bool qkv_fuse = false;
    // qkv_v_now: the fused launch's variant that issues its V tiles right
    // after the q/k/v wait (long contexts); chosen when the step graph is built
    bool qkv_v_now = false;
    int qkv_sets = 1;
    float *qkv_buf = nullptr;
    // binary16 K/V, paged: per layer kv_pages pages of 64 positions ([page][row in page][kv_dim]);
    // page_table[logical page] = the page's index in every layer's pool
    __half *kc = nullptr, *vc = nullptr;
    uint32_t kv_pages = 0;
    uint32_t *page_table = nullptr;
    std::vector<uint32_t> pages;  // host copy of page_table
    StepState *st = nullptr;
    StepState *st_host = nullptr;  // pinned staging for the host-driven step state
    uint32_t *prompt = nullptr, *history = nullptr;
    uint32_t prompt_cap = 0, history_cap = 0;
    hipGraphExec_t graph = nullptr;
    const uint32_t *graph_prompt = nullptr, *graph_history = nullptr;  // the buffers the graph's step_begin reads
    bool graph_v_now = false;                                          // the graph's fused-launch variant
    // batched verify (allocated on first use): [kVerifyMax] rows each
    float *b_hidden = nullptr, *b_normed = nullptr, *b_q = nullptr, *b_k = nullptr, *b_v = nullptr;
    float *b_attn = nullptr, *b_act = nullptr, *b_up = nullptr, *b_logits = nullptr;
    float *b_ss = nullptr;  // verify: the deferred norms' row sums of squares, [2][kPassMax]
    // output shortlist (allocated on first use): packed keys, entries
    unsigned long long *sl_keys = nullptr;
    uint32_t *sl_entries = nullptr;
    uint32_t *b_tokens = nullptr;
    unsigned long long *b_argmax = nullptr;
    // multi-query attention of a verify pass: partials and arrival counters
    // of head_count_kv * query-group slots
    float *b_part_o = nullptr, *b_part_ml = nullptr;
    zh::XPlanes xp{};  // the o and down products' inputs, split once per pass
    unsigned *b_counters = nullptr;
    uint32_t position = 0;
    // the token whose K/V rows sit at each position below `position`, while
    // every row came from a token step (prefix reuse); block-level calls,
    // which write rows from hidden states, clear fed_ok
    std::vector<uint32_t> fed;
    bool fed_ok = true;
    bool logits_valid = false;
    std::vector<void *> allocs;
};

namespace {

// Start of layer l's pages in the K or V pool, and the row of position pos in it.
size_t kv_layer_base(const ZiggyHipSession *s, int l) {
    return (size_t)l * ((size_t)s->kv_pages << kKvPageShift) * s->kv_size;
}
size_t kv_row_host(const ZiggyHipSession *s, uint32_t pos) {
    return ((size_t)s->pages[pos >> kKvPageShift] << kKvPageShift) + (pos & ((1u << kKvPageShift) - 1));
}

int fail(char *err, size_t err_len, int code, const char *msg) {
    set_err(err, err_len, "%s", msg);
    return code;
}

// Plans a matvec over one or more row segments sharing the input.
MvParams mv_params(const ZiggyHipSession *s, const DT *const *mats, float *const *ys, int n, int cols,
                   const float *x) {
    MvParams p{};
    p.nseg = n;
    for (int i = 0; i < n; i++) {
        p.seg[i].w = mats[i]->p;
        p.seg[i].stride = mats[i]->stride;
        p.seg[i].y = ys[i];
        p.seg[i].rows = (int)mats[i]->rows;
        p.seg[i].fmt = mats[i]->type;
    }
    p.cols = cols;
    p.x = x;
    p.eps = s->md.rms_norm_eps;
    plan_matvec(p, 1024);
    return p;
}

// The decode step's single-query attention parameters for layer l (fused
// mode: the projection's q, k, v epilogue and the K/V store), with the polled
// merge's partials sets taken in turn.
AttnParams step_attention_params(ZiggyHipSession *s, int l, const int *pos_dev, int pos, const float *q,
                             const float *k, const float *v) {
    const ZiggyHipModelDesc &md = s->md;
    const LayerW &L = s->layers[l < 0 ? 0 : l];
    const size_t layer_base = kv_layer_base(s, l < 0 ? 0 : l);
    AttnParams a{};
    a.q = q;
    a.k_new = k;
    a.v_new = v;
    a.q_bias = L.q_bias.present ? (const float *)L.q_bias.p : nullptr;
    a.k_bias = L.k_bias.present ? (const float *)L.k_bias.p : nullptr;
    a.v_bias = L.v_bias.present ? (const float *)L.v_bias.p : nullptr;
    a.q_norm = L.q_norm.present ? (const float *)L.q_norm.p : nullptr;
    a.k_norm = L.k_norm.present ? (const float *)L.k_norm.p : nullptr;
    a.k_cache = s->kc + layer_base;
    a.v_cache = s->vc + layer_base;
    a.page_table = s->page_table;
    a.page_shift = kKvPageShift;
    a.out = s->attn;
    a.part_o = s->part_o;
    a.part_ml = s->part_ml;
    a.counters = s->counters;
    a.head_count = (int)md.head_count;
    a.head_count_kv = (int)md.head_count_kv;
    a.head_dim = (int)md.head_dim;
    a.kv_dim = s->kv_size;
    a.position = pos;
    a.position_dev = pos_dev;
    a.window_start = 0;
    a.scale = 1.0f / sqrtf((float)md.head_dim);
    a.max_splits = s->max_splits;
    a.eps = md.rms_norm_eps;
    a.rope_base = md.rope_freq_base;
    a.rope_denom = s->rope_denom;
    a.rope_dim = (int)md.rope_dim;
    a.rope_style = (int)md.rope_style;
    a.ctx = (int)md.context_length;
    if (s->attn_poll) {
        const int set = s->attn_set ^ 1;
        a.part_o = set ? s->part_o2 : s->part_o;
        a.part_ml = set ? s->part_ml2 : s->part_ml;
        a.reset_o = set ? s->part_o : s->part_o2;
        a.reset_ml = set ? s->part_ml : s->part_ml2;
        a.poll_merge = 1;
        a.poll_err = s->poll_err;
        a.min_tiles = attention_poll_min_tiles();
        s->attn_set = set;
    }
    return a;
}

// Enqueues one kernel of the step (ZIGGY_HIP_KERNEL_*) for layer l.  With
// pos_dev set the position comes from device memory (graph replay).
hipError_t enqueue_kernel(ZiggyHipSession *s, int id, int l, const int *pos_dev, int pos, hipStream_t st) {
    const ZiggyHipModelDesc &md = s->md;
    const int H = (int)md.embedding_length, F = (int)md.feed_forward_length;
    const LayerW &L = s->layers[l < 0 ? 0 : l];
    const size_t layer_base = kv_layer_base(s, l < 0 ? 0 : l);
    switch (id) {
    case ZIGGY_HIP_KERNEL_QKV: {
        const DT *m[3] = {&L.q, &L.k, &L.v};
        float *ys[3] = {s->q, s->k, s->v};
        MvParams p = mv_params(s, m, ys, 3, H, s->hidden);
        p.norm_w = (const float *)L.attn_norm.p;
        return launch_matvec(p, IN_NORM, OUT_STORE, st);
    }
    case ZIGGY_HIP_KERNEL_ROPE_KV:
        // the q/k/v epilogue and the K/V store run inside the attention kernel
        return hipSuccess;
    case ZIGGY_HIP_KERNEL_ATTENTION: {
        AttnParams a = step_attention_params(s, l, pos_dev, pos, s->q, s->k, s->v);
        return launch_attention(a, st);
    }
    case ZIGGY_HIP_KERNEL_O_PROJ: {
        const DT *m[1] = {&L.o};
        float *ys[1] = {s->hidden};
        MvParams p = mv_params(s, m, ys, 1, s->q_size, s->attn);
        return launch_matvec(p, IN_PLAIN, OUT_ADD, st);
    }
    case ZIGGY_HIP_KERNEL_GATE_UP: {
        const DT *m[1] = {&L.gate};
        float *ys[1] = {s->act};
        MvParams p = mv_params(s, m, ys, 1, H, s->hidden);
        p.norm_w = (const float *)L.ffn_norm.p;
        if (L.gate.type == L.up.type) {
            p.seg[0].w2 = L.up.p;
            return launch_matvec(p, IN_NORM, OUT_SWIGLU, st);
        }
        // gate and up in different formats: two projections; the down kernel gates
        hipError_t e = launch_matvec(p, IN_NORM, OUT_STORE, st);
        if (e != hipSuccess) return e;
        const DT *mu[1] = {&L.up};
        float *yu[1] = {s->logits};  // the logits buffer is at least F long (sized at create)
        MvParams pu = mv_params(s, mu, yu, 1, H, s->hidden);
        pu.norm_w = (const float *)L.ffn_norm.p;
        return launch_matvec(pu, IN_NORM, OUT_STORE, st);
    }
    case ZIGGY_HIP_KERNEL_DOWN: {
        const DT *m[1] = {&L.down};
        float *ys[1] = {s->hidden};
        MvParams p = mv_params(s, m, ys, 1, F, s->act);
        if (L.gate.type == L.up.type) return launch_matvec(p, IN_PLAIN, OUT_ADD, st);
        p.x2 = s->logits;
        return launch_matvec(p, IN_SILU, OUT_ADD, st);
    }
    case ZIGGY_HIP_KERNEL_OUTPUT: {
        // fused final RMSNorm + output matvec + argmax (session.zig:633-651);
        // on the device-driven step it is skipped on prompt steps (out_flag)
        const DT *m[1] = {&s->out};
        float *ys[1] = {s->logits};
        MvParams p = mv_params(s, m, ys, 1, H, s->hidden);
        p.norm_w = (const float *)s->out_norm.p;
        p.gate_flag = pos_dev ? &s->st->out_flag : nullptr;
        p.argmax_slot = &s->st->argmax;
        return launch_matvec(p, IN_NORM, OUT_ARGMAX, st);
    }
    default: return hipErrorInvalidValue;
    }
}

// The attention block of one layer (session.zig:339-466).
hipError_t enqueue_attention_block(ZiggyHipSession *s, int l, const int *pos_dev, int pos, hipStream_t st) {
    for (int id : {ZIGGY_HIP_KERNEL_QKV, ZIGGY_HIP_KERNEL_ROPE_KV, ZIGGY_HIP_KERNEL_ATTENTION, ZIGGY_HIP_KERNEL_O_PROJ}) {
        hipError_t e = enqueue_kernel(s, id, l, pos_dev, pos, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Layer l's q/k/v projection and attention in one launch (qkv_fuse): q/k/v
// in layer l's set, the next layer's set refilled.  The position comes from
// pos_dev when set (graph replay), else pos.
hipError_t launch_qkv_attention_layer(ZiggyHipSession *s, int l, const int *pos_dev, int pos, hipStream_t st) {
    const int L = (int)s->layers.size();
    const LayerW &W = s->layers[l];
    const size_t per = (size_t)s->q_size + 2 * (size_t)s->kv_size;
    float *set = s->qkv_buf + (size_t)(l % s->qkv_sets) * per;
    float *next = s->qkv_buf + (size_t)(((l + 1) % L) % s->qkv_sets) * per;
    float *q = set, *k = set + s->q_size, *v = k + s->kv_size;
    const DT *m[3] = {&W.q, &W.k, &W.v};
    float *ys[3] = {q, k, v};
    MvParams p = mv_params(s, m, ys, 3, (int)s->md.embedding_length, s->hidden);
    p.norm_w = (const float *)W.attn_norm.p;
    AttnParams a = step_attention_params(s, l, pos_dev, pos, q, k, v);
    a.qkv_refill = next;
    return launch_qkv_attention(p, a, st, s->qkv_v_now);
}

// The attention block of layer l inside a whole decode step: with qkv_fuse
// the q/k/v projection and the attention in one launch, then o_proj;
// otherwise the launches of enqueue_attention_block.
hipError_t enqueue_attention_step(ZiggyHipSession *s, int l, const int *pos_dev, hipStream_t st) {
    if (!s->qkv_fuse) return enqueue_attention_block(s, l, pos_dev, 0, st);
    const hipError_t e = launch_qkv_attention_layer(s, l, pos_dev, 0, st);
    if (e != hipSuccess) return e;
    return enqueue_kernel(s, ZIGGY_HIP_KERNEL_O_PROJ, l, pos_dev, 0, st);
}

// The FFN block of one layer (session.zig:468-513).
hipError_t enqueue_ffn_block(ZiggyHipSession *s, int l, hipStream_t st) {
    hipError_t e = enqueue_kernel(s, ZIGGY_HIP_KERNEL_GATE_UP, l, nullptr, 0, st);
    if (e != hipSuccess) return e;
    return enqueue_kernel(s, ZIGGY_HIP_KERNEL_DOWN, l, nullptr, 0, st);
}

// Output head into the logits buffer, without argmax (session.zig:615-631).
hipError_t enqueue_output_logits(ZiggyHipSession *s, hipStream_t st) {
    const DT *m[1] = {&s->out};
    float *ys[1] = {s->logits};
    MvParams p = mv_params(s, m, ys, 1, (int)s->md.embedding_length, s->hidden);
    p.norm_w = (const float *)s->out_norm.p;
    return launch_matvec(p, IN_NORM, OUT_STORE, st);
}

// Algorithmic HBM bytes one launch of kernel `id` streams at position pos.
uint64_t kernel_bytes(const ZiggyHipSession *s, int id, int l, int pos) {
    const LayerW &L = s->layers[l];
    auto mb = [](const DT &d) { return d.stride * d.rows; };
    switch (id) {
    case ZIGGY_HIP_KERNEL_QKV: return mb(L.q) + mb(L.k) + mb(L.v);
    case ZIGGY_HIP_KERNEL_ROPE_KV: return 0;
    case ZIGGY_HIP_KERNEL_ATTENTION: return (uint64_t)(pos + 1) * s->kv_size * 2 * 2;
    case ZIGGY_HIP_KERNEL_O_PROJ: return mb(L.o);
    case ZIGGY_HIP_KERNEL_GATE_UP: return mb(L.gate) + mb(L.up);
    case ZIGGY_HIP_KERNEL_DOWN: return mb(L.down);
    case ZIGGY_HIP_KERNEL_OUTPUT: return mb(s->out);
    default: return 0;
    }
}

hipError_t enqueue_step(ZiggyHipSession *s, hipStream_t st) {
    hipError_t e = launch_step_begin(s->st, s->prompt, s->history, s->embd.p, s->embd.stride, (int)s->embd.rows,
                                     s->embd.type, (int)s->md.embedding_length, s->hidden, st);
    if (e != hipSuccess) return e;
    for (int l = 0; l < (int)s->md.block_count; l++) {
        e = enqueue_attention_step(s, l, &s->st->pos, st);
        if (e != hipSuccess) return e;
        e = enqueue_ffn_block(s, l, st);
        if (e != hipSuccess) return e;
    }
    return enqueue_kernel(s, ZIGGY_HIP_KERNEL_OUTPUT, 0, &s->st->pos, 0, st);
}

// One step: a replay of the captured graph, or (ZIGGY_HIP_GRAPH=0, e.g. under
// a profiler that cannot intercept graph launches) the same kernels enqueued
// directly; both read token and position from the device step state.
hipError_t launch_step(ZiggyHipSession *s, hipStream_t st) {
    if (!s->graph) return enqueue_step(s, st);
    if (s->attn_poll && s->attn_set == s->graph_set0) {
        // the graph's first attention launch takes the set the last launch used: refill it
        hipError_t e = launch_fill_u64(reinterpret_cast<unsigned long long *>(s->graph_set0 ? s->part_o2 : s->part_o),
                                       ~0ull, (int)(s->attn_scratch / 2), st);
        if (e != hipSuccess) return e;
    }
    s->attn_set = s->graph_set1;
    return hipGraphLaunch(s->graph, st);
}

// The polled attention's error flag: set when one of its waits ran out (the
// step's outputs are then not valid); read after the stream is synchronized.
int poll_check(ZiggyHipSession *s, char *err, size_t err_len) {
    if (!s->attn_poll) return ZIGGY_HIP_OK;
    int flag = 0;
    ZH_TRY(hipMemcpy(&flag, s->poll_err, 4, hipMemcpyDeviceToHost), "poll flag");
    if (flag) return fail(err, err_len, ZIGGY_HIP_EXECUTION_FAILED, "an attention split never arrived (polled merge)");
    return ZIGGY_HIP_OK;
}

bool graphs_enabled() {
    const char *e = getenv("ZIGGY_HIP_GRAPH");
    return !(e && e[0] == '0');
}

int build_graph(ZiggyHipSession *s, char *err, size_t err_len) {
    if (!graphs_enabled()) return ZIGGY_HIP_OK;
    hipStream_t st = s->ctx->stream;
    hipGraph_t g = nullptr;
    ZH_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "graph capture begin");
    // capture runs nothing: the partials sets the graph bakes in are recorded and the
    // host's record of the last set used is put back
    const int set_before = s->attn_set;
    hipError_t e = enqueue_step(s, st);
    hipError_t e2 = hipStreamEndCapture(st, &g);
    s->graph_set0 = set_before ^ 1;
    s->graph_set1 = s->attn_set;
    s->attn_set = set_before;
    if (e != hipSuccess) {
        if (g) hipGraphDestroy(g);
        return hip_fail(e, "graph capture", err, err_len);
    }
    if (e2 != hipSuccess) return hip_fail(e2, "graph capture end", err, err_len);
    e = hipGraphInstantiate(&s->graph, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "graph instantiate", err, err_len);
    s->graph_prompt = s->prompt;
    s->graph_history = s->history;
    s->graph_v_now = s->qkv_v_now;
    return ZIGGY_HIP_OK;
}

void free_session(ZiggyHipSession *s) {
    if (!s) return;
    if (s->ctx) {
        hipSetDevice(s->ctx->device);
        hipStreamSynchronize(s->ctx->stream);
    }
    if (s->graph) hipGraphExecDestroy(s->graph);
    for (void *p : s->allocs) hipFree(p);
    if (s->st_host) hipHostFree(s->st_host);
    delete s;
}

}  // namespace

extern "C" {

int ziggy_hip_session_create(ZiggyHipContext *ctx, const ZiggyHipModelDesc *model, const ZiggyHipTensorDesc *token_embd,
                             const ZiggyHipTensorDesc *output_norm, const ZiggyHipTensorDesc *output,
                             const ZiggyHipLayerDesc *layers, ZiggyHipSession **out_session, char *err, size_t err_len) {
    if (!ctx || !model || !token_embd || !output_norm || !output || !layers || !out_session)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "null argument");
    *out_session = nullptr;
    const ZiggyHipModelDesc &md = *model;
    if (md.block_count == 0 || md.embedding_length == 0 || md.head_count == 0 || md.head_count_kv == 0 ||
        md.head_count % md.head_count_kv || md.head_count / md.head_count_kv > 8 ||
        (md.head_dim != 64 && md.head_dim != 96 && md.head_dim != 128 && md.head_dim != 256) ||
        md.rope_dim > md.head_dim || md.rope_style > 1 ||
        md.context_length == 0 || md.embedding_length % 64 || md.feed_forward_length % 64 ||
        md.embedding_length > (uint32_t)kMaxMatvecCols || md.feed_forward_length > (uint32_t)kMaxMatvecRowLen ||
        (md.head_count * md.head_dim) % 64)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "unsupported model shape");
    ZiggyHipSession *s = new (std::nothrow) ZiggyHipSession();
    if (!s) return fail(err, err_len, ZIGGY_HIP_INITIALIZATION_FAILED, "out of host memory");
    s->ctx = ctx;
    s->md = md;
    s->q_size = (int)(md.head_count * md.head_dim);
    s->kv_size = (int)(md.head_count_kv * md.head_dim);
    s->max_splits = attention_splits((int)md.head_count_kv, (int)md.context_length);
    const uint64_t H = md.embedding_length, F = md.feed_forward_length, Q = (uint64_t)s->q_size,
                   KV = (uint64_t)s->kv_size;

    // ---- weight residency: one arena, every tensor 256-byte aligned ----
    size_t off = 0;
    std::vector<std::pair<const ZiggyHipTensorDesc *, DT *>> todo;
    bool ok = take_tensor(token_embd, 0, H, true, false, &s->embd, &off, todo) &&
              take_tensor(output_norm, 1, H, true, true, &s->out_norm, &off, todo) &&
              take_tensor(output, md.vocab_size, H, true, false, &s->out, &off, todo);
    s->layers.resize(md.block_count);
    for (uint32_t l = 0; l < md.block_count && ok; l++) {
        const ZiggyHipLayerDesc &d = layers[l];
        LayerW &L = s->layers[l];
        ok = take_tensor(&d.attn_norm, 1, H, true, true, &L.attn_norm, &off, todo) &&
             take_tensor(&d.attn_q, Q, H, true, false, &L.q, &off, todo) &&
             take_tensor(&d.attn_k, KV, H, true, false, &L.k, &off, todo) &&
             take_tensor(&d.attn_v, KV, H, true, false, &L.v, &off, todo) &&
             take_tensor(&d.attn_output, H, Q, true, false, &L.o, &off, todo) &&
             take_tensor(&d.attn_q_bias, 1, Q, false, true, &L.q_bias, &off, todo) &&
             take_tensor(&d.attn_k_bias, 1, KV, false, true, &L.k_bias, &off, todo) &&
             take_tensor(&d.attn_v_bias, 1, KV, false, true, &L.v_bias, &off, todo) &&
             take_tensor(&d.attn_q_norm, 1, md.head_dim, false, true, &L.q_norm, &off, todo) &&
             take_tensor(&d.attn_k_norm, 1, md.head_dim, false, true, &L.k_norm, &off, todo) &&
             take_tensor(&d.ffn_norm, 1, H, true, true, &L.ffn_norm, &off, todo) &&
             take_tensor(&d.ffn_gate, F, H, true, false, &L.gate, &off, todo) &&
             take_tensor(&d.ffn_up, F, H, true, false, &L.up, &off, todo) &&
             take_tensor(&d.ffn_down, H, F, true, false, &L.down, &off, todo);
        // q, k and v share one launch: at most two distinct formats, Q4_K/Q6_K mixed only
        if (ok) {
            const int a = L.q.type, b = L.k.type, c = L.v.type;
            const bool uniform = a == b && b == c;
            const bool mixed = ((a == ZIGGY_HIP_TYPE_Q4_K || a == ZIGGY_HIP_TYPE_Q6_K) &&
                                (b == ZIGGY_HIP_TYPE_Q4_K || b == ZIGGY_HIP_TYPE_Q6_K) &&
                                (c == ZIGGY_HIP_TYPE_Q4_K || c == ZIGGY_HIP_TYPE_Q6_K));
            if (!uniform && !mixed) ok = false;
            // the per-head norm reduces over whole wavefronts (heads of 64, 128 or 256)
            if (md.head_dim % 64 && (L.q_norm.present || L.k_norm.present)) ok = false;
        }
    }
    if (!ok) {
        free_session(s);
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT,
                    "tensor missing, of an unsupported type, or of the wrong shape");
    }
    hipSetDevice(ctx->device);
    hipError_t e = hipMalloc(&s->arena, off);
    if (e != hipSuccess) {
        free_session(s);
        return hip_fail(e, "weight arena hipMalloc", err, err_len);
    }
    s->allocs.push_back(s->arena);
    s->arena_len = off;
    for (auto &t : todo) {
        const size_t o = reinterpret_cast<size_t>(t.second->p);
        t.second->p = s->arena + o;
        e = hipMemcpyAsync(s->arena + o, t.first->data, t.second->stride * t.second->rows, hipMemcpyHostToDevice,
                           ctx->stream);
        if (e != hipSuccess) {
            free_session(s);
            return hip_fail(e, "weight upload", err, err_len);
        }
    }

    // ---- activations, KV cache, step state ----
    s->kv_pages = (md.context_length + (1u << kKvPageShift) - 1) >> kKvPageShift;
    const size_t cache_elems = (size_t)md.block_count * ((size_t)s->kv_pages << kKvPageShift) * KV;
    const size_t logits_len = md.vocab_size > F ? md.vocab_size : F;
    // the attention partials (an even count: the polled sets are refilled as u64 words)
    const size_t attn_scratch =
        (attention_scratch_floats((int)md.head_count, (int)md.head_dim, s->max_splits) + 1) & ~(size_t)1;
    struct {
        void **p;
        size_t bytes;
    } reqs[] = {
        {(void **)&s->hidden, H * 4}, {(void **)&s->q, Q * 4}, {(void **)&s->k, KV * 4}, {(void **)&s->v, KV * 4},
        {(void **)&s->attn, Q * 4}, {(void **)&s->act, F * 4}, {(void **)&s->logits, logits_len * 4},
        {(void **)&s->part_o, attn_scratch * 4}, {(void **)&s->kc, cache_elems * 2}, {(void **)&s->vc, cache_elems * 2},
        {(void **)&s->st, sizeof(StepState)}, {(void **)&s->counters, md.head_count_kv * sizeof(unsigned)},
        {(void **)&s->rope_denom, 4 * (size_t)(md.head_dim / 2 + 1)},
        {(void **)&s->page_table, 4 * (size_t)s->kv_pages},
    };
    for (auto &r : reqs) {
        e = hipMalloc(r.p, r.bytes);
        if (e == hipSuccess) e = hipMemsetAsync(*r.p, 0, r.bytes, ctx->stream);
        if (e != hipSuccess) {
            free_session(s);
            return hip_fail(e, "session buffer allocation", err, err_len);
        }
        s->allocs.push_back(*r.p);
    }
    s->part_ml = s->part_o + (size_t)md.head_count * s->max_splits * 8 * md.head_dim;
    s->attn_scratch = attn_scratch;
    s->attn_poll = attention_poll_supported((int)md.head_dim, s->max_splits);
    if (s->attn_poll) {
        // the second partials set and the flag; both sets start all kPollEmpty
        e = hipMalloc((void **)&s->part_o2, attn_scratch * 4);
        if (e == hipSuccess) s->allocs.push_back(s->part_o2);
        if (e == hipSuccess) e = hipMalloc((void **)&s->poll_err, 4);
        if (e == hipSuccess) s->allocs.push_back(s->poll_err);
        if (e == hipSuccess) e = hipMemsetAsync(s->poll_err, 0, 4, ctx->stream);
        if (e == hipSuccess) e = hipMemsetAsync(s->part_o, 0xFF, attn_scratch * 4, ctx->stream);
        if (e == hipSuccess) e = hipMemsetAsync(s->part_o2, 0xFF, attn_scratch * 4, ctx->stream);
        if (e != hipSuccess) {
            free_session(s);
            return hip_fail(e, "attention partials allocation", err, err_len);
        }
        s->part_ml2 = s->part_o2 + (s->part_ml - s->part_o);
    }
    {
        // the q/k/v projection and the attention in one launch: every layer with a served
        // format pair and shape, the polled merge, more than one layer (ZIGGY_HIP_QKV_FUSE=0
        // keeps two launches)
        const char *env = getenv("ZIGGY_HIP_QKV_FUSE");
        bool fuse = !(env && env[0] == '0') && md.block_count >= 2 && s->attn_poll;
        for (uint32_t l = 0; l < md.block_count && fuse; l++) {
            const LayerW &W = s->layers[l];
            const int f1 = W.q.type;
            int f2 = f1;
            for (const DT *d : {&W.k, &W.v})
                if (d->type != f1) f2 = d->type;
            fuse = (W.k.type == f1 || W.k.type == f2) && (W.v.type == f1 || W.v.type == f2) &&
                   qkv_attention_supported(f1, f2, (int)H, (int)md.head_dim,
                                           (int)(md.head_count / md.head_count_kv));
        }
        if (fuse) {
            int n = 2;
            while ((md.block_count - 1) % n == 0) n++;
            const size_t bytes = (size_t)n * (Q + 2 * KV) * 4;
            e = hipMalloc((void **)&s->qkv_buf, bytes);
            if (e == hipSuccess) s->allocs.push_back(s->qkv_buf);
            if (e == hipSuccess) e = hipMemsetAsync(s->qkv_buf, 0xFF, bytes, ctx->stream);
            if (e != hipSuccess) {
                free_session(s);
                return hip_fail(e, "q/k/v sets allocation", err, err_len);
            }
            s->qkv_fuse = true;
            s->qkv_sets = n;
            s->qkv_v_now = qkv_attention_v_now(0, s->max_splits);
        }
    }
    // pages in order until the caller sets a block table
    s->pages.resize(s->kv_pages);
    for (uint32_t i = 0; i < s->kv_pages; i++) s->pages[i] = i;
    // on the session stream, after the zero fill queued there above (a copy on the
    // null stream would not be ordered after it)
    e = hipMemcpyAsync(s->page_table, s->pages.data(), 4 * (size_t)s->kv_pages, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        free_session(s);
        return hip_fail(e, "block table upload", err, err_len);
    }
    {
        const int n_rot = (int)(md.rope_dim < md.head_dim ? md.rope_dim : md.head_dim);
        std::vector<float> den((size_t)md.head_dim / 2 + 1, 1.0f);
        rope_denominators(md.rope_freq_base, n_rot, den.data());
        e = hipMemcpyAsync(s->rope_denom, den.data(), den.size() * 4, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            free_session(s);
            return hip_fail(e, "rope table upload", err, err_len);
        }
    }
    e = hipHostMalloc((void **)&s->st_host, sizeof(StepState), hipHostMallocDefault);
    if (e != hipSuccess) {
        free_session(s);
        return hip_fail(e, "pinned step state", err, err_len);
    }
    memset(s->st_host, 0, sizeof(StepState));
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        free_session(s);
        return hip_fail(e, "session upload", err, err_len);
    }
    int st = build_graph(s, err, err_len);
    if (st) {
        free_session(s);
        return st;
    }
    *out_session = s;
    return ZIGGY_HIP_OK;
}

void ziggy_hip_session_destroy(ZiggyHipSession *s) { free_session(s); }

int ziggy_hip_session_reset(ZiggyHipSession *s, char *err, size_t err_len) {
    if (!s) return ZIGGY_HIP_INVALID_ARGUMENT;
    const size_t cache_bytes = (size_t)s->md.block_count * ((size_t)s->kv_pages << kKvPageShift) * s->kv_size * 2;
    ZH_TRY(hipMemsetAsync(s->kc, 0, cache_bytes, s->ctx->stream), "reset");
    ZH_TRY(hipMemsetAsync(s->vc, 0, cache_bytes, s->ctx->stream), "reset");
    ZH_TRY(hipStreamSynchronize(s->ctx->stream), "reset");
    s->position = 0;
    s->fed.clear();
    s->fed_ok = true;
    s->logits_valid = false;
    return ZIGGY_HIP_OK;
}

uint32_t ziggy_hip_session_position(const ZiggyHipSession *s) { return s ? s->position : 0; }

int ziggy_hip_session_rewind(ZiggyHipSession *s, uint32_t position, char *err, size_t err_len) {
    if (!s) return ZIGGY_HIP_INVALID_ARGUMENT;
    if (position > s->position) {
        set_err(err, err_len, "rewind to %u: past the current position %u", position, s->position);
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    s->position = position;
    if (s->fed.size() > position) s->fed.resize(position);
    s->logits_valid = false;
    return ZIGGY_HIP_OK;
}

// ---- per-layer contract (gpu.Session) ----

int ziggy_hip_session_begin_token(ZiggyHipSession *s, const float *hidden, char *err, size_t err_len) {
    if (!s || !hidden) return ZIGGY_HIP_INVALID_ARGUMENT;
    ZH_TRY(hipMemcpyAsync(s->hidden, hidden, (size_t)s->md.embedding_length * 4, hipMemcpyHostToDevice,
                          s->ctx->stream),
           "begin_token");
    ZH_TRY(hipStreamSynchronize(s->ctx->stream), "begin_token");
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_run_attention_block(ZiggyHipSession *s, uint32_t layer, uint32_t position, char *err,
                                          size_t err_len) {
    if (!s || layer >= s->md.block_count) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "bad layer");
    if (position >= s->md.context_length) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "context overflow");
    s->fed_ok = false;  // a K/V row from a hidden state, not from a token step
    ZH_TRY(enqueue_attention_block(s, (int)layer, nullptr, (int)position, s->ctx->stream), "attention block");
    return finish_op(s->ctx, "attention block", err, err_len);
}

int ziggy_hip_session_run_ffn_block(ZiggyHipSession *s, uint32_t layer, char *err, size_t err_len) {
    if (!s || layer >= s->md.block_count) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "bad layer");
    ZH_TRY(enqueue_ffn_block(s, (int)layer, s->ctx->stream), "ffn block");
    return finish_op(s->ctx, "ffn block", err, err_len);
}

int ziggy_hip_session_run_output(ZiggyHipSession *s, float *logits, char *err, size_t err_len) {
    if (!s || !logits) return ZIGGY_HIP_INVALID_ARGUMENT;
    ZH_TRY(enqueue_output_logits(s, s->ctx->stream), "output");
    ZH_TRY(hipMemcpyAsync(logits, s->logits, (size_t)s->md.vocab_size * 4, hipMemcpyDeviceToHost, s->ctx->stream),
           "output readback");
    ZH_TRY(hipStreamSynchronize(s->ctx->stream), "output");
    s->logits_valid = true;
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_run_output_argmax(ZiggyHipSession *s, uint32_t *token, char *err, size_t err_len) {
    if (!s || !token) return ZIGGY_HIP_INVALID_ARGUMENT;
    ZH_TRY(launch_fill_u64(&s->st->argmax, 0ull, 1, s->ctx->stream), "output argmax reset");
    ZH_TRY(enqueue_kernel(s, ZIGGY_HIP_KERNEL_OUTPUT, 0, nullptr, 0, s->ctx->stream), "output argmax");
    unsigned long long k = 0;
    ZH_TRY(hipMemcpyAsync(&k, &s->st->argmax, 8, hipMemcpyDeviceToHost, s->ctx->stream), "argmax readback");
    ZH_TRY(hipStreamSynchronize(s->ctx->stream), "output argmax");
    *token = 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull);
    s->logits_valid = true;
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_read_hidden(ZiggyHipSession *s, float *out, char *err, size_t err_len) {
    if (!s || !out) return ZIGGY_HIP_INVALID_ARGUMENT;
    ZH_TRY(hipMemcpyAsync(out, s->hidden, (size_t)s->md.embedding_length * 4, hipMemcpyDeviceToHost, s->ctx->stream),
           "read_hidden");
    ZH_TRY(hipStreamSynchronize(s->ctx->stream), "read_hidden");
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_write_hidden(ZiggyHipSession *s, const float *v, char *err, size_t err_len) {
    return ziggy_hip_session_begin_token(s, v, err, err_len);
}

int ziggy_hip_session_read_kv(ZiggyHipSession *s, uint32_t layer, uint32_t pos, float *k_out, float *v_out, char *err,
                              size_t err_len) {
    if (!s || layer >= s->md.block_count || pos >= s->md.context_length || !k_out || !v_out)
        return ZIGGY_HIP_INVALID_ARGUMENT;
    std::vector<__half> tmp(2 * (size_t)s->kv_size);
    const size_t base = kv_layer_base(s, (int)layer) + kv_row_host(s, pos) * s->kv_size;
    ZH_TRY(hipMemcpyAsync(tmp.data(), s->kc + base, (size_t)s->kv_size * 2, hipMemcpyDeviceToHost, s->ctx->stream),
           "read_kv");
    ZH_TRY(hipMemcpyAsync(tmp.data() + s->kv_size, s->vc + base, (size_t)s->kv_size * 2, hipMemcpyDeviceToHost,
                          s->ctx->stream),
           "read_kv");
    ZH_TRY(hipStreamSynchronize(s->ctx->stream), "read_kv");
    for (int i = 0; i < s->kv_size; i++) {
        k_out[i] = __half2float(tmp[i]);
        v_out[i] = __half2float(tmp[s->kv_size + i]);
    }
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_set_block_table(ZiggyHipSession *s, const uint32_t *table, uint32_t count, char *err,
                                      size_t err_len) {
    if (!s || !table) return ZIGGY_HIP_INVALID_ARGUMENT;
    if (count != s->kv_pages) {
        set_err(err, err_len, "block table of %u pages; this session has %u", count, s->kv_pages);
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    std::vector<uint8_t> seen(count, 0);
    for (uint32_t i = 0; i < count; i++) {
        if (table[i] >= count || seen[table[i]]) {
            set_err(err, err_len, "block table entry %u (page %u) out of range or repeated", i, table[i]);
            return ZIGGY_HIP_INVALID_ARGUMENT;
        }
        seen[table[i]] = 1;
    }
    if (s->position != 0)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "the block table is set on an empty cache (position 0)");
    ZH_TRY(hipStreamSynchronize(s->ctx->stream), "set_block_table");
    ZH_TRY(hipMemcpy(s->page_table, table, 4 * (size_t)count, hipMemcpyHostToDevice), "set_block_table");
    s->pages.assign(table, table + count);
    return ZIGGY_HIP_OK;
}

uint32_t ziggy_hip_session_kv_pages(const ZiggyHipSession *s) { return s ? s->kv_pages : 0; }

int ziggy_hip_session_fill_kv_pattern(ZiggyHipSession *s, uint32_t position, uint64_t seed, char *err,
                                      size_t err_len) {
    if (!s) return ZIGGY_HIP_INVALID_ARGUMENT;
    if (position > s->md.context_length) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "context overflow");
    const size_t n = (size_t)position * s->kv_size;
    std::vector<__half> kb(n ? n : 1), vb(n ? n : 1);
    ZH_TRY(hipStreamSynchronize(s->ctx->stream), "fill_kv_pattern");  // the copies below are on the null stream
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + 1;
    for (uint32_t l = 0; l < s->md.block_count; l++) {
        for (size_t i = 0; i < n; i++) {
            x ^= x << 13;
            x ^= x >> 7;
            x ^= x << 17;
            const float v = (float)((int)(x >> 40 & 0x7FF) - 1024) * (1.0f / 1024.0f);
            kb[i] = __float2half(v);
            vb[i] = __float2half(-v);
        }
        const size_t base = kv_layer_base(s, (int)l);
        // a page's positions are consecutive rows: one copy per page
        const uint32_t P = 1u << kKvPageShift;
        for (uint32_t p0 = 0; p0 < position; p0 += P) {
            const size_t cnt = (size_t)std::min(P, position - p0) * s->kv_size;
            const size_t dst = base + kv_row_host(s, p0) * s->kv_size, src = (size_t)p0 * s->kv_size;
            ZH_TRY(hipMemcpy(s->kc + dst, kb.data() + src, cnt * 2, hipMemcpyHostToDevice), "fill_kv_pattern");
            ZH_TRY(hipMemcpy(s->vc + dst, vb.data() + src, cnt * 2, hipMemcpyHostToDevice), "fill_kv_pattern");
        }
    }
    s->position = position;
    s->fed.clear();
    s->fed_ok = false;  // rows not written by token steps: nothing to reuse
    s->logits_valid = false;
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_read_logits(ZiggyHipSession *s, float *out, char *err, size_t err_len) {
    if (!s || !out) return ZIGGY_HIP_INVALID_ARGUMENT;
    if (!s->logits_valid) return fail(err, err_len, ZIGGY_HIP_EXECUTION_FAILED, "no logits computed yet");
    ZH_TRY(hipMemcpyAsync(out, s->logits, (size_t)s->md.vocab_size * 4, hipMemcpyDeviceToHost, s->ctx->stream),
           "read_logits");
    ZH_TRY(hipStreamSynchronize(s->ctx->stream), "read_logits");
    return ZIGGY_HIP_OK;
}

// ---- whole steps ----

static int host_step(ZiggyHipSession *s, uint32_t token, bool output, uint32_t *next, char *err, size_t err_len) {
    if (s->position >= s->md.context_length) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "context overflow");
    if (token >= s->embd.rows) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "token id out of range");
    StepState *h = s->st_host;
    memset(h, 0, sizeof(*h));
    h->mode = 0;
    h->pos = (int)s->position;
    h->out_flag = output ? 1 : 0;
    h->token = token;
    hipStream_t st = s->ctx->stream;
    ZH_TRY(hipMemcpyAsync(s->st, h, sizeof(StepState), hipMemcpyHostToDevice, st), "step state");
    ZH_TRY(launch_step(s, st), "step graph");
    if (output) ZH_TRY(hipMemcpyAsync(h, s->st, sizeof(StepState), hipMemcpyDeviceToHost, st), "step readback");
    ZH_TRY(hipStreamSynchronize(st), "step");
    if (int pe = poll_check(s, err, err_len)) return pe;
    s->fed.resize(s->position);
    s->fed.push_back(token);
    s->position++;
    if (output) {
        s->logits_valid = true;
        if (next) *next = 0xFFFFFFFFu - (uint32_t)(h->argmax & 0xFFFFFFFFull);
    }
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_step_greedy(ZiggyHipSession *s, uint32_t token, uint32_t *out_next, char *err, size_t err_len) {
    if (!s || !out_next) return ZIGGY_HIP_INVALID_ARGUMENT;
    return host_step(s, token, true, out_next, err, err_len);
}

int ziggy_hip_session_step_no_output(ZiggyHipSession *s, uint32_t token, char *err, size_t err_len) {
    if (!s) return ZIGGY_HIP_INVALID_ARGUMENT;
    return host_step(s, token, false, nullptr, err, err_len);
}

int ziggy_hip_session_prefill_cached(ZiggyHipSession *s, const uint32_t *prompt, uint32_t prompt_len,
                                     uint32_t *out_reused, uint32_t *out_next, char *err, size_t err_len) {
    if (!s || !prompt || prompt_len == 0 || !out_reused || !out_next)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "invalid prefill_cached arguments");
    if (prompt_len > s->md.context_length) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "context overflow");
    // commonPrefixLen of the cached tokens and the prompt (model/loader.zig:2310-2313); the
    // last prompt token is always fed again, for its logits
    uint32_t matched = 0;
    if (s->fed_ok && s->fed.size() == s->position)
        while (matched < s->position && matched < prompt_len && s->fed[matched] == prompt[matched]) matched++;
    const uint32_t common = matched >= prompt_len ? prompt_len - 1 : matched;
    s->position = common;
    s->fed.resize(common);
    if (common == 0) s->fed_ok = true;  // every row from here on comes from token steps
    ZiggyHipGenerateStats st{};
    const int r = ziggy_hip_session_generate(s, prompt + common, prompt_len - common, 0, nullptr, &st, err, err_len);
    if (r != ZIGGY_HIP_OK) return r;
    *out_reused = matched;  // commonPrefixLen, as the reference reports it (reused_prompt_token_count)
    *out_next = st.next_token;
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_step_shortlist(ZiggyHipSession *s, uint32_t token, uint32_t count,
                                     ZiggyHipShortlistEntry *out, char *err, size_t err_len) {
    if (!s || !out) return ZIGGY_HIP_INVALID_ARGUMENT;
    const int V = (int)s->md.vocab_size;
    if (count == 0 || count > 64 || (int)count > V)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "shortlist length must be 1..64 and at most the vocabulary");
    if (V > 262144) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "vocabulary too large for the shortlist");
    if (!s->sl_keys) {
        ZH_TRY(hipMalloc((void **)&s->sl_keys, shortlist_scratch_keys(V) * 8), "shortlist buffers");
        s->allocs.push_back(s->sl_keys);
        ZH_TRY(hipMalloc((void **)&s->sl_entries, 64 * 8), "shortlist buffers");
        s->allocs.push_back(s->sl_entries);
    }
    const int st = host_step(s, token, false, nullptr, err, err_len);
    if (st != ZIGGY_HIP_OK) return st;
    hipStream_t sm = s->ctx->stream;
    ZH_TRY(enqueue_output_logits(s, sm), "shortlist output");
    ZH_TRY(launch_shortlist(s->logits, V, (int)count, s->sl_keys, s->sl_entries, sm), "shortlist");
    ZH_TRY(hipMemcpyAsync(out, s->sl_entries, (size_t)count * 8, hipMemcpyDeviceToHost, sm), "shortlist readback");
    ZH_TRY(hipStreamSynchronize(sm), "shortlist");
    s->logits_valid = true;
    return ZIGGY_HIP_OK;
}

}  // extern "C"

static hipError_t pass_alloc(ZiggyHipSession *s);
static hipError_t pass_enqueue(ZiggyHipSession *s, const uint32_t *tokens, int M, int pos, bool output,
                               hipStream_t st);
constexpr uint32_t kPrefillMax = 256;  // prompt rows per batched pass at most (the pass buffers' row count)
// prompt rows per batched pass (ZIGGY_HIP_PREFILL_CHUNK, 16 .. 256; a tuning knob): the whole
// buffer by default (4096 tokens: 725 ms in passes of 64, 635 in 128, 613 in 256)
static uint32_t prefill_chunk() {
    static const uint32_t v = [] {
        const char *e = getenv("ZIGGY_HIP_PREFILL_CHUNK");
        const int c = e ? atoi(e) : (int)kPrefillMax;
        return (uint32_t)(c < 16 ? 16 : c > (int)kPrefillMax ? (int)kPrefillMax : c);
    }();
    return v;
}

// Prompt rows go through batched passes on the matrix cores unless the head
// size lacks the multi-query attention or ZIGGY_HIP_PREFILL=steps asks for
// the token-by-token path.
static bool prefill_batched(const ZiggyHipSession *s) {
    static const bool steps = [] {
        const char *e = getenv("ZIGGY_HIP_PREFILL");
        return e && strcmp(e, "steps") == 0;
    }();
    return !steps && attention_multi_supported((int)s->md.head_dim);
}

extern "C" {

int ziggy_hip_session_generate(ZiggyHipSession *s, const uint32_t *prompt, uint32_t prompt_len, uint32_t steps,
                               uint32_t *out_tokens, ZiggyHipGenerateStats *stats, char *err, size_t err_len) {
    if (!s || !prompt || prompt_len == 0 || (steps && !out_tokens))
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "invalid generate arguments");
    const uint64_t total = (uint64_t)prompt_len + steps;
    if (s->position + total > s->md.context_length)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "context overflow");
    for (uint32_t i = 0; i < prompt_len; i++)
        if (prompt[i] >= s->embd.rows) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "token id out of range");
    hipStream_t st = s->ctx->stream;
    if (prompt_len > s->prompt_cap) {
        if (s->prompt) {
            hipFree(s->prompt);
            s->allocs.erase(std::find(s->allocs.begin(), s->allocs.end(), (void *)s->prompt));
        }
        ZH_TRY(hipMalloc(&s->prompt, (size_t)prompt_len * 4), "prompt buffer");
        s->allocs.push_back(s->prompt);
        s->prompt_cap = prompt_len;
    }
    if (steps > s->history_cap || !s->history) {
        if (s->history) {
            hipFree(s->history);
            s->allocs.erase(std::find(s->allocs.begin(), s->allocs.end(), (void *)s->history));
        }
        const uint32_t cap = steps ? steps : 1;
        ZH_TRY(hipMalloc(&s->history, (size_t)cap * 4), "history buffer");
        s->allocs.push_back(s->history);
        s->history_cap = cap;
    }
    // step_begin reads the prompt/history pointers baked into the graph, and
    // the fused launch's variant follows the position the decode starts at:
    // rebuild it only if either changed
    if (s->qkv_fuse) s->qkv_v_now = qkv_attention_v_now((int)(s->position + prompt_len - 1), s->max_splits);
    if (s->graph && (s->graph_prompt != s->prompt || s->graph_history != s->history ||
                     s->graph_v_now != s->qkv_v_now)) {
        hipGraphExecDestroy(s->graph);
        s->graph = nullptr;
    }
    if (!s->graph && graphs_enabled()) {
        int bst = build_graph(s, err, err_len);
        if (bst) return bst;
    }
    ZH_TRY(hipMemcpyAsync(s->prompt, prompt, (size_t)prompt_len * 4, hipMemcpyHostToDevice, st), "prompt upload");
    // every prompt row but the last in batched passes of up to prefill_chunk()
    // tokens (GEMMs on the matrix cores, multi-query causal attention), the
    // last one through the step graph for its logits; the reference feeds
    // the prompt token by token (runPrompt, model/loader.zig:1016-1036)
    const bool batched = prompt_len > 1 && prefill_batched(s);
    const uint32_t n_batched = batched ? prompt_len - 1 : 0;
    if (batched) ZH_TRY(pass_alloc(s), "prefill buffers");
    StepState *h = s->st_host;
    memset(h, 0, sizeof(*h));
    h->mode = 1;
    h->base_pos = (int)s->position;
    h->step = (int)n_batched;  // the graph's first step takes prompt[n_batched]
    h->n_prompt = (int)prompt_len;
    h->n_gen = (int)steps;
    ZH_TRY(hipMemcpyAsync(s->st, h, sizeof(StepState), hipMemcpyHostToDevice, st), "step state");
    ZH_TRY(hipStreamSynchronize(st), "generate setup");
    const uint64_t tp0 = now_ns();
    const uint32_t chunk = prefill_chunk();
    for (uint32_t off = 0; off < n_batched; off += chunk) {
        const uint32_t m = std::min(chunk, n_batched - off);
        ZH_TRY(pass_enqueue(s, s->prompt + off, (int)m, (int)(s->position + off), false, st), "prefill pass");
    }
    // prompt steps, then the timed decode steps (the decode_ns bracket of model/loader.zig:2135-2257)
    for (uint32_t i = n_batched; i < prompt_len; i++) ZH_TRY(launch_step(s, st), "prompt step");
    ZH_TRY(hipStreamSynchronize(st), "prompt");
    const uint64_t tp1 = now_ns();
    ZH_TRY(hipEventRecord(s->ctx->seq_begin, st), "generate");
    const uint64_t t0 = now_ns();
    for (uint32_t i = 0; i < steps; i++) ZH_TRY(launch_step(s, st), "decode step");
    ZH_TRY(hipEventRecord(s->ctx->seq_end, st), "generate");
    ZH_TRY(hipStreamSynchronize(st), "decode");
    const uint64_t t1 = now_ns();
    if (steps) ZH_TRY(hipMemcpy(out_tokens, s->history, (size_t)steps * 4, hipMemcpyDeviceToHost), "history");
    ZH_TRY(hipMemcpy(h, s->st, sizeof(StepState), hipMemcpyDeviceToHost), "state readback");
    if (h->error) return fail(err, err_len, ZIGGY_HIP_EXECUTION_FAILED, "a generated token was out of range");
    if (int pe = poll_check(s, err, err_len)) return pe;
    // rows of the prompt, then of each generated token but the last (still pending)
    s->fed.resize(s->position);
    s->fed.insert(s->fed.end(), prompt, prompt + prompt_len);
    s->fed.insert(s->fed.end(), out_tokens, out_tokens + steps);
    s->position += (uint32_t)total;
    s->logits_valid = true;
    if (stats) {
        float ms = 0.f;
        hipEventElapsedTime(&ms, s->ctx->seq_begin, s->ctx->seq_end);
        stats->steps = steps;
        stats->gpu_elapsed_ns = (uint64_t)((double)ms * 1e6);
        stats->wall_ns = t1 - t0;
        stats->next_token = 0xFFFFFFFFu - (uint32_t)(h->argmax & 0xFFFFFFFFull);
        stats->prompt_ns = tp1 - tp0;
    }
    return ZIGGY_HIP_OK;
}

// ---- speculative verify: a batch of tokens in one pass ----

constexpr uint32_t kVerifyMax = 16;  // tokens of one verify pass (one MFMA token tile)
constexpr uint32_t kPassMax = kPrefillMax;  // token rows of one batched pass
static_assert(kPassMax >= kVerifyMax, "a verify pass fits the pass buffers");

// Row buffers of the batched passes (verify, prompt chunks), allocated on first use.
static hipError_t pass_alloc(ZiggyHipSession *s) {
    if (s->b_hidden) return hipSuccess;
    const size_t H = s->md.embedding_length, F = s->md.feed_forward_length, Q = (size_t)s->q_size,
                 KV = (size_t)s->kv_size, M = kPassMax;
    struct {
        void **p;
        size_t bytes;
    } reqs[] = {{(void **)&s->b_hidden, M * H * 4}, {(void **)&s->b_normed, M * H * 4}, {(void **)&s->b_q, M * Q * 4},
                {(void **)&s->b_k, M * KV * 4},      {(void **)&s->b_v, M * KV * 4},      {(void **)&s->b_attn, M * Q * 4},
                {(void **)&s->b_act, M * F * 4},     {(void **)&s->b_up, M * F * 4},      {(void **)&s->b_tokens, M * 4},
                {(void **)&s->b_argmax, M * 8},     {(void **)&s->b_logits, kVerifyMax * s->md.vocab_size * 4},
                {(void **)&s->b_ss, 2 * M * 4}};
    for (auto &r : reqs) {
        hipError_t e = hipMalloc(r.p, r.bytes);
        if (e != hipSuccess) return e;
        s->allocs.push_back(*r.p);
    }
    {
        const size_t ld = (std::max(std::max(Q, F), H) + 31) / 32 * 32;
        uint8_t *base = nullptr;
        hipError_t e = hipMalloc((void **)&base, M * ld * 4 + M * (ld / 32) * 4);
        if (e != hipSuccess) return e;
        s->allocs.push_back(base);
        s->xp.hi = reinterpret_cast<uint16_t *>(base);
        s->xp.lo = s->xp.hi + M * ld;
        s->xp.sum = reinterpret_cast<float *>(s->xp.lo + M * ld);
        s->xp.ld = (int)ld;
    }
    if (attention_multi_supported((int)s->md.head_dim)) {
        const size_t slots = (size_t)s->md.head_count_kv *
                             attention_query_groups((int)s->md.head_count, (int)s->md.head_count_kv, (int)M);
        const size_t po = slots * s->max_splits * kMultiHeads * s->md.head_dim,
                     pml = slots * s->max_splits * kMultiHeads * 2;
        hipError_t e = hipMalloc((void **)&s->b_part_o, (po + pml) * 4);
        if (e != hipSuccess) return e;
        s->allocs.push_back(s->b_part_o);
        s->b_part_ml = s->b_part_o + po;
        e = hipMalloc((void **)&s->b_counters, slots * sizeof(unsigned));
        if (e != hipSuccess) return e;
        s->allocs.push_back(s->b_counters);
        e = hipMemsetAsync(s->b_counters, 0, slots * sizeof(unsigned), s->ctx->stream);  // the merge resets them
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// One batched pass of M tokens at positions pos .. pos + M - 1: embedding,
// per layer per-token RMSNorm + q/k/v GEMMs, the q/k epilogue and K/V stores
// of all M tokens then one multi-query attention launch (or, for head sizes
// the matrix-core kernel lacks, attention query by query, each storing its
// K/V row in order), o_proj / gate-up / down GEMMs with the residual adds,
// final norm and the output GEMM fused with a per-token argmax.
// ZIGGY_HIP_VERIFY_SWIGLU=fused keeps gate/up as one SWIGLU product (its
// reduction never splits); by default they are two products and SiLU * up.
static bool verify_fused_swiglu() {
    static const bool f = [] {
        const char *e = getenv("ZIGGY_HIP_VERIFY_SWIGLU");
        return e && strcmp(e, "fused") == 0;
    }();
    return f;
}

static hipError_t pass_enqueue(ZiggyHipSession *s, const uint32_t *tokens, int M, int pos, bool output,
                               hipStream_t st) {
    const ZiggyHipModelDesc &md = s->md;
    const bool fused_swiglu = verify_fused_swiglu();
    const int H = (int)md.embedding_length, F = (int)md.feed_forward_length, Q = s->q_size, KV = s->kv_size;
    const float eps = md.rms_norm_eps;
    hipError_t e = launch_embed_rows(tokens, M, s->embd.p, s->embd.stride, (int)s->embd.rows, s->embd.type, H,
                                     s->b_hidden, st);
    // Prompt chunks are deterministic: no reduction split onto the residual,
    // at most two onto cleared rows (0 + a + b is the same sum in either
    // order), none for gate/up, which store their rows; their token tiles
    // fill the chip.  Verify passes (one token
    // tile) keep the split for speed; their sums vary in the last bits.
    const bool det = !output;
    // ZIGGY_HIP_VERIFY_SPLIT: the verify pass's largest reduction split (a tuning knob)
    static const int vsplit = [] {
        const char *v = getenv("ZIGGY_HIP_VERIFY_SPLIT");
        const int n = v ? atoi(v) : 16;
        return n == 1 || n == 2 || n == 4 || n == 8 || n == 16 ? n : 16;
    }();
    const int split_add = det ? 1 : vsplit, split_clear = det ? 2 : vsplit;
    auto gemm = [&](const DT &w, const DT *w2, const float *x, int ldx, float *y, int ldy, int out,
                    const XPlanes *xp = nullptr) {
        if (e != hipSuccess) return;
        e = launch_gemm(w.type, w.p, w2 ? w2->p : nullptr, w.stride, x, ldx, y, ldy, M, (int)w.rows, (int)w.cols,
                        out, s->b_argmax, st, false, out == OUT_ADD ? split_add : split_clear, xp);
    };
    // Prompt passes of more than one token tile give the products their
    // inputs as pieces split once here: the products then take two token
    // tiles per workgroup, and no workgroup splits the rows again.  (A verify
    // pass, one token tile, lets the products split their own.)
    const bool split_in = det && M > 16 && H % 32 == 0, split_o = det && M > 16 && Q % 32 == 0,
               split_down = det && M > 16 && F % 32 == 0;
    // products of the normed rows that accumulate (OUT_ADD) onto cleared
    // outputs, or store them (no reduction split): one launch for the
    // matrices that share a format and row size
    auto multi3 = [&](const DT &a, float *ya, int lda, const DT &b, float *yb, int ldb, const DT *c, float *yc,
                      int ldc, const XPlanes *xp, bool store = false, const float *xin = nullptr,
                      const RowNorm *rn = nullptr) {
        if (e != hipSuccess) return;
        if (!xin) xin = s->b_normed;
        const DT *d[3] = {&a, &b, c};
        float *ys[3] = {ya, yb, yc};
        const int lds[3] = {lda, ldb, ldc};
        const int n = c ? 3 : 2;
        int i = 0;
        while (i < n && e == hipSuccess) {
            int j = i + 1;  // a run of matrices of one type and row size
            while (j < n && d[j]->type == d[i]->type && d[j]->stride == d[i]->stride && d[j]->cols == d[i]->cols) j++;
            const uint8_t *ws[3];
            int Ns[3];
            for (int k = i; k < j; k++) ws[k - i] = d[k]->p, Ns[k - i] = (int)d[k]->rows;
            // the deferred norm's row sums once: with the first run of matrices
            const RowNorm rn_i = rn ? RowNorm{rn->w, i == 0 ? rn->ss : nullptr} : RowNorm{};
            e = launch_gemm_multi(d[i]->type, j - i, ws, ys + i, lds + i, Ns, d[i]->stride, xin, H, M,
                                  (int)d[i]->cols, store ? OUT_STORE : OUT_ADD, st, store ? 1 : split_clear, xp,
                                  rn ? &rn_i : nullptr);
            i = j;
        }
    };
    // Verify passes defer the RMSNorms (RowNorm): the q/k/v and gate/up
    // products take hidden * norm weights and add each row's sum of squares
    // to ss_attn / ss_ffn; attention prep and SiLU * up scale their rows by
    // 1 / sqrt(ss / H + eps).  No norm launches: the rows the accumulating
    // products add onto are cleared by the launch before them (the q/k/v rows
    // and ss_attn by SiLU * up of the layer before, or here for layer 0; the
    // gate/up rows and ss_ffn by attention prep).
    bool dn = !det && s->b_counters && s->b_ss && !fused_swiglu;
    for (int l = 0; l < (int)md.block_count && dn; l++) {
        const LayerW &L = s->layers[l];
        for (const DT *d : {&L.q, &L.k, &L.v, &L.gate, &L.up})
            dn = dn && gemm_rownorm_supported(d->type, (int)d->cols, d->p, d->stride);
    }
    float *ss_attn = s->b_ss, *ss_ffn = s->b_ss ? s->b_ss + kPassMax : nullptr;
    const ZeroSpans clear_qkv{{s->b_q, s->b_k, s->b_v, ss_attn}, {(size_t)M * Q, (size_t)M * KV, (size_t)M * KV, (size_t)M}};
    const ZeroSpans clear_ffn{{s->b_act, s->b_up, ss_ffn, nullptr}, {(size_t)M * F, (size_t)M * F, (size_t)M, 0}};
    if (dn && e == hipSuccess) e = launch_zero_spans(clear_qkv, st);
    for (int l = 0; l < (int)md.block_count && e == hipSuccess; l++) {
        const LayerW &L = s->layers[l];
        if (dn) {
            const RowNorm rn{(const float *)L.attn_norm.p, ss_attn};
            multi3(L.q, s->b_q, Q, L.k, s->b_k, KV, &L.v, s->b_v, KV, nullptr, false, s->b_hidden, &rn);
        } else {
            // the norm clears the q/k/v rows, which the products then accumulate onto
            e = launch_rms_norm_rows(s->b_hidden, (const float *)L.attn_norm.p, s->b_normed, M, H, eps, st, s->b_q,
                                     (size_t)M * Q, s->b_k, (size_t)M * KV, s->b_v, (size_t)M * KV,
                                     split_in ? &s->xp : nullptr);
            multi3(L.q, s->b_q, Q, L.k, s->b_k, KV, &L.v, s->b_v, KV, split_in ? &s->xp : nullptr);
        }
        const size_t layer_base = kv_layer_base(s, l);
        if (s->b_counters && e == hipSuccess) {
            AttnParams a{};
            a.q = s->b_q;
            a.k_new = s->b_k;
            a.v_new = s->b_v;
            a.q_bias = L.q_bias.present ? (const float *)L.q_bias.p : nullptr;
            a.k_bias = L.k_bias.present ? (const float *)L.k_bias.p : nullptr;
            a.v_bias = L.v_bias.present ? (const float *)L.v_bias.p : nullptr;
            a.q_norm = L.q_norm.present ? (const float *)L.q_norm.p : nullptr;
            a.k_norm = L.k_norm.present ? (const float *)L.k_norm.p : nullptr;
            a.k_cache = s->kc + layer_base;
            a.v_cache = s->vc + layer_base;
            a.page_table = s->page_table;
            a.page_shift = kKvPageShift;
            a.head_count = (int)md.head_count;
            a.head_count_kv = (int)md.head_count_kv;
            a.head_dim = (int)md.head_dim;
            a.kv_dim = s->kv_size;
            a.position = pos;
            a.eps = eps;
            a.rope_base = md.rope_freq_base;
            a.rope_denom = s->rope_denom;
            a.rope_dim = (int)md.rope_dim;
            a.rope_style = (int)md.rope_style;
            a.ctx = (int)md.context_length;
            a.n_query = M;
            a.q_stride = Q;
            a.out_stride = Q;
            e = dn ? launch_attention_prep(a, s->b_q, st, RowScale{ss_attn, H, eps}, clear_ffn)
                   : launch_attention_prep(a, s->b_q, st);
            // plain mode over the stored rows
            a.k_new = a.v_new = nullptr;
            a.out = s->b_attn;
            a.part_o = s->b_part_o;
            a.part_ml = s->b_part_ml;
            a.counters = s->b_counters;
            a.window_start = 0;
            a.scale = 1.0f / sqrtf((float)md.head_dim);
            a.max_splits = s->max_splits;
            if (e == hipSuccess) e = launch_attention(a, st);
        }
        // token by token where the multi-query kernel does not serve the shape (head_dim 256, the
        // vector kernel): never with the polled merge, which needs the matrix-core kernel too
        for (int m = 0; m < M && e == hipSuccess && !s->b_counters; m++) {
            AttnParams a{};
            a.q = s->b_q + (size_t)m * Q;
            a.k_new = s->b_k + (size_t)m * KV;
            a.v_new = s->b_v + (size_t)m * KV;
            a.q_bias = L.q_bias.present ? (const float *)L.q_bias.p : nullptr;
            a.k_bias = L.k_bias.present ? (const float *)L.k_bias.p : nullptr;
            a.v_bias = L.v_bias.present ? (const float *)L.v_bias.p : nullptr;
            a.q_norm = L.q_norm.present ? (const float *)L.q_norm.p : nullptr;
            a.k_norm = L.k_norm.present ? (const float *)L.k_norm.p : nullptr;
            a.k_cache = s->kc + layer_base;
            a.v_cache = s->vc + layer_base;
            a.page_table = s->page_table;
            a.page_shift = kKvPageShift;
            a.out = s->b_attn + (size_t)m * Q;
            a.part_o = s->part_o;
            a.part_ml = s->part_ml;
            a.counters = s->counters;
            a.head_count = (int)md.head_count;
            a.head_count_kv = (int)md.head_count_kv;
            a.head_dim = (int)md.head_dim;
            a.kv_dim = s->kv_size;
            a.position = pos + m;
            a.window_start = 0;
            a.scale = 1.0f / sqrtf((float)md.head_dim);
            a.max_splits = s->max_splits;
            a.eps = eps;
            a.rope_base = md.rope_freq_base;
            a.rope_denom = s->rope_denom;
            a.rope_dim = (int)md.rope_dim;
            a.rope_style = (int)md.rope_style;
            a.ctx = (int)md.context_length;
            e = launch_attention(a, st);
        }
        if (split_o && e == hipSuccess) e = launch_split_rows(s->b_attn, Q, M, Q, s->xp, st);
        gemm(L.o, nullptr, s->b_attn, Q, s->b_hidden, H, OUT_ADD, split_o ? &s->xp : nullptr);
        bool down_split = false;
        if (dn) {
            const RowNorm rn{(const float *)L.ffn_norm.p, ss_ffn};
            multi3(L.gate, s->b_act, F, L.up, s->b_up, F, nullptr, nullptr, 0, nullptr, false, s->b_hidden, &rn);
            if (e == hipSuccess) e = launch_silu_mul_rows(s->b_act, s->b_up, M, F, RowScale{ss_ffn, H, eps}, clear_qkv, st);
        } else if (fused_swiglu && L.gate.type == L.up.type) {
            if (e == hipSuccess)
                e = launch_rms_norm_rows(s->b_hidden, (const float *)L.ffn_norm.p, s->b_normed, M, H, eps, st);
            gemm(L.gate, &L.up, s->b_normed, H, s->b_act, F, OUT_SWIGLU);
        } else {
            // gate and up (prompt chunks: stores; verify passes: onto rows
            // the norm clears, each product may split its reduction), then
            // SiLU(gate) * up
            if (e == hipSuccess)
                e = launch_rms_norm_rows(s->b_hidden, (const float *)L.ffn_norm.p, s->b_normed, M, H, eps, st,
                                         det ? nullptr : s->b_act, det ? 0 : (size_t)M * F, det ? nullptr : s->b_up,
                                         det ? 0 : (size_t)M * F, nullptr, 0, split_in ? &s->xp : nullptr);
            multi3(L.gate, s->b_act, F, L.up, s->b_up, F, nullptr, nullptr, 0, split_in ? &s->xp : nullptr, det);
            down_split = split_down;
            if (e == hipSuccess)
                e = down_split ? launch_silu_mul_split(s->b_act, s->b_up, M, F, s->xp, st)
                               : launch_silu_mul(s->b_act, s->b_up, M * F, st);
        }
        gemm(L.down, nullptr, s->b_act, F, s->b_hidden, H, OUT_ADD, down_split ? &s->xp : nullptr);
    }
    if (!output) return e;  // a prompt chunk: K/V rows only
    // the final norm also clears the argmax keys; the output product stores
    // the logits (its reduction may split), then a per-token argmax
    if (e == hipSuccess)
        e = launch_rms_norm_rows(s->b_hidden, (const float *)s->out_norm.p, s->b_normed, M, H, eps, st,
                                 reinterpret_cast<float *>(s->b_argmax), (size_t)M * 2);
    const int V = (int)md.vocab_size;
    gemm(s->out, nullptr, s->b_normed, H, s->b_logits, V, OUT_STORE);
    if (e == hipSuccess) e = launch_argmax_rows(s->b_logits, M, (int)s->out.rows, V, s->b_argmax, st);
    return e;
}

int ziggy_hip_session_verify(ZiggyHipSession *s, uint32_t current_token, const uint32_t *drafts, uint32_t draft_count,
                             uint32_t *out_predicted, uint32_t *out_count, char *err, size_t err_len) {
    if (!s || !out_predicted || !out_count || (draft_count && !drafts))
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "null argument");
    const uint32_t M = draft_count + 1;
    if (M > kVerifyMax) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "at most 15 draft tokens");
    if (s->position + M > s->md.context_length) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "context overflow");
    uint32_t toks[kVerifyMax];
    toks[0] = current_token;
    for (uint32_t i = 0; i < draft_count; i++) toks[i + 1] = drafts[i];
    for (uint32_t i = 0; i < M; i++)
        if (toks[i] >= s->embd.rows) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "token id out of range");
    hipStream_t st = s->ctx->stream;
    ZH_TRY(pass_alloc(s), "verify buffers");
    ZH_TRY(hipMemcpyAsync(s->b_tokens, toks, M * 4, hipMemcpyHostToDevice, st), "verify tokens");
    ZH_TRY(pass_enqueue(s, s->b_tokens, (int)M, (int)s->position, true, st), "verify");
    unsigned long long keys[kVerifyMax];
    ZH_TRY(hipMemcpyAsync(keys, s->b_argmax, M * 8, hipMemcpyDeviceToHost, st), "verify readback");
    ZH_TRY(hipStreamSynchronize(st), "verify");
    // verifyDraftTokensSequential (model/loader.zig:1131-1151): emit predictions until one
    // differs from its draft; all drafts accepted adds the bonus prediction
    for (uint32_t i = 0; i < M; i++) out_predicted[i] = 0xFFFFFFFFu - (uint32_t)(keys[i] & 0xFFFFFFFFull);
    uint32_t n = 0;
    for (uint32_t i = 0; i < M; i++) {
        n = i + 1;
        if (i < draft_count && out_predicted[i] != drafts[i]) break;
    }
    *out_count = n;
    s->fed.resize(s->position);
    s->fed.insert(s->fed.end(), toks, toks + n);  // the current token and the accepted drafts
    s->position += n;
    s->logits_valid = false;
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_time_kernel(ZiggyHipSession *s, uint32_t kernel, uint32_t iterations, uint64_t *avg_ns,
                                  uint64_t *bytes_per_launch, char *err, size_t err_len) {
    if (!s || kernel > ZIGGY_HIP_KERNEL_QKV_ATTENTION || iterations == 0 || !avg_ns || !bytes_per_launch)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "invalid time_kernel arguments");
    const bool fused = kernel == ZIGGY_HIP_KERNEL_QKV_ATTENTION;
    if (fused && !s->qkv_fuse)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "the session runs q/k/v and the attention separately");
    if (s->position >= s->md.context_length)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "no free cache row to time at");
    const int pos = (int)s->position, L = (int)s->md.block_count;
    hipStream_t st = s->ctx->stream;
    hipEvent_t e0, e1;
    ZH_TRY(hipEventCreate(&e0), "time_kernel");
    if (hipEventCreate(&e1) != hipSuccess) {
        hipEventDestroy(e0);
        return fail(err, err_len, ZIGGY_HIP_EXECUTION_FAILED, "event creation failed");
    }
    // one warm-up launch, then `iterations` back-to-back launches (rotating
    // over the layers so weights stream from HBM) between one event pair.
    // The fused launch's q/k/v sets assume layers in order from layer 0: its
    // launches end on the last layer, which re-arms layer 0's set.
    if (fused) iterations = ((iterations + (uint32_t)L) / (uint32_t)L) * (uint32_t)L - 1;
    auto launch = [&](int l) {
        return fused ? launch_qkv_attention_layer(s, l, nullptr, pos, st)
                     : enqueue_kernel(s, (int)kernel, l, nullptr, pos, st);
    };
    uint64_t bytes = 0;
    float ms = 0.f;
    hipError_t e = launch(0);
    if (e == hipSuccess) e = hipEventRecord(e0, st);
    for (uint32_t i = 0; i < iterations && e == hipSuccess; i++) {
        const int l = (int)((i + 1) % (uint32_t)L);
        e = launch(l);
        bytes += fused ? kernel_bytes(s, ZIGGY_HIP_KERNEL_QKV, l, pos) + kernel_bytes(s, ZIGGY_HIP_KERNEL_ATTENTION, l, pos)
                       : kernel_bytes(s, (int)kernel, l, pos);
    }
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (e != hipSuccess) return hip_fail(e, "time_kernel", err, err_len);
    *avg_ns = (uint64_t)((double)ms * 1e6 / iterations);
    *bytes_per_launch = bytes / iterations;
    return ZIGGY_HIP_OK;
}

int ziggy_hip_session_profile_decode(ZiggyHipSession *s, uint32_t token, uint32_t steps, uint32_t *out_tokens,
                                     ZiggyHipProfileRecord *records, size_t capacity, size_t *out_count, char *err,
                                     size_t err_len) {
    if (!s || !steps || !out_tokens || !out_count)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "invalid profile_decode arguments");
    const ZiggyHipModelDesc &md = s->md;
    const int L = (int)md.block_count;
    // the step's launches per layer: q/k/v, attention, o, gate/up, down (q/k/v with the attention when fused)
    const int per_layer = s->qkv_fuse ? 4 : 5;
    const size_t per_step = (size_t)per_layer * L + 7;  // markers, step begin, the layers', output, wait, gpu, readback
    *out_count = per_step * steps;
    if (!records || capacity < per_step * steps)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "profile record buffer too small");
    if ((uint64_t)s->position + steps > md.context_length)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "context overflow");
    if (token >= s->embd.rows) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "token id out of range");
    *out_count = 0;
    hipStream_t st = s->ctx->stream;
    const int nev = per_layer * L + 3;  // before the step, after the step begin, after each launch
    std::vector<hipEvent_t> ev(nev, nullptr);
    hipError_t e = hipSuccess;
    for (int i = 0; i < nev && e == hipSuccess; i++) e = hipEventCreate(&ev[i]);
    auto release = [&] {
        for (hipEvent_t x : ev)
            if (x) hipEventDestroy(x);
    };
    if (e != hipSuccess) {
        release();
        return hip_fail(e, "profile events", err, err_len);
    }
    const int H = (int)md.embedding_length;
    // the op of each launch, under the reference's category and shape
    struct Op {
        uint32_t kind;
        uint64_t rows, cols, depth, extra;
        uint32_t type;
    };
    const Op argmax_shape{ZIGGY_HIP_PROFILE_OUTPUT_REDUCE, 1, 1, md.vocab_size, 0, (uint32_t)s->out.type};
    size_t n = 0;
    auto put = [&](uint32_t kind, uint64_t ns, const Op *shape) {
        ZiggyHipProfileRecord &r = records[n++];
        r = ZiggyHipProfileRecord{};
        r.kind = kind;
        r.ns = ns;
        if (shape) {
            r.has_shape = 1;
            r.rows = shape->rows, r.cols = shape->cols, r.depth = shape->depth, r.extra = shape->extra;
            r.tensor_type = shape->type;
        }
    };
    constexpr int kQkvAttn = -1;  // the q/k/v projection and the attention in one launch
    const int kSeparate[5] = {ZIGGY_HIP_KERNEL_QKV, ZIGGY_HIP_KERNEL_ATTENTION, ZIGGY_HIP_KERNEL_O_PROJ,
                              ZIGGY_HIP_KERNEL_GATE_UP, ZIGGY_HIP_KERNEL_DOWN};
    const int kFused[4] = {kQkvAttn, ZIGGY_HIP_KERNEL_O_PROJ, ZIGGY_HIP_KERNEL_GATE_UP, ZIGGY_HIP_KERNEL_DOWN};
    const int *kLayerKernels = s->qkv_fuse ? kFused : kSeparate;
    std::vector<Op> ops(nev - 1);
    for (uint32_t t = 0; t < steps && e == hipSuccess; t++) {
        const int pos = (int)s->position;
        StepState *h = s->st_host;
        memset(h, 0, sizeof(*h));
        h->pos = pos;
        h->out_flag = 1;
        h->token = token;
        e = hipMemcpyAsync(s->st, h, sizeof(StepState), hipMemcpyHostToDevice, st);
        // the step's launches (enqueue_step's order), an event after each
        int k = 0;
        if (e == hipSuccess) e = hipEventRecord(ev[k], st);
        if (e == hipSuccess)
            e = launch_step_begin(s->st, s->prompt, s->history, s->embd.p, s->embd.stride, (int)s->embd.rows,
                                  s->embd.type, H, s->hidden, st);
        ops[k] = Op{ZIGGY_HIP_PROFILE_ELEMENTWISE_OPS, 1, (uint64_t)H, 0, 0, 0};
        if (e == hipSuccess) e = hipEventRecord(ev[++k], st);
        for (int l = 0; l < L && e == hipSuccess; l++) {
            const LayerW &W = s->layers[l];
            for (int j = 0; j < per_layer; j++) {
                const int id = kLayerKernels[j];
                if (e == hipSuccess) {
                    // the fused launch alone (enqueue_attention_step without its o_proj)
                    if (id == kQkvAttn) e = launch_qkv_attention_layer(s, l, &s->st->pos, 0, st);
                    else e = enqueue_kernel(s, id, l, &s->st->pos, 0, st);
                }
                switch (id) {
                case ZIGGY_HIP_KERNEL_QKV:
                    ops[k] = Op{ZIGGY_HIP_PROFILE_PROJECTIONS, W.q.rows + W.k.rows + W.v.rows, W.q.cols, 0, 3,
                                (uint32_t)W.q.type};
                    break;
                case ZIGGY_HIP_KERNEL_ATTENTION:  // session.zig:445-450
                case kQkvAttn:                    // (with the q/k/v projection inside)
                    ops[k] = Op{ZIGGY_HIP_PROFILE_ATTENTION, md.head_count, md.rope_dim, (uint64_t)pos + 1,
                                md.head_count_kv, 0};
                    break;
                case ZIGGY_HIP_KERNEL_O_PROJ:
                    ops[k] = Op{ZIGGY_HIP_PROFILE_PROJECTIONS, W.o.rows, W.o.cols, 0, 0, (uint32_t)W.o.type};
                    break;
                case ZIGGY_HIP_KERNEL_GATE_UP:  // the pair and its SwiGLU
                    ops[k] = Op{ZIGGY_HIP_PROFILE_PROJECTIONS, W.gate.rows, W.gate.cols, 0, 2, (uint32_t)W.gate.type};
                    break;
                default:
                    ops[k] = Op{ZIGGY_HIP_PROFILE_PROJECTIONS, W.down.rows, W.down.cols, 0, 0, (uint32_t)W.down.type};
                    break;
                }
                if (e == hipSuccess) e = hipEventRecord(ev[++k], st);
            }
        }
        if (e == hipSuccess) e = enqueue_kernel(s, ZIGGY_HIP_KERNEL_OUTPUT, 0, &s->st->pos, 0, st);
        ops[k] = argmax_shape;
        if (e == hipSuccess) e = hipEventRecord(ev[++k], st);
        // commit and wait (commitOutputSequence), then read the token back
        const auto w0 = std::chrono::steady_clock::now();
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        const auto w1 = std::chrono::steady_clock::now();
        if (e == hipSuccess) e = hipMemcpy(h, s->st, sizeof(StepState), hipMemcpyDeviceToHost);
        const auto w2 = std::chrono::steady_clock::now();
        if (e != hipSuccess) break;
        if (int pe = poll_check(s, err, err_len)) {
            release();
            return pe;
        }
        put(ZIGGY_HIP_PROFILE_TOKEN_BEGIN, 0, nullptr);
        for (int i = 0; i < k && e == hipSuccess; i++) {
            float ms = 0.f;
            e = hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
            put(ops[i].kind, (uint64_t)((double)ms * 1e6), &ops[i]);
        }
        float total_ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&total_ms, ev[0], ev[k]);
        if (e != hipSuccess) break;
        Op wait_shape = argmax_shape;
        wait_shape.kind = ZIGGY_HIP_PROFILE_COMMIT_WAIT;
        put(ZIGGY_HIP_PROFILE_COMMIT_WAIT,
            (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(w1 - w0).count(), &wait_shape);
        put(ZIGGY_HIP_PROFILE_COMMIT_WAIT_GPU, (uint64_t)((double)total_ms * 1e6), nullptr);
        Op rb_shape = argmax_shape;
        rb_shape.kind = ZIGGY_HIP_PROFILE_HOST_READBACK;
        put(ZIGGY_HIP_PROFILE_HOST_READBACK,
            (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(w2 - w1).count(), &rb_shape);
        put(ZIGGY_HIP_PROFILE_TOKEN_END, 0, nullptr);
        *out_count = n;
        s->fed.resize(s->position);
        s->fed.push_back(token);
        s->position++;
        s->logits_valid = true;
        token = 0xFFFFFFFFu - (uint32_t)(h->argmax & 0xFFFFFFFFull);
        out_tokens[t] = token;
    }
    release();
    if (e != hipSuccess) return hip_fail(e, "profile_decode", err, err_len);
    return ZIGGY_HIP_OK;
}

}  // extern "C"
