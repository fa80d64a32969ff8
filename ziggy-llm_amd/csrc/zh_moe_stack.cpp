// zh_moe_stack.cpp -- host side of the MoE FFN layer stack (ziggy_hip_moe_stack_*):
// weight residency, buffers, and the per-layer launch sequence of zh_moe.hip
// captured into one HIP graph.
#include <new>
#include <vector>

#include "zh_arena.h"
#include "zh_internal.h"

using namespace zh;

namespace {

struct MoeLayerW {
    DT norm, router, gate, up, down, gate_sh, up_sh, down_sh, gate_inp_sh;
};

}  // namespace

struct ZiggyHipMoeStack {
    ZiggyHipContext *ctx = nullptr;
    ZiggyHipMoeDesc d{};
    std::vector<MoeLayerW> layers;
    uint8_t *arena = nullptr;
    float *hidden = nullptr, *logits = nullptr, *act = nullptr, *tmp = nullptr;
    uint32_t *route = nullptr;  // [layers][2k + 2]
    int act_stride = 0, route_stride = 0;
    bool shared = false, shared_gate = false;
    hipGraphExec_t graph = nullptr;
    std::vector<void *> allocs;
};

namespace {

int fail(char *err, size_t err_len, int code, const char *msg) {
    set_err(err, err_len, "%s", msg);
    return code;
}

void free_stack(ZiggyHipMoeStack *s) {
    if (!s) return;
    if (s->ctx) {
        hipSetDevice(s->ctx->device);
        hipStreamSynchronize(s->ctx->stream);
    }
    if (s->graph) hipGraphExecDestroy(s->graph);
    for (void *p : s->allocs) hipFree(p);
    delete s;
}

MvSeg seg_of(const DT &t, float *y) {
    MvSeg g{};
    g.w = t.p;
    g.stride = t.stride;
    g.y = y;
    g.rows = (int)t.rows;
    g.fmt = t.type;
    g.expert_slot = -1;
    return g;
}

// One layer's five launches (see zh_moe.hip).
hipError_t enqueue_layer(ZiggyHipMoeStack *s, int l, hipStream_t st) {
    const MoeLayerW &L = s->layers[l];
    const ZiggyHipMoeDesc &d = s->d;
    const int H = (int)d.hidden, E = (int)d.expert_count, K = (int)d.expert_used_count, FF = (int)d.expert_ff_length;
    uint32_t *route = s->route + (size_t)l * s->route_stride;
    // router (+ the shared expert's gate row) on the normed hidden state
    {
        MvParams p{};
        p.nseg = 1;
        p.seg[0] = seg_of(L.router, s->logits);
        if (s->shared_gate) {
            p.seg[1] = seg_of(L.gate_inp_sh, s->logits + E);
            p.nseg = 2;
        }
        p.cols = H;
        p.x = s->hidden;
        p.norm_w = (const float *)L.norm.p;
        p.eps = d.rms_norm_eps;
        hipError_t e = launch_matvec(p, IN_NORM, OUT_STORE, st);
        if (e != hipSuccess) return e;
    }
    hipError_t e = launch_moe_route(s->logits, E, K, (int)d.gating_func, (int)d.weights_norm, d.weights_scale,
                                    s->shared_gate ? 1 : 0, route, st);
    if (e != hipSuccess) return e;
    // routed experts' gate/up (+ shared), SiLU(gate) * up
    {
        MvParams p{};
        for (int k = 0; k < K; k++) {
            p.seg[k] = seg_of(L.gate, s->act + (size_t)k * s->act_stride);
            p.seg[k].rows = FF;
            p.seg[k].w2 = L.up.p;
            p.seg[k].expert_slot = k;
        }
        p.nseg = K;
        if (s->shared) {
            p.seg[K] = seg_of(L.gate_sh, s->act + (size_t)K * s->act_stride);
            p.seg[K].w2 = L.up_sh.p;
            p.nseg = K + 1;
        }
        p.cols = H;
        p.x = s->hidden;
        p.norm_w = (const float *)L.norm.p;
        p.eps = d.rms_norm_eps;
        p.expert = route;
        p.rows_per_expert = FF;
        p.expert_limit = E;
        e = launch_matvec(p, IN_NORM, OUT_SWIGLU, st);
        if (e != hipSuccess) return e;
    }
    // down projections, each of its own activation row
    {
        MvParams p{};
        for (int k = 0; k < K; k++) {
            p.seg[k] = seg_of(L.down, s->tmp + (size_t)k * H);
            p.seg[k].rows = H;
            p.seg[k].x = s->act + (size_t)k * s->act_stride;
            p.seg[k].expert_slot = k;
        }
        p.nseg = K;
        const bool same_cols = (int)d.shared_ff_length == FF;
        if (s->shared && same_cols) {
            p.seg[K] = seg_of(L.down_sh, s->tmp + (size_t)K * H);
            p.seg[K].x = s->act + (size_t)K * s->act_stride;
            p.nseg = K + 1;
        }
        p.cols = FF;
        p.expert = route;
        p.rows_per_expert = H;
        p.expert_limit = E;
        e = launch_matvec(p, IN_PLAIN, OUT_STORE, st);
        if (e != hipSuccess) return e;
        if (s->shared && !same_cols) {
            MvParams q{};
            q.seg[0] = seg_of(L.down_sh, s->tmp + (size_t)K * H);
            q.seg[0].x = s->act + (size_t)K * s->act_stride;
            q.nseg = 1;
            q.cols = (int)d.shared_ff_length;
            e = launch_matvec(q, IN_PLAIN, OUT_STORE, st);
            if (e != hipSuccess) return e;
        }
    }
    return launch_moe_combine(s->hidden, s->tmp, route, H, K, s->shared ? 1 : 0, st);
}

hipError_t enqueue_stack(ZiggyHipMoeStack *s, hipStream_t st) {
    for (int l = 0; l < (int)s->layers.size(); l++) {
        hipError_t e = enqueue_layer(s, l, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

extern "C" {

int ziggy_hip_moe_stack_create(ZiggyHipContext *ctx, const ZiggyHipMoeDesc *desc, const ZiggyHipMoeLayerDesc *layers,
                               uint32_t layer_count, ZiggyHipMoeStack **out_stack, char *err, size_t err_len) {
    if (!ctx || !desc || !layers || !out_stack || layer_count == 0)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "null argument");
    *out_stack = nullptr;
    const ZiggyHipMoeDesc &d = *desc;
    const uint64_t H = d.hidden, E = d.expert_count, K = d.expert_used_count, FF = d.expert_ff_length,
                   SF = d.shared_ff_length;
    if (H == 0 || H % 64 || H / 64 > 256 || E == 0 || E > 1024 || K == 0 || K > 8 || K > E || FF == 0 || FF % 64 ||
        FF / 64 > 256 || SF % 64 || SF / 64 > 256 || d.gating_func > 2)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "unsupported MoE shape");
    ZiggyHipMoeStack *s = new (std::nothrow) ZiggyHipMoeStack();
    if (!s) return fail(err, err_len, ZIGGY_HIP_INITIALIZATION_FAILED, "out of host memory");
    s->ctx = ctx;
    s->d = d;
    s->layers.resize(layer_count);
    size_t off = 0;
    ArenaTodo todo;
    bool ok = true;
    for (uint32_t l = 0; l < layer_count && ok; l++) {
        const ZiggyHipMoeLayerDesc &t = layers[l];
        MoeLayerW &L = s->layers[l];
        ok = take_tensor(&t.ffn_norm, 1, H, true, true, &L.norm, &off, todo) &&
             take_tensor(&t.router, E, H, true, false, &L.router, &off, todo) &&
             take_tensor(&t.gate_exps, E * FF, H, true, false, &L.gate, &off, todo) &&
             take_tensor(&t.up_exps, E * FF, H, true, false, &L.up, &off, todo) &&
             take_tensor(&t.down_exps, E * H, FF, true, false, &L.down, &off, todo) &&
             take_tensor(&t.gate_shexp, SF, H, false, false, &L.gate_sh, &off, todo) &&
             take_tensor(&t.up_shexp, SF, H, false, false, &L.up_sh, &off, todo) &&
             take_tensor(&t.down_shexp, H, SF, false, false, &L.down_sh, &off, todo) &&
             take_tensor(&t.gate_inp_shexp, 1, H, false, false, &L.gate_inp_sh, &off, todo);
        if (!ok) break;
        // the same routed / shared / router types in every layer, launched together
        const bool sh = L.gate_sh.present;
        if (l == 0) {
            s->shared = sh && SF > 0;
            s->shared_gate = L.gate_inp_sh.present;
        }
        ok = L.gate.type == L.up.type && L.gate.type == L.down.type && sh == s->shared &&
             L.gate_inp_sh.present == s->shared_gate && (!sh || (L.up_sh.present && L.down_sh.present &&
                                                                 L.gate_sh.type == L.up_sh.type &&
                                                                 L.gate_sh.type == L.down_sh.type)) &&
             (!s->shared_gate || L.gate_inp_sh.type == L.router.type);
        // routed + shared in one launch: one format, or IQ4_XS routed with Q3_K shared
        if (ok && sh && L.gate_sh.type != L.gate.type)
            ok = L.gate.type == ZIGGY_HIP_TYPE_IQ4_XS && L.gate_sh.type == ZIGGY_HIP_TYPE_Q3_K;
    }
    if (!ok) {
        free_stack(s);
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "MoE tensor missing, of an unsupported type, or of the wrong shape");
    }
    hipSetDevice(ctx->device);
    hipError_t e = hipMalloc(&s->arena, off ? off : 256);
    if (e != hipSuccess) {
        free_stack(s);
        return hip_fail(e, "MoE weight arena hipMalloc", err, err_len);
    }
    s->allocs.push_back(s->arena);
    for (auto &t : todo) {
        const size_t o = reinterpret_cast<size_t>(t.second->p);
        t.second->p = s->arena + o;
        e = hipMemcpyAsync(s->arena + o, t.first->data, t.second->stride * t.second->rows, hipMemcpyHostToDevice,
                           ctx->stream);
        if (e != hipSuccess) {
            free_stack(s);
            return hip_fail(e, "MoE weight upload", err, err_len);
        }
    }
    s->act_stride = (int)(FF > SF ? FF : SF);
    s->route_stride = (int)(2 * K + 2);
    struct {
        void **p;
        size_t bytes;
    } reqs[] = {
        {(void **)&s->hidden, H * 4},
        {(void **)&s->logits, (E + 1) * 4},
        {(void **)&s->act, (K + 1) * (size_t)s->act_stride * 4},
        {(void **)&s->tmp, (K + 1) * H * 4},
        {(void **)&s->route, (size_t)layer_count * s->route_stride * 4},
    };
    for (auto &r : reqs) {
        e = hipMalloc(r.p, r.bytes);
        if (e == hipSuccess) e = hipMemsetAsync(*r.p, 0, r.bytes, ctx->stream);
        if (e != hipSuccess) {
            free_stack(s);
            return hip_fail(e, "MoE buffer allocation", err, err_len);
        }
        s->allocs.push_back(*r.p);
    }
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        free_stack(s);
        return hip_fail(e, "MoE upload", err, err_len);
    }
    // capture every layer once; each forward replays the graph
    hipStream_t st = ctx->stream;
    hipGraph_t g = nullptr;
    e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
    if (e == hipSuccess) {
        hipError_t e1 = enqueue_stack(s, st);
        hipError_t e2 = hipStreamEndCapture(st, &g);
        e = e1 != hipSuccess ? e1 : e2;
    }
    if (e == hipSuccess) e = hipGraphInstantiate(&s->graph, g, nullptr, nullptr, 0);
    if (g) hipGraphDestroy(g);
    if (e != hipSuccess) {
        free_stack(s);
        return hip_fail(e, "MoE graph capture", err, err_len);
    }
    *out_stack = s;
    return ZIGGY_HIP_OK;
}

void ziggy_hip_moe_stack_destroy(ZiggyHipMoeStack *s) { free_stack(s); }

int ziggy_hip_moe_stack_forward(ZiggyHipMoeStack *s, const float *hidden_in, float *hidden_out, uint32_t *selected,
                                float *weights, char *err, size_t err_len) {
    if (!s || !hidden_in || !hidden_out) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "null argument");
    hipStream_t st = s->ctx->stream;
    const size_t H = s->d.hidden, K = s->d.expert_used_count, NL = s->layers.size();
    ZH_TRY(hipMemcpyAsync(s->hidden, hidden_in, H * 4, hipMemcpyHostToDevice, st), "MoE input");
    ZH_TRY(hipGraphLaunch(s->graph, st), "MoE stack");
    ZH_TRY(hipMemcpyAsync(hidden_out, s->hidden, H * 4, hipMemcpyDeviceToHost, st), "MoE output");
    std::vector<uint32_t> r;
    if (selected || weights) {
        r.resize(NL * s->route_stride);
        ZH_TRY(hipMemcpyAsync(r.data(), s->route, r.size() * 4, hipMemcpyDeviceToHost, st), "MoE routing");
    }
    ZH_TRY(hipStreamSynchronize(st), "MoE stack");
    for (size_t l = 0; l < r.size() / s->route_stride; l++)
        for (size_t k = 0; k < K; k++) {
            const uint32_t *e = &r[l * s->route_stride + 2 * k];
            if (selected) selected[l * K + k] = e[0];
            if (weights) memcpy(&weights[l * K + k], &e[1], 4);
        }
    return ZIGGY_HIP_OK;
}

int ziggy_hip_moe_stack_time(ZiggyHipMoeStack *s, uint32_t iterations, uint64_t *avg_ns, char *err, size_t err_len) {
    if (!s || !iterations || !avg_ns) return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "invalid arguments");
    hipStream_t st = s->ctx->stream;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    ZH_TRY(hipEventCreate(&e0), "MoE time");
    hipError_t e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipGraphLaunch(s->graph, st);  // warm-up
    if (e == hipSuccess) e = hipEventRecord(e0, st);
    for (uint32_t i = 0; i < iterations && e == hipSuccess; i++) e = hipGraphLaunch(s->graph, st);
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (e != hipSuccess) return hip_fail(e, "MoE time", err, err_len);
    *avg_ns = (uint64_t)((double)ms * 1e6 / iterations);
    return ZIGGY_HIP_OK;
}

}  // extern "C"
