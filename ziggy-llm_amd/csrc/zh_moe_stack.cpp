// zh_moe_stack.cpp -- host side of the MoE FFN layer stack (ziggy_hip_moe_stack_*):
// weight residency, buffers, and the per-layer launch sequence of zh_moe.hip
// captured into one HIP graph.
#include <algorithm>
#include <cstdlib>
#include <new>
#include <vector>

#include "zh_arena.h"
#include "zh_internal.h"
#include "zh_route.h"

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
    // fuse_combine: layer l > 0's router launch runs layer l - 1's combine,
    // from the hidden state of layer l - 1 into the other of two buffers
    // (hidden, hidden2); the buffers alternate so that the last layer's is
    // `hidden`, where its own combine kernel runs in place
    float *hidden2 = nullptr;
    bool fuse_combine = false;
    uint32_t *route = nullptr;  // [layers][2k + 2]
    int act_stride = 0, route_stride = 0;
    // fuse_ffn: each layer's gate/up and down run as one launch
    // (launch_moe_ffn).  The act rows then come in act_sets sets, layer l
    // using set l % act_sets, every word kPollEmpty until published; layer l's
    // launch refills the set of layer l + 1 (cyclically), which differs from
    // its own: act_sets is the smallest n >= 2 with (layers - 1) % n != 0.
    bool fuse_ffn = false;
    int act_sets = 1;
    int *poll_err = nullptr;
    bool shared = false, shared_gate = false;
    hipGraphExec_t graph = nullptr;
    std::vector<void *> allocs;
    // prefill (token batches of up to pre_max rows), allocated at the first call
    int pre_max = 0;
    float *p_input = nullptr, *p_hidden = nullptr, *p_normed = nullptr, *p_logits = nullptr, *p_act = nullptr,
          *p_act_sh = nullptr, *p_tmp = nullptr, *p_sh = nullptr, *p_up_sh = nullptr;
    zh::XPlanes p_xp{};  // the shared expert's inputs, split once per layer
    uint32_t *p_route = nullptr;  // [layers][pre_max][2k + 2]
    int *p_list = nullptr, *p_tiles = nullptr, *p_ntiles = nullptr;
};

namespace {

int fail(char *err, size_t err_len, int code, const char *msg) {
    set_err(err, err_len, "%s", msg);
    return code;
}

// The fused launches' error flag: set when a wait for an act row ran out
// (the outputs are then not valid); read and cleared after the stream is
// synchronized.
int poll_check_moe(ZiggyHipMoeStack *s, char *err, size_t err_len) {
    if (!s->fuse_ffn) return ZIGGY_HIP_OK;
    int flag = 0;
    ZH_TRY(hipMemcpy(&flag, s->poll_err, 4, hipMemcpyDeviceToHost), "MoE poll flag");
    if (!flag) return ZIGGY_HIP_OK;
    ZH_TRY(hipMemset(s->poll_err, 0, 4), "MoE poll flag");
    return fail(err, err_len, ZIGGY_HIP_EXECUTION_FAILED, "an MoE act row never arrived (fused expert launch)");
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

float *act_of(const ZiggyHipMoeStack *s, int l) {
    const size_t set = (size_t)((l % (int)s->layers.size()) % s->act_sets);
    return s->act + set * (s->d.expert_used_count + 1) * (size_t)s->act_stride;
}

// The hidden state layer l reads (and its gate/up normalises).
float *hidden_of(const ZiggyHipMoeStack *s, int l) {
    if (!s->fuse_combine) return s->hidden;
    return ((int)s->layers.size() - 1 - l) % 2 == 0 ? s->hidden : s->hidden2;
}

// One layer's launches (see zh_moe.hip).
hipError_t enqueue_layer(ZiggyHipMoeStack *s, int l, hipStream_t st) {
    const MoeLayerW &L = s->layers[l];
    const ZiggyHipMoeDesc &d = s->d;
    const int H = (int)d.hidden, E = (int)d.expert_count, K = (int)d.expert_used_count, FF = (int)d.expert_ff_length;
    uint32_t *route = s->route + (size_t)l * s->route_stride;
    float *hidden = hidden_of(s, l);
    float *act = act_of(s, l);
    // router (+ the shared expert's gate row) on the normed hidden state;
    // with fuse_combine, layer l - 1's combine first (its result to `hidden`)
    {
        MvParams p{};
        p.nseg = 1;
        p.seg[0] = seg_of(L.router, s->logits);
        if (s->shared_gate) {
            p.seg[1] = seg_of(L.gate_inp_sh, s->logits + E);
            p.nseg = 2;
        }
        p.cols = H;
        p.x = hidden;
        if (s->fuse_combine && l > 0) {
            p.x = hidden_of(s, l - 1);
            p.pro_in = s->tmp;
            p.pro_out = hidden;
            p.expert = s->route + (size_t)(l - 1) * s->route_stride;
            p.pro_cfg = (uint32_t)K | (s->shared ? 1u : 0u) << 4;
        }
        p.norm_w = (const float *)L.norm.p;
        p.eps = d.rms_norm_eps;
        hipError_t e = launch_matvec(p, IN_NORM, OUT_STORE, st);
        if (e != hipSuccess) return e;
    }
    // up to 256 experts: the gate/up launch routes the token itself (each
    // routed workgroup, one wavefront) and writes the route for the launches
    // after it; more experts take the routing kernel
    const bool route_in_gate_up = E <= kRouteWaveExperts && K <= kRouteMaxK && d.gating_func <= 15;
    hipError_t e = hipSuccess;
    const uint32_t route_cfg = (uint32_t)E | (uint32_t)K << 16 | d.gating_func << 20 | (d.weights_norm ? 1u : 0u) << 24 |
                               (s->shared_gate ? 1u : 0u) << 25;
    if (s->fuse_ffn) {
        // gate/up and down in one launch: the down workgroups route
        // themselves and read the act rows as gate/up publishes them
        MvParams pg{}, pd{};
        for (int k = 0; k < K; k++) {
            pg.seg[k] = seg_of(L.gate, act + (size_t)k * s->act_stride);
            pg.seg[k].rows = FF;
            pg.seg[k].w2 = L.up.p;
            pg.seg[k].expert_slot = k;
            pd.seg[k] = seg_of(L.down, s->tmp + (size_t)k * H);
            pd.seg[k].rows = H;
            pd.seg[k].x = act + (size_t)k * s->act_stride;
            pd.seg[k].expert_slot = k;
        }
        pg.nseg = pd.nseg = K;
        if (s->shared) {
            pg.seg[K] = seg_of(L.gate_sh, act + (size_t)K * s->act_stride);
            pg.seg[K].w2 = L.up_sh.p;
            pd.seg[K] = seg_of(L.down_sh, s->tmp + (size_t)K * H);
            pd.seg[K].x = act + (size_t)K * s->act_stride;
            pg.nseg = pd.nseg = K + 1;
        }
        pg.cols = H;
        pg.x = hidden;
        pg.norm_w = (const float *)L.norm.p;
        pg.eps = d.rms_norm_eps;
        pg.rows_per_expert = FF;
        pg.expert_limit = E;
        pg.pro_in = s->logits;
        pg.pro_out = route;
        pg.pro_cfg = route_cfg;
        pg.pro_scale = d.weights_scale;
        pd.cols = FF;
        pd.rows_per_expert = H;
        pd.expert_limit = E;
        pd.pro_in = s->logits;
        pd.pro_cfg = route_cfg;
        e = launch_moe_ffn(pg, pd, s->poll_err, act_of(s, l + 1), (K + 1) * s->act_stride, st);
        if (e != hipSuccess) return e;
        if (s->fuse_combine && l + 1 < (int)s->layers.size()) return hipSuccess;
        return launch_moe_combine(hidden, s->tmp, route, H, K, s->shared ? 1 : 0, st);
    }
    if (!route_in_gate_up) {
        e = launch_moe_route(s->logits, E, K, (int)d.gating_func, (int)d.weights_norm, d.weights_scale,
                             s->shared_gate ? 1 : 0, route, st);
        if (e != hipSuccess) return e;
    }
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
        p.x = hidden;
        p.norm_w = (const float *)L.norm.p;
        p.eps = d.rms_norm_eps;
        p.rows_per_expert = FF;
        p.expert_limit = E;
        if (route_in_gate_up) {
            p.pro_in = s->logits;
            p.pro_out = route;
            p.pro_cfg = route_cfg;
            p.pro_scale = d.weights_scale;
        } else {
            p.expert = route;
        }
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
    // the next layer's router runs this combine when fused
    if (s->fuse_combine && l + 1 < (int)s->layers.size()) return hipSuccess;
    return launch_moe_combine(hidden, s->tmp, route, H, K, s->shared ? 1 : 0, st);
}

// One layer over M token rows (prefill): the rows are independent, so each
// goes through the same operations as the decode path; the routed experts
// run grouped (launch_moe_group), one expert's token tile per GEMM workgroup,
// so every routed expert's weights stream once per tile.
//   norm     per-row RMSNorm into p_normed
//   router   f32-exact MFMA GEMM (the top-k must see the matvec's logits),
//            plus the shared expert's gate row into column E
//   route    per row, as in decode; group: assignments by expert
//   gate/up  grouped SWIGLU GEMM -> p_act[t * k + s]; shared -> p_act_sh[t]
//   down     grouped GEMM -> p_tmp[t * k + s]; shared -> p_sh[t]
//   combine  per row, slot order as in decode
hipError_t enqueue_prefill_layer(ZiggyHipMoeStack *s, int l, int M, hipStream_t st) {
    const MoeLayerW &L = s->layers[l];
    const ZiggyHipMoeDesc &d = s->d;
    const int H = (int)d.hidden, E = (int)d.expert_count, K = (int)d.expert_used_count, FF = (int)d.expert_ff_length,
              SF = (int)d.shared_ff_length;
    uint32_t *route = s->p_route + (size_t)l * s->pre_max * s->route_stride;
    // the shared expert on split inputs (more than one token tile): the norm
    // also splits its rows; gate and up as two stores in one launch, then
    // SiLU * up split for down
    const bool sh_split = s->shared && M > 16 && H % 32 == 0 && SF % 32 == 0 && s->p_xp.hi;
    hipError_t e = launch_rms_norm_rows(s->p_hidden, (const float *)L.norm.p, s->p_normed, M, H, d.rms_norm_eps, st,
                                        nullptr, 0, nullptr, 0, nullptr, 0, sh_split ? &s->p_xp : nullptr);
    // the shared gate row, stored right after the router's rows, is row E of one launch
    const bool gate_row_next = s->shared_gate && L.gate_inp_sh.p == L.router.p + (uint64_t)E * L.router.stride &&
                               L.gate_inp_sh.stride == L.router.stride;
    if (e == hipSuccess)
        e = launch_gemm(L.router.type, L.router.p, nullptr, L.router.stride, s->p_normed, H, s->p_logits, E + 1, M,
                        gate_row_next ? E + 1 : E, H, OUT_STORE, nullptr, st, true);
    if (e == hipSuccess && s->shared_gate && !gate_row_next)
        e = launch_gemm(L.gate_inp_sh.type, L.gate_inp_sh.p, nullptr, L.gate_inp_sh.stride, s->p_normed, H,
                        s->p_logits + E, E + 1, M, 1, H, OUT_STORE, nullptr, st, true);
    if (e == hipSuccess)
        e = launch_moe_route(s->p_logits, E, K, (int)d.gating_func, (int)d.weights_norm, d.weights_scale,
                             s->shared_gate ? 1 : 0, route, st, M, E + 1);
    if (e == hipSuccess) e = launch_moe_group(route, s->route_stride, M, K, E, s->p_list, s->p_tiles, s->p_ntiles, st);
    // tiles <= assignments / 16 + one partial tile per expert touched
    const int max_tiles = M * K / 16 + (E < M * K ? E : M * K);
    if (e == hipSuccess)
        e = launch_gemm_grouped(L.gate.type, L.gate.p, L.up.p, L.gate.stride, (uint64_t)FF * L.gate.stride,
                                s->p_normed, H, K, s->p_act, FF, FF, H, OUT_SWIGLU, s->p_tiles, s->p_list,
                                s->p_ntiles, max_tiles, st);
    if (e == hipSuccess && sh_split) {
        const uint8_t *ws[2] = {L.gate_sh.p, L.up_sh.p};
        float *ys[2] = {s->p_act_sh, s->p_up_sh};
        const int lds[2] = {SF, SF}, Ns[2] = {SF, SF};
        if (e == hipSuccess)
            e = launch_gemm_multi(L.gate_sh.type, 2, ws, ys, lds, Ns, L.gate_sh.stride, s->p_normed, H, M, H,
                                  OUT_STORE, st, 1, &s->p_xp);
        if (e == hipSuccess) e = launch_silu_mul_split(s->p_act_sh, s->p_up_sh, M, SF, s->p_xp, st);
    } else if (e == hipSuccess && s->shared) {
        e = launch_gemm(L.gate_sh.type, L.gate_sh.p, L.up_sh.p, L.gate_sh.stride, s->p_normed, H, s->p_act_sh, SF, M,
                        SF, H, OUT_SWIGLU, nullptr, st);
    }
    if (e == hipSuccess)
        e = launch_gemm_grouped(L.down.type, L.down.p, nullptr, L.down.stride, (uint64_t)H * L.down.stride, s->p_act,
                                FF, 1, s->p_tmp, H, H, FF, OUT_STORE, s->p_tiles, s->p_list, s->p_ntiles, max_tiles,
                                st);
    if (e == hipSuccess && s->shared)
        e = launch_gemm(L.down_sh.type, L.down_sh.p, nullptr, L.down_sh.stride, s->p_act_sh, SF, s->p_sh, H, M, H, SF,
                        OUT_STORE, nullptr, st, false, 16, sh_split ? &s->p_xp : nullptr);
    if (e == hipSuccess)
        e = launch_moe_combine(s->p_hidden, s->p_tmp, route, H, K, s->shared ? 1 : 0, st, M,
                               s->shared ? s->p_sh : nullptr);
    return e;
}

hipError_t prefill_alloc(ZiggyHipMoeStack *s) {
    if (s->pre_max) return hipSuccess;
    const ZiggyHipMoeDesc &d = s->d;
    const size_t H = d.hidden, E = d.expert_count, K = d.expert_used_count, FF = d.expert_ff_length,
                 SF = d.shared_ff_length, NL = s->layers.size();
    const size_t Mc = 4096 / K < 512 ? 4096 / K : 512;
    const size_t tiles = Mc * K / 16 + E;
    struct {
        void **p;
        size_t bytes;
    } reqs[] = {
        {(void **)&s->p_input, Mc * H * 4},
        {(void **)&s->p_hidden, Mc * H * 4},
        {(void **)&s->p_normed, Mc * H * 4},
        {(void **)&s->p_logits, Mc * (E + 1) * 4},
        {(void **)&s->p_act, Mc * K * FF * 4},
        {(void **)&s->p_act_sh, Mc * (SF ? SF : 1) * 4},
        {(void **)&s->p_up_sh, Mc * (SF ? SF : 1) * 4},
        {(void **)&s->p_tmp, Mc * K * H * 4},
        {(void **)&s->p_sh, Mc * H * 4},
        {(void **)&s->p_route, NL * Mc * s->route_stride * 4},
        {(void **)&s->p_list, Mc * K * 4},
        {(void **)&s->p_tiles, tiles * 3 * 4},
        {(void **)&s->p_ntiles, 256},
    };
    for (auto &r : reqs) {
        hipError_t e = hipMalloc(r.p, r.bytes);
        if (e == hipSuccess) e = hipMemsetAsync(*r.p, 0, r.bytes, s->ctx->stream);
        if (e != hipSuccess) return e;
        s->allocs.push_back(*r.p);
    }
    {
        const size_t ld = (std::max(H, SF) + 31) / 32 * 32;
        uint8_t *base = nullptr;
        hipError_t e = hipMalloc((void **)&base, Mc * ld * 4 + Mc * (ld / 32) * 4);
        if (e != hipSuccess) return e;
        s->allocs.push_back(base);
        s->p_xp.hi = reinterpret_cast<uint16_t *>(base);
        s->p_xp.lo = s->p_xp.hi + Mc * ld;
        s->p_xp.sum = reinterpret_cast<float *>(s->p_xp.lo + Mc * ld);
        s->p_xp.ld = (int)ld;
    }
    s->pre_max = (int)Mc;
    return hipSuccess;
}

hipError_t enqueue_prefill(ZiggyHipMoeStack *s, int M, hipStream_t st) {
    hipError_t e = hipMemcpyAsync(s->p_hidden, s->p_input, (size_t)M * s->d.hidden * 4, hipMemcpyDeviceToDevice, st);
    for (int l = 0; l < (int)s->layers.size() && e == hipSuccess; l++) e = enqueue_prefill_layer(s, l, M, st);
    return e;
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
             // right after the router: one prefill launch takes both as E + 1 rows
             take_tensor(&t.gate_inp_shexp, 1, H, false, false, &L.gate_inp_sh, &off, todo) &&
             take_tensor(&t.gate_exps, E * FF, H, true, false, &L.gate, &off, todo) &&
             take_tensor(&t.up_exps, E * FF, H, true, false, &L.up, &off, todo) &&
             take_tensor(&t.down_exps, E * H, FF, true, false, &L.down, &off, todo) &&
             take_tensor(&t.gate_shexp, SF, H, false, false, &L.gate_sh, &off, todo) &&
             take_tensor(&t.up_shexp, SF, H, false, false, &L.up_sh, &off, todo) &&
             take_tensor(&t.down_shexp, H, SF, false, false, &L.down_sh, &off, todo);
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
    // gate/up and down fused: routing in the gate/up launch, the shared
    // expert's down rows as long as the routed ones, a served kernel, and
    // more than one layer (ZIGGY_HIP_MOE_FUSE=0 keeps separate launches)
    {
        const char *env = getenv("ZIGGY_HIP_MOE_FUSE");
        const MoeLayerW &L0 = s->layers[0];
        s->fuse_ffn = !(env && env[0] == '0') && layer_count >= 2 && E <= (uint64_t)kRouteWaveExperts &&
                      K <= (uint64_t)kRouteMaxK && (!s->shared || SF == FF) &&
                      moe_ffn_supported(L0.gate.type, s->shared ? L0.gate_sh.type : L0.gate.type, (int)H, (int)FF);
        if (s->fuse_ffn) {
            s->act_sets = 2;
            while ((layer_count - 1) % s->act_sets == 0) s->act_sets++;
        }
    }
    struct {
        void **p;
        size_t bytes;
    } reqs[] = {
        {(void **)&s->hidden, H * 4},
        {(void **)&s->hidden2, H * 4},
        {(void **)&s->logits, (E + 1) * 4},
        {(void **)&s->act, (size_t)s->act_sets * (K + 1) * (size_t)s->act_stride * 4},
        {(void **)&s->poll_err, 4},
        {(void **)&s->tmp, (K + 1) * H * 4},
        {(void **)&s->route, (size_t)layer_count * s->route_stride * 4},
    };
    for (auto &r : reqs) {
        e = hipMalloc(r.p, r.bytes);
        // the fused launches' act words start as kPollEmpty (outside any graph)
        const int fill = r.p == (void **)&s->act && s->fuse_ffn ? 0xFF : 0;
        if (e == hipSuccess) e = hipMemsetAsync(*r.p, fill, r.bytes, ctx->stream);
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
    // the combine fuses into the next router launch when that launch is the
    // f32 matvec (the kernel holds the combined row in LDS)
    s->fuse_combine = layer_count > 1 && H <= (size_t)kCombineMaxCols && H % 4 == 0;
    for (const MoeLayerW &L : s->layers)
        if (L.router.type != ZIGGY_HIP_TYPE_F32 || (s->shared_gate && L.gate_inp_sh.type != ZIGGY_HIP_TYPE_F32))
            s->fuse_combine = false;
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
    ZH_TRY(hipMemcpyAsync(hidden_of(s, 0), hidden_in, H * 4, hipMemcpyHostToDevice, st), "MoE input");
    ZH_TRY(hipGraphLaunch(s->graph, st), "MoE stack");
    ZH_TRY(hipMemcpyAsync(hidden_out, s->hidden, H * 4, hipMemcpyDeviceToHost, st), "MoE output");
    std::vector<uint32_t> r;
    if (selected || weights) {
        r.resize(NL * s->route_stride);
        ZH_TRY(hipMemcpyAsync(r.data(), s->route, r.size() * 4, hipMemcpyDeviceToHost, st), "MoE routing");
    }
    ZH_TRY(hipStreamSynchronize(st), "MoE stack");
    if (int pe = poll_check_moe(s, err, err_len)) return pe;
    for (size_t l = 0; l < r.size() / s->route_stride; l++)
        for (size_t k = 0; k < K; k++) {
            const uint32_t *e = &r[l * s->route_stride + 2 * k];
            if (selected) selected[l * K + k] = e[0];
            if (weights) memcpy(&weights[l * K + k], &e[1], 4);
        }
    return ZIGGY_HIP_OK;
}

int ziggy_hip_moe_stack_prefill(ZiggyHipMoeStack *s, const float *hidden_in, uint32_t tokens, float *hidden_out,
                                uint32_t *selected, float *weights, char *err, size_t err_len) {
    if (!s || !hidden_in || !hidden_out || tokens == 0)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "invalid arguments");
    hipSetDevice(s->ctx->device);
    hipStream_t st = s->ctx->stream;
    ZH_TRY(prefill_alloc(s), "MoE prefill buffers");
    const size_t H = s->d.hidden, K = s->d.expert_used_count, NL = s->layers.size(), RS = s->route_stride;
    std::vector<uint32_t> r;
    for (uint32_t t0 = 0; t0 < tokens; t0 += (uint32_t)s->pre_max) {
        const uint32_t M = tokens - t0 < (uint32_t)s->pre_max ? tokens - t0 : (uint32_t)s->pre_max;
        ZH_TRY(hipMemcpyAsync(s->p_input, hidden_in + (size_t)t0 * H, M * H * 4, hipMemcpyHostToDevice, st),
               "MoE prefill input");
        ZH_TRY(enqueue_prefill(s, (int)M, st), "MoE prefill");
        ZH_TRY(hipMemcpyAsync(hidden_out + (size_t)t0 * H, s->p_hidden, M * H * 4, hipMemcpyDeviceToHost, st),
               "MoE prefill output");
        if (selected || weights) {
            r.resize(NL * s->pre_max * RS);
            ZH_TRY(hipMemcpyAsync(r.data(), s->p_route, r.size() * 4, hipMemcpyDeviceToHost, st), "MoE routing");
        }
        ZH_TRY(hipStreamSynchronize(st), "MoE prefill");
        if (!r.empty())
            for (size_t t = 0; t < M; t++)
                for (size_t l = 0; l < NL; l++)
                    for (size_t k = 0; k < K; k++) {
                        const uint32_t *e = &r[(l * s->pre_max + t) * RS + 2 * k];
                        const size_t o = ((t0 + t) * NL + l) * K + k;
                        if (selected) selected[o] = e[0];
                        if (weights) memcpy(&weights[o], &e[1], 4);
                    }
    }
    return ZIGGY_HIP_OK;
}

int ziggy_hip_moe_stack_time_prefill(ZiggyHipMoeStack *s, uint32_t tokens, uint32_t iterations, uint64_t *avg_ns,
                                     char *err, size_t err_len) {
    if (!s || !iterations || !avg_ns || tokens == 0)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT, "invalid arguments");
    if (!s->pre_max || tokens > (uint32_t)s->pre_max)
        return fail(err, err_len, ZIGGY_HIP_INVALID_ARGUMENT,
                    "time_prefill replays the last prefill input: run a prefill of at least `tokens` rows first");
    hipSetDevice(s->ctx->device);
    hipStream_t st = s->ctx->stream;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    ZH_TRY(hipEventCreate(&e0), "MoE prefill time");
    hipError_t e = hipEventCreate(&e1);
    if (e == hipSuccess) e = enqueue_prefill(s, (int)tokens, st);  // warm-up
    if (e == hipSuccess) e = hipEventRecord(e0, st);
    for (uint32_t i = 0; i < iterations && e == hipSuccess; i++) e = enqueue_prefill(s, (int)tokens, st);
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (e != hipSuccess) return hip_fail(e, "MoE prefill time", err, err_len);
    *avg_ns = (uint64_t)((double)ms * 1e6 / iterations);
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
    if (int pe = poll_check_moe(s, err, err_len)) return pe;
    *avg_ns = (uint64_t)((double)ms * 1e6 / iterations);
    return ZIGGY_HIP_OK;
}

}  // extern "C"
