// zh_runtime.cpp -- context, buffers, sequences and the primitive-op entry
// points of the C ABI (include/ziggy_hip.h).
//
// Execution model (runtime/metal/bridge.m:324-485 for Metal): one HIP stream
// per context; while a sequence is open every op is only enqueued, otherwise
// it is enqueued and the stream is synchronised before returning.
// commit_sequence_timed brackets the sequence with HIP events.
#include <chrono>
#include <new>

#include "zh_internal.h"
#include "zh_quant.h"

using namespace zh;

namespace {

constexpr size_t kCtxScratch = 64u << 20;  // attention partials + argmax/topk slots
constexpr size_t kCtxCounters = 1024;      // attention arrival counters (one per kv head)

int gguf_row_bytes(uint32_t type, uint32_t cols, uint64_t *out) {
    switch (type) {
    case ZIGGY_HIP_TYPE_F32: *out = (uint64_t)cols * 4; return 0;
    case ZIGGY_HIP_TYPE_F16: *out = (uint64_t)cols * 2; return 0;
    case ZIGGY_HIP_TYPE_Q8_0: if (cols % 32) return -1; *out = (uint64_t)cols / 32 * 34; return 0;
    case ZIGGY_HIP_TYPE_Q3_K: if (cols % 256) return -1; *out = (uint64_t)cols / 256 * 110; return 0;
    case ZIGGY_HIP_TYPE_Q4_K: if (cols % 256) return -1; *out = (uint64_t)cols / 256 * 144; return 0;
    case ZIGGY_HIP_TYPE_Q6_K: if (cols % 256) return -1; *out = (uint64_t)cols / 256 * 210; return 0;
    case ZIGGY_HIP_TYPE_IQ4_XS: if (cols % 256) return -1; *out = (uint64_t)cols / 256 * 136; return 0;
    default: return -1;
    }
}

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

// Validates a matvec call: shapes, alignment of the x slot layout, buffer sizes.
int check_matvec(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *m, size_t moff, const ZiggyHipBuffer *in,
                 const ZiggyHipBuffer *out, size_t ooff, uint32_t rows, uint32_t cols, uint64_t *stride, char *err,
                 size_t err_len, uint32_t max_cols) {
    if (!ctx) {
        set_err(err, err_len, "null context");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    if (gguf_row_bytes(type, cols, stride)) {
        set_err(err, err_len, "unsupported tensor type %u or row length %u", type, cols);
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    if (cols % 64 || cols == 0) {
        set_err(err, err_len, "row length %u must be a non-zero multiple of 64", cols);
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    if (cols > max_cols) {
        set_err(err, err_len, "row length %u exceeds %u", cols, max_cols);
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    if (!buf_ok(m, moff + *stride * rows) || !buf_ok(in, (size_t)cols * 4) || !out ||
        (ooff % 4) || !buf_ok(out, ooff + (size_t)rows * 4)) {
        set_err(err, err_len, "buffer too small or misaligned for %ux%u matvec", rows, cols);
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    return ZIGGY_HIP_OK;
}

}  // namespace

namespace zh {

hipError_t ctx_rope_denom(ZiggyHipContext *ctx, float base, int n_rot, const float **out) {
    for (auto &t : ctx->rope_tables)
        if (t.dev && t.base == base && t.n_rot == n_rot) {
            *out = t.dev;
            return hipSuccess;
        }
    // a new (base, n_rot): a table of its own (never overwritten, so launches
    // still queued on the stream keep reading theirs); the oldest is replaced
    // once eight are held, after the stream drains
    ZiggyHipContext::RopeTable *slot = nullptr;
    for (auto &t : ctx->rope_tables)
        if (!t.dev) {
            slot = &t;
            break;
        }
    if (!slot) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return e;
        slot = &ctx->rope_tables[0];
        hipFree(slot->dev);
        for (int i = 0; i + 1 < 8; i++) ctx->rope_tables[i] = ctx->rope_tables[i + 1];
        slot = &ctx->rope_tables[7];
        slot->dev = nullptr;
    }
    float host[128];
    const int half = n_rot / 2 > 0 ? n_rot / 2 : 1;
    if (half > 128) return hipErrorInvalidValue;
    rope_denominators(base, n_rot, host);
    float *dev = nullptr;
    hipError_t e = hipMalloc((void **)&dev, (size_t)half * 4);
    if (e != hipSuccess) return e;
    e = hipMemcpy(dev, host, (size_t)half * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        hipFree(dev);
        return e;
    }
    *slot = {base, n_rot, dev};
    *out = dev;
    return hipSuccess;
}

int attention_call_params(const ZiggyHipBuffer *q, const ZiggyHipBuffer *kc, const ZiggyHipBuffer *vc,
                          const ZiggyHipBuffer *out, uint32_t heads, uint32_t heads_kv, uint32_t hd, uint32_t kv_dim,
                          uint32_t ctx_len, uint32_t pos, uint32_t layer_base, uint32_t window_start, float scale,
                          float softcap, AttnParams *p, char *err, size_t err_len) {
    if (heads == 0 || heads_kv == 0 || heads % heads_kv || heads / heads_kv > 8 ||
        (hd != 64 && hd != 96 && hd != 128 && hd != 256) || kv_dim != heads_kv * hd || pos >= ctx_len || window_start > pos ||
        (uint64_t)ctx_len > ((uint64_t)kIdentityPages << kKvPageShift)) {
        set_err(err, err_len, "unsupported attention shape");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    if (softcap != 0.f) {
        set_err(err, err_len, "attention softcapping is not supported on this path");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    const size_t cache_need = ((size_t)layer_base + (size_t)ctx_len * kv_dim) * 2;
    if (!buf_ok(q, (size_t)heads * hd * 4) || !buf_ok(kc, cache_need) || !buf_ok(vc, cache_need) ||
        !buf_ok(out, (size_t)heads * hd * 4)) {
        set_err(err, err_len, "attention buffers too small");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    *p = AttnParams{};
    p->q = (const float *)q->ptr;
    p->k_cache = (__half *)kc->ptr + layer_base;
    p->v_cache = (__half *)vc->ptr + layer_base;
    p->out = (float *)out->ptr;
    p->head_count = (int)heads;
    p->head_count_kv = (int)heads_kv;
    p->head_dim = (int)hd;
    p->kv_dim = (int)kv_dim;
    p->position = (int)pos;
    p->window_start = (int)window_start;
    p->scale = scale;
    p->max_splits = attention_splits((int)heads_kv, (int)(pos + 1 - window_start));
    return ZIGGY_HIP_OK;
}

}  // namespace zh

extern "C" {

const char *ziggy_hip_version(void) { return "libziggy_hip gfx950 " __DATE__; }

int ziggy_hip_create_context(int device_index, ZiggyHipContext **out_ctx, ZiggyHipDeviceInfo *out_info, char *err,
                             size_t err_len) {
    if (!out_ctx) {
        set_err(err, err_len, "null output pointer");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    *out_ctx = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        set_err(err, err_len, "no HIP device available");
        return ZIGGY_HIP_UNAVAILABLE;
    }
    if (device_index < 0 || device_index >= count) {
        set_err(err, err_len, "device index %d out of range (%d devices)", device_index, count);
        return ZIGGY_HIP_UNAVAILABLE;
    }
    hipDeviceProp_t prop;
    if (hipSetDevice(device_index) != hipSuccess || hipGetDeviceProperties(&prop, device_index) != hipSuccess) {
        set_err(err, err_len, "hipSetDevice/hipGetDeviceProperties failed");
        return ZIGGY_HIP_INITIALIZATION_FAILED;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_err(err, err_len, "device %s is not gfx950; this library carries gfx950 code only", prop.gcnArchName);
        return ZIGGY_HIP_UNAVAILABLE;
    }
    ZiggyHipContext *ctx = new (std::nothrow) ZiggyHipContext();
    if (!ctx) {
        set_err(err, err_len, "out of host memory");
        return ZIGGY_HIP_INITIALIZATION_FAILED;
    }
    ctx->device = device_index;
    snprintf(ctx->info.name, sizeof(ctx->info.name), "%s", prop.name);
    snprintf(ctx->info.arch, sizeof(ctx->info.arch), "%s", prop.gcnArchName);
    ctx->info.total_memory = prop.totalGlobalMem;
    ctx->info.compute_units = (uint32_t)prop.multiProcessorCount;
    ctx->info.wavefront_size = (uint32_t)prop.warpSize;
    ctx->info.clock_khz = (uint32_t)prop.clockRate;
    ctx->info.l2_bytes = (uint32_t)prop.l2CacheSize;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&ctx->seq_begin) != hipSuccess || hipEventCreate(&ctx->seq_end) != hipSuccess ||
        hipMalloc(&ctx->scratch, kCtxScratch) != hipSuccess ||
        hipMalloc((void **)&ctx->counters, kCtxCounters * sizeof(unsigned)) != hipSuccess ||
        hipMemset(ctx->counters, 0, kCtxCounters * sizeof(unsigned)) != hipSuccess ||
        hipMalloc((void **)&ctx->identity_pages, kIdentityPages * sizeof(uint32_t)) != hipSuccess ||
        launch_iota_u32(ctx->identity_pages, kIdentityPages, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        set_err(err, err_len, "stream/event/scratch creation failed");
        ziggy_hip_destroy_context(ctx);
        return ZIGGY_HIP_INITIALIZATION_FAILED;
    }
    ctx->scratch_len = kCtxScratch;
    const int nst = noalloc_init_device(device_index, err, err_len);
    if (nst != ZIGGY_HIP_OK) {
        ziggy_hip_destroy_context(ctx);
        return nst;
    }
    if (out_info) *out_info = ctx->info;
    *out_ctx = ctx;
    return ZIGGY_HIP_OK;
}

void ziggy_hip_destroy_context(ZiggyHipContext *ctx) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    if (ctx->stream) hipStreamSynchronize(ctx->stream);
    for (auto &t : ctx->rope_tables)
        if (t.dev) hipFree(t.dev);
    if (ctx->scratch) hipFree(ctx->scratch);
    if (ctx->counters) hipFree(ctx->counters);
    if (ctx->identity_pages) hipFree(ctx->identity_pages);
    if (ctx->seq_begin) hipEventDestroy(ctx->seq_begin);
    if (ctx->seq_end) hipEventDestroy(ctx->seq_end);
    if (ctx->stream) hipStreamDestroy(ctx->stream);
    delete ctx;
}

int ziggy_hip_create_empty_buffer(ZiggyHipContext *ctx, size_t length, ZiggyHipBuffer **out, char *err,
                                  size_t err_len) {
    if (!ctx || !out || length == 0) {
        set_err(err, err_len, "invalid buffer request");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    *out = nullptr;
    ZiggyHipBuffer *b = new (std::nothrow) ZiggyHipBuffer();
    if (!b) return ZIGGY_HIP_BUFFER_FAILED;
    hipSetDevice(ctx->device);
    hipError_t e = hipMalloc(&b->ptr, length);
    if (e != hipSuccess) {
        delete b;
        set_err(err, err_len, "hipMalloc(%zu): %s", length, hipGetErrorString(e));
        return ZIGGY_HIP_BUFFER_FAILED;
    }
    e = hipMemsetAsync(b->ptr, 0, length, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        hipFree(b->ptr);
        delete b;
        set_err(err, err_len, "clearing buffer: %s", hipGetErrorString(e));
        return ZIGGY_HIP_BUFFER_FAILED;
    }
    b->ctx = ctx;
    b->device = ctx->device;
    b->len = length;
    *out = b;
    return ZIGGY_HIP_OK;
}

int ziggy_hip_create_buffer(ZiggyHipContext *ctx, const void *bytes, size_t length, ZiggyHipBuffer **out, char *err,
                            size_t err_len) {
    if (!bytes) {
        set_err(err, err_len, "null source bytes");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    int st = ziggy_hip_create_empty_buffer(ctx, length, out, err, err_len);
    if (st) return st;
    hipError_t e = hipMemcpy((*out)->ptr, bytes, length, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        ziggy_hip_destroy_buffer(*out);
        *out = nullptr;
        set_err(err, err_len, "upload: %s", hipGetErrorString(e));
        return ZIGGY_HIP_BUFFER_FAILED;
    }
    return ZIGGY_HIP_OK;
}

void ziggy_hip_destroy_buffer(ZiggyHipBuffer *b) {
    if (!b) return;
    if (b->ptr) {
        // hipFree waits for the device; the context may already be gone
        hipSetDevice(b->device);
        hipFree(b->ptr);
    }
    delete b;
}

size_t ziggy_hip_buffer_length(const ZiggyHipBuffer *b) { return b ? b->len : 0; }

int ziggy_hip_write_buffer(ZiggyHipBuffer *b, const void *bytes, size_t length, size_t offset, char *err,
                           size_t err_len) {
    if (!b || !bytes || offset > b->len || length > b->len - offset) {
        set_err(err, err_len, "write out of bounds");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    ZiggyHipContext *ctx = b->ctx;
    ZH_TRY(hipMemcpyAsync((char *)b->ptr + offset, bytes, length, hipMemcpyHostToDevice, ctx->stream), "write_buffer");
    ZH_TRY(hipStreamSynchronize(ctx->stream), "write_buffer");
    return ZIGGY_HIP_OK;
}

int ziggy_hip_read_buffer(const ZiggyHipBuffer *b, void *out, size_t length, size_t offset, char *err,
                          size_t err_len) {
    if (!b || !out || offset > b->len || length > b->len - offset) {
        set_err(err, err_len, "read out of bounds");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    ZiggyHipContext *ctx = b->ctx;
    ZH_TRY(hipMemcpyAsync(out, (const char *)b->ptr + offset, length, hipMemcpyDeviceToHost, ctx->stream),
           "read_buffer");
    ZH_TRY(hipStreamSynchronize(ctx->stream), "read_buffer");
    return ZIGGY_HIP_OK;
}

int ziggy_hip_copy_buffer_region(ZiggyHipContext *ctx, const ZiggyHipBuffer *src, size_t src_off, ZiggyHipBuffer *dst,
                                 size_t dst_off, size_t length, char *err, size_t err_len) {
    if (!ctx || !src || !dst || src_off > src->len || length > src->len - src_off || dst_off > dst->len ||
        length > dst->len - dst_off) {
        set_err(err, err_len, "copy out of bounds");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    ZH_TRY(hipMemcpyAsync((char *)dst->ptr + dst_off, (const char *)src->ptr + src_off, length,
                          hipMemcpyDeviceToDevice, ctx->stream),
           "copy_buffer_region");
    return finish_op(ctx, "copy_buffer_region", err, err_len);
}

int ziggy_hip_begin_sequence(ZiggyHipContext *ctx, char *err, size_t err_len) {
    if (!ctx) return ZIGGY_HIP_INVALID_ARGUMENT;
    if (ctx->seq_open) {
        set_err(err, err_len, "a sequence is already open");
        return ZIGGY_HIP_EXECUTION_FAILED;
    }
    ZH_TRY(hipEventRecord(ctx->seq_begin, ctx->stream), "begin_sequence");
    ctx->seq_open = true;
    return ZIGGY_HIP_OK;
}

int ziggy_hip_commit_sequence_timed(ZiggyHipContext *ctx, ZiggyHipCommitStats *stats, char *err, size_t err_len) {
    if (!ctx) return ZIGGY_HIP_INVALID_ARGUMENT;
    const bool was_open = ctx->seq_open;
    ctx->seq_open = false;
    if (was_open) ZH_TRY(hipEventRecord(ctx->seq_end, ctx->stream), "commit_sequence");
    const uint64_t t0 = now_ns();
    ZH_TRY(hipStreamSynchronize(ctx->stream), "commit_sequence");
    const uint64_t t1 = now_ns();
    if (stats) {
        stats->cpu_wait_ns = t1 - t0;
        stats->gpu_elapsed_ns = 0;
        stats->gpu_timestamps_valid = false;
        float ms = 0.f;
        if (was_open && hipEventElapsedTime(&ms, ctx->seq_begin, ctx->seq_end) == hipSuccess) {
            stats->gpu_elapsed_ns = (uint64_t)((double)ms * 1e6);
            stats->gpu_timestamps_valid = true;
        }
    }
    return ZIGGY_HIP_OK;
}

int ziggy_hip_commit_sequence(ZiggyHipContext *ctx, char *err, size_t err_len) {
    return ziggy_hip_commit_sequence_timed(ctx, nullptr, err, err_len);
}

// ---------------- matvec family ----------------

static int run_matvec_mode(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *m, size_t moff,
                           const ZiggyHipBuffer *in, const ZiggyHipBuffer *in2, ZiggyHipBuffer *out, size_t ooff,
                           uint32_t rows, uint32_t cols, int in_mode, int out_mode, const char *what, char *err,
                           size_t err_len) {
    uint64_t stride;
    // plain and SiLU inputs: rows longer than one team run as column windows
    int st = check_matvec(ctx, type, m, moff, in, out, ooff, rows, cols, &stride, err, err_len, kMaxMatvecRowLen);
    if (st) return st;
    if (in2 && !buf_ok(in2, (size_t)cols * 4)) {
        set_err(err, err_len, "second input too small");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    MvParams p{};
    p.nseg = 1;
    p.seg[0].w = (const uint8_t *)m->ptr + moff;
    p.seg[0].stride = stride;
    p.seg[0].y = (float *)((char *)out->ptr + ooff);
    p.seg[0].rows = (int)rows;
    p.seg[0].fmt = (int)type;
    p.cols = (int)cols;
    p.x = (const float *)in->ptr;
    p.x2 = in2 ? (const float *)in2->ptr : nullptr;
    plan_matvec(p, 1024);
    ZH_TRY(launch_matvec(p, in_mode, out_mode, ctx->stream), what);
    return finish_op(ctx, what, err, err_len);
}

int ziggy_hip_run_matvec(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *m, size_t moff,
                         const ZiggyHipBuffer *in, ZiggyHipBuffer *out, size_t ooff, uint32_t rows, uint32_t cols,
                         int add, char *err, size_t err_len) {
    return run_matvec_mode(ctx, type, m, moff, in, nullptr, out, ooff, rows, cols, IN_PLAIN,
                           add ? OUT_ADD : OUT_STORE, "run_matvec", err, err_len);
}

#define ZH_DEFINE_MATVEC(sfx, TYPE)                                                                                    \
    int ziggy_hip_run_matvec_##sfx##_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *m, const ZiggyHipBuffer *in,    \
                                         ZiggyHipBuffer *out, uint32_t rows, uint32_t cols, char *err,               \
                                         size_t err_len) {                                                           \
        return ziggy_hip_run_matvec(ctx, TYPE, m, 0, in, out, 0, rows, cols, 0, err, err_len);                       \
    }                                                                                                                \
    int ziggy_hip_run_matvec_##sfx##_f32_to_dst(ZiggyHipContext *ctx, const ZiggyHipBuffer *m,                      \
                                                const ZiggyHipBuffer *in, ZiggyHipBuffer *out, size_t ooff,          \
                                                uint32_t rows, uint32_t cols, char *err, size_t err_len) {           \
        return ziggy_hip_run_matvec(ctx, TYPE, m, 0, in, out, ooff, rows, cols, 0, err, err_len);                    \
    }                                                                                                                \
    int ziggy_hip_run_matvec_##sfx##_add_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *m, const ZiggyHipBuffer *in, \
                                             ZiggyHipBuffer *out, uint32_t rows, uint32_t cols, char *err,           \
                                             size_t err_len) {                                                       \
        return ziggy_hip_run_matvec(ctx, TYPE, m, 0, in, out, 0, rows, cols, 1, err, err_len);                      \
    }
ZH_DEFINE_MATVEC(q4k, ZIGGY_HIP_TYPE_Q4_K)
ZH_DEFINE_MATVEC(q6k, ZIGGY_HIP_TYPE_Q6_K)
ZH_DEFINE_MATVEC(q8_0, ZIGGY_HIP_TYPE_Q8_0)
ZH_DEFINE_MATVEC(q3k, ZIGGY_HIP_TYPE_Q3_K)
ZH_DEFINE_MATVEC(f16, ZIGGY_HIP_TYPE_F16)
ZH_DEFINE_MATVEC(dense, ZIGGY_HIP_TYPE_F32)

int ziggy_hip_run_matvec_silu_down_add(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *m,
                                       const ZiggyHipBuffer *gate, const ZiggyHipBuffer *up, ZiggyHipBuffer *out,
                                       uint32_t rows, uint32_t cols, char *err, size_t err_len) {
    return run_matvec_mode(ctx, type, m, 0, gate, up, out, 0, rows, cols, IN_SILU, OUT_ADD, "silu_down_add", err,
                           err_len);
}

int ziggy_hip_run_matvec_q4k_silu_down_add_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *m,
                                               const ZiggyHipBuffer *gate, const ZiggyHipBuffer *up,
                                               ZiggyHipBuffer *out, uint32_t rows, uint32_t cols, char *err,
                                               size_t err_len) {
    return ziggy_hip_run_matvec_silu_down_add(ctx, ZIGGY_HIP_TYPE_Q4_K, m, gate, up, out, rows, cols, err, err_len);
}

int ziggy_hip_run_matvec_argmax(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *m,
                                const ZiggyHipBuffer *in, ZiggyHipBuffer *state, uint32_t rows, uint32_t cols,
                                char *err, size_t err_len) {
    uint64_t stride;
    if (!buf_ok(state, 8)) {
        set_err(err, err_len, "argmax state must hold 2 x u32");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    // the logits themselves are not kept: output buffer check uses the state buffer only
    if (!ctx || gguf_row_bytes(type, cols, &stride) || cols % 64 || cols / 64 > 256 ||
        !buf_ok(m, stride * rows) || !buf_ok(in, (size_t)cols * 4)) {
        set_err(err, err_len, "invalid argmax matvec arguments");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    unsigned long long *slot = (unsigned long long *)ctx->scratch;
    MvParams p{};
    p.nseg = 1;
    p.seg[0].w = (const uint8_t *)m->ptr;
    p.seg[0].stride = stride;
    p.seg[0].y = nullptr;
    p.seg[0].rows = (int)rows;
    p.seg[0].fmt = (int)type;
    p.cols = (int)cols;
    p.x = (const float *)in->ptr;
    p.argmax_slot = slot;
    plan_matvec(p, 1024);
    ZH_TRY(launch_fill_u64(slot, 0ull, 1, ctx->stream), "argmax reset");
    ZH_TRY(launch_matvec(p, IN_PLAIN, OUT_ARGMAX, ctx->stream), "matvec_argmax");
    ZH_TRY(launch_argmax_finalize(slot, (uint32_t *)state->ptr, ctx->stream), "argmax finalize");
    return finish_op(ctx, "matvec_argmax", err, err_len);
}

int ziggy_hip_run_matvec_q6k_argmax_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *m, const ZiggyHipBuffer *in,
                                        ZiggyHipBuffer *state, uint32_t rows, uint32_t cols, char *err,
                                        size_t err_len) {
    return ziggy_hip_run_matvec_argmax(ctx, ZIGGY_HIP_TYPE_Q6_K, m, in, state, rows, cols, err, err_len);
}

int ziggy_hip_dequantize_rows(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *m, size_t moff,
                              ZiggyHipBuffer *out, uint32_t rows, uint32_t cols, char *err, size_t err_len) {
    uint64_t stride;
    if (!ctx || gguf_row_bytes(type, cols, &stride) || !buf_ok(m, moff + stride * rows) ||
        !buf_ok(out, (size_t)rows * cols * 4)) {
        set_err(err, err_len, "invalid dequantize arguments");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    ZH_TRY(launch_dequant((int)type, (const uint8_t *)m->ptr + moff, stride, (float *)out->ptr, (int)rows, (int)cols,
                          ctx->stream),
           "dequantize_rows");
    return finish_op(ctx, "dequantize_rows", err, err_len);
}

// ---------------- MFMA GEMM for M >= 8 tokens ----------------

extern "C" int ziggy_hip_run_gemm(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *m,
                                  const ZiggyHipBuffer *in, ZiggyHipBuffer *out, uint32_t tokens, uint32_t rows,
                                  uint32_t cols, int add, char *err, size_t err_len) {
    uint64_t stride;
    int st = check_matvec(ctx, type, m, 0, in, out, 0, rows, cols, &stride, err, err_len, kMaxMatvecCols);
    if (st) return st;
    if (tokens == 0 || cols % 16 || !buf_ok(in, (size_t)tokens * cols * 4) || !buf_ok(out, (size_t)tokens * rows * 4)) {
        set_err(err, err_len, "buffers too small for a %u-token %ux%u GEMM", tokens, rows, cols);
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    ZH_TRY(launch_gemm((int)type, (const uint8_t *)m->ptr, nullptr, stride, (const float *)in->ptr, (int)cols,
                       (float *)out->ptr, (int)rows, (int)tokens, (int)rows, (int)cols, add ? OUT_ADD : OUT_STORE,
                       nullptr, ctx->stream),
           "gemm");
    return finish_op(ctx, "gemm", err, err_len);
}

// ---------------- expert-indexed matvec ----------------

static int indexed_common(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *ma, const ZiggyHipBuffer *mb,
                          const ZiggyHipBuffer *in, ZiggyHipBuffer *outa, ZiggyHipBuffer *outb, uint32_t rows,
                          uint32_t cols, const ZiggyHipBuffer *entries, uint32_t slot, uint32_t rpe, int out_mode,
                          const char *what, char *err, size_t err_len) {
    uint64_t stride;
    int st = check_matvec(ctx, type, ma, 0, in, outa, 0, rows, cols, &stride, err, err_len, kMaxMatvecCols);
    if (st) return st;
    if (!buf_ok(entries, (size_t)(slot + 1) * 8) || rows > rpe) {
        set_err(err, err_len, "invalid expert entries/slot");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    if (mb && (!buf_ok(mb, ma->len) || !buf_ok(outb, (size_t)rows * 4))) {
        set_err(err, err_len, "second matrix/output too small");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    MvParams p{};
    p.cols = (int)cols;
    p.x = (const float *)in->ptr;
    p.expert = (const uint32_t *)entries->ptr;
    p.rows_per_expert = (int)rpe;
    // the number of whole experts the matrix holds bounds the device-side expert id
    p.expert_limit = (int)(ma->len / (stride * rpe));
    if (mb && (int)(mb->len / (stride * rpe)) < p.expert_limit) p.expert_limit = (int)(mb->len / (stride * rpe));
    p.nseg = 1;
    p.seg[0].w = (const uint8_t *)ma->ptr;
    p.seg[0].stride = stride;
    p.seg[0].y = (float *)outa->ptr;
    p.seg[0].rows = (int)rows;
    p.seg[0].fmt = (int)type;
    p.seg[0].expert_slot = (int)slot;
    plan_matvec(p, 512);
    ZH_TRY(launch_matvec(p, IN_PLAIN, out_mode, ctx->stream), what);
    if (mb) {
        p.seg[0].w = (const uint8_t *)mb->ptr;
        p.seg[0].y = (float *)outb->ptr;
        ZH_TRY(launch_matvec(p, IN_PLAIN, out_mode, ctx->stream), what);
    }
    return finish_op(ctx, what, err, err_len);
}

int ziggy_hip_indexed_matvec(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *m, const ZiggyHipBuffer *in,
                             ZiggyHipBuffer *out, uint32_t rows, uint32_t cols, const ZiggyHipBuffer *entries,
                             uint32_t slot, uint32_t rpe, int add_weighted, char *err, size_t err_len) {
    return indexed_common(ctx, type, m, nullptr, in, out, nullptr, rows, cols, entries, slot, rpe,
                          add_weighted ? OUT_WADD : OUT_STORE, "indexed_matvec", err, err_len);
}

int ziggy_hip_dual_indexed_matvec(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *ma,
                                  const ZiggyHipBuffer *mb, const ZiggyHipBuffer *in, ZiggyHipBuffer *oa,
                                  ZiggyHipBuffer *ob, uint32_t rows, uint32_t cols, const ZiggyHipBuffer *entries,
                                  uint32_t slot, uint32_t rpe, char *err, size_t err_len) {
    return indexed_common(ctx, type, ma, mb, in, oa, ob, rows, cols, entries, slot, rpe, OUT_STORE,
                          "dual_indexed_matvec", err, err_len);
}

#define ZH_DEFINE_INDEXED(sfx, TYPE)                                                                                   \
    int ziggy_hip_indexed_matvec_##sfx##_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *m, const ZiggyHipBuffer *in, \
                                             ZiggyHipBuffer *out, uint32_t rows, uint32_t cols,                      \
                                             const ZiggyHipBuffer *e, uint32_t slot, uint32_t rpe, char *err,        \
                                             size_t err_len) {                                                       \
        return ziggy_hip_indexed_matvec(ctx, TYPE, m, in, out, rows, cols, e, slot, rpe, 0, err, err_len);           \
    }                                                                                                                \
    int ziggy_hip_indexed_matvec_##sfx##_add_weighted_f32(                                                           \
        ZiggyHipContext *ctx, const ZiggyHipBuffer *m, const ZiggyHipBuffer *in, ZiggyHipBuffer *out, uint32_t rows, \
        uint32_t cols, const ZiggyHipBuffer *e, uint32_t slot, uint32_t rpe, char *err, size_t err_len) {            \
        return ziggy_hip_indexed_matvec(ctx, TYPE, m, in, out, rows, cols, e, slot, rpe, 1, err, err_len);           \
    }
ZH_DEFINE_INDEXED(iq4_xs, ZIGGY_HIP_TYPE_IQ4_XS)
ZH_DEFINE_INDEXED(q3k, ZIGGY_HIP_TYPE_Q3_K)

int ziggy_hip_dual_indexed_matvec_q3k_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *ma, const ZiggyHipBuffer *mb,
                                          const ZiggyHipBuffer *in, ZiggyHipBuffer *oa, ZiggyHipBuffer *ob,
                                          uint32_t rows, uint32_t cols, const ZiggyHipBuffer *e, uint32_t slot,
                                          uint32_t rpe, char *err, size_t err_len) {
    return ziggy_hip_dual_indexed_matvec(ctx, ZIGGY_HIP_TYPE_Q3_K, ma, mb, in, oa, ob, rows, cols, e, slot, rpe, err,
                                         err_len);
}

// ---------------- elementwise / attention ----------------

static int rope_common(ZiggyHipContext *ctx, const ZiggyHipBuffer *src, size_t soff, ZiggyHipBuffer *dst,
                       size_t doff, uint32_t heads, uint32_t hd, uint32_t rope_dim, uint32_t pos, float base,
                       uint32_t style, char *err, size_t err_len) {
    const size_t n = (size_t)heads * hd * 4;
    if (!ctx || !buf_ok(src, soff + n) || !buf_ok(dst, doff + n) || (soff % 4) || (doff % 4) || rope_dim > hd ||
        style > 1) {
        set_err(err, err_len, "invalid rope arguments");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    const float *denom = nullptr;
    ZH_TRY(ctx_rope_denom(ctx, base, (int)(rope_dim < hd ? rope_dim : hd), &denom), "rope table");
    ZH_TRY(launch_rope((const float *)((const char *)src->ptr + soff), (float *)((char *)dst->ptr + doff), (int)heads,
                       (int)hd, (int)rope_dim, (int)pos, denom, (int)style, ctx->stream),
           "apply_rope");
    return finish_op(ctx, "apply_rope", err, err_len);
}

int ziggy_hip_apply_rope_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *v, uint32_t heads, uint32_t hd, uint32_t rope_dim,
                             uint32_t pos, float base, uint32_t style, char *err, size_t err_len) {
    return rope_common(ctx, v, 0, v, 0, heads, hd, rope_dim, pos, base, style, err, err_len);
}

int ziggy_hip_apply_rope_at_offset_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *v, size_t off, uint32_t heads,
                                       uint32_t hd, uint32_t rope_dim, uint32_t pos, float base, uint32_t style,
                                       char *err, size_t err_len) {
    return rope_common(ctx, v, off, v, off, heads, hd, rope_dim, pos, base, style, err, err_len);
}

int ziggy_hip_apply_rope_to_dst_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *src, ZiggyHipBuffer *dst,
                                    size_t doff, uint32_t heads, uint32_t hd, uint32_t rope_dim, uint32_t pos,
                                    float base, uint32_t style, char *err, size_t err_len) {
    return rope_common(ctx, src, 0, dst, doff, heads, hd, rope_dim, pos, base, style, err, err_len);
}

int ziggy_hip_store_kv_half(ZiggyHipContext *ctx, const ZiggyHipBuffer *src, ZiggyHipBuffer *dst, size_t doff_el,
                            uint32_t count, char *err, size_t err_len) {
    if (!ctx || !buf_ok(src, (size_t)count * 4) || !buf_ok(dst, (doff_el + count) * 2)) {
        set_err(err, err_len, "invalid store_kv_half arguments");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    ZH_TRY(launch_store_kv_half((const float *)src->ptr, (__half *)dst->ptr + doff_el, (int)count, ctx->stream),
           "store_kv_half");
    return finish_op(ctx, "store_kv_half", err, err_len);
}

int ziggy_hip_attention_fused_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *q, const ZiggyHipBuffer *kc,
                                  const ZiggyHipBuffer *vc, ZiggyHipBuffer *out, uint32_t heads, uint32_t heads_kv,
                                  uint32_t hd, uint32_t kv_dim, uint32_t ctx_len, uint32_t pos, uint32_t layer_base,
                                  uint32_t window_start, float scale, float softcap, char *err, size_t err_len) {
    if (!ctx || heads_kv > kCtxCounters) {
        set_err(err, err_len, "unsupported attention shape");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    AttnParams p{};
    const int st = attention_call_params(q, kc, vc, out, heads, heads_kv, hd, kv_dim, ctx_len, pos, layer_base,
                                         window_start, scale, softcap, &p, err, err_len);
    if (st != ZIGGY_HIP_OK) return st;
    p.counters = ctx->counters;
    p.page_table = ctx->identity_pages;
    p.page_shift = kKvPageShift;
    const size_t need = attention_scratch_floats((int)heads, (int)hd, p.max_splits) * 4;
    if (need > ctx->scratch_len) {
        set_err(err, err_len, "context too long for the context scratch (%zu bytes)", need);
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    p.part_o = (float *)ctx->scratch;
    p.part_ml = p.part_o + (size_t)heads * p.max_splits * 8 * hd;
    ZH_TRY(launch_attention(p, ctx->stream), "attention");
    return finish_op(ctx, "attention", err, err_len);
}

#define ZH_N_CHECK(cond)                                      \
    if (!(cond)) {                                            \
        set_err(err, err_len, "invalid arguments");          \
        return ZIGGY_HIP_INVALID_ARGUMENT;                    \
    }

int ziggy_hip_silu_mul_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *g, const ZiggyHipBuffer *u, uint32_t n, char *err,
                           size_t err_len) {
    ZH_N_CHECK(ctx && buf_ok(g, (size_t)n * 4) && buf_ok(u, (size_t)n * 4));
    ZH_TRY(launch_silu_mul((float *)g->ptr, (const float *)u->ptr, (int)n, ctx->stream), "silu_mul");
    return finish_op(ctx, "silu_mul", err, err_len);
}

int ziggy_hip_add_in_place_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *d, const ZiggyHipBuffer *s, uint32_t n,
                               char *err, size_t err_len) {
    ZH_N_CHECK(ctx && buf_ok(d, (size_t)n * 4) && buf_ok(s, (size_t)n * 4));
    ZH_TRY(launch_add((float *)d->ptr, (const float *)s->ptr, (int)n, ctx->stream), "add_in_place");
    return finish_op(ctx, "add_in_place", err, err_len);
}

int ziggy_hip_add_bias_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *d, const ZiggyHipBuffer *b, uint32_t n, char *err,
                           size_t err_len) {
    return ziggy_hip_add_in_place_f32(ctx, d, b, n, err, err_len);
}

int ziggy_hip_rms_norm_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *in, const ZiggyHipBuffer *w,
                           ZiggyHipBuffer *out, uint32_t n, float eps, float off, char *err, size_t err_len) {
    ZH_N_CHECK(ctx && n > 0 && buf_ok(in, (size_t)n * 4) && buf_ok(w, (size_t)n * 4) && buf_ok(out, (size_t)n * 4));
    ZH_TRY(launch_rms_norm((const float *)in->ptr, (const float *)w->ptr, (float *)out->ptr, (int)n, eps, off,
                           ctx->stream),
           "rms_norm");
    return finish_op(ctx, "rms_norm", err, err_len);
}

int ziggy_hip_rms_norm_per_head_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *in, const ZiggyHipBuffer *w,
                                    ZiggyHipBuffer *out, uint32_t heads, uint32_t hd, float eps, float off, char *err,
                                    size_t err_len) {
    ZH_N_CHECK(ctx && heads > 0 && hd > 0 && buf_ok(in, (size_t)heads * hd * 4) && buf_ok(w, (size_t)hd * 4) &&
               buf_ok(out, (size_t)heads * hd * 4));
    ZH_TRY(launch_rms_norm_per_head((const float *)in->ptr, (const float *)w->ptr, (float *)out->ptr, (int)heads,
                                    (int)hd, eps, off, ctx->stream),
           "rms_norm_per_head");
    return finish_op(ctx, "rms_norm_per_head", err, err_len);
}

int ziggy_hip_argmax_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *in, ZiggyHipBuffer *tok, uint32_t n, char *err,
                         size_t err_len) {
    ZH_N_CHECK(ctx && n > 0 && buf_ok(in, (size_t)n * 4) && buf_ok(tok, 4));
    ZH_TRY(launch_argmax((const float *)in->ptr, (int)n, (uint32_t *)tok->ptr, (unsigned long long *)ctx->scratch,
                         ctx->stream),
           "argmax");
    return finish_op(ctx, "argmax", err, err_len);
}

int ziggy_hip_topk_f32(ZiggyHipContext *ctx, const ZiggyHipBuffer *in, ZiggyHipBuffer *entries, uint32_t n,
                       uint32_t k, char *err, size_t err_len) {
    ZH_N_CHECK(ctx && n > 0 && k > 0 && k <= 64 && k <= n && buf_ok(in, (size_t)n * 4) && buf_ok(entries, (size_t)k * 8));
    if (n <= 262144) {
        // two-stage shortlist (per-slice top k, then the top k of those); packed keys in the context scratch
        ZH_N_CHECK(shortlist_scratch_keys((int)n) * 8 <= ctx->scratch_len);
        ZH_TRY(launch_shortlist((const float *)in->ptr, (int)n, (int)k, (unsigned long long *)ctx->scratch,
                                (uint32_t *)entries->ptr, ctx->stream),
               "topk");
        return finish_op(ctx, "topk", err, err_len);
    }
    // longer inputs: k rounds of a workgroup argmax; entries in the context
    // scratch (k slots + per-value flags), then copied out
    ZH_N_CHECK(64 * 8 + (size_t)n <= ctx->scratch_len);
    ZH_TRY(launch_topk((const float *)in->ptr, (int)n, (int)k, ctx->scratch, ctx->stream), "topk");
    ZH_TRY(hipMemcpyAsync(entries->ptr, ctx->scratch, (size_t)k * 8, hipMemcpyDeviceToDevice, ctx->stream), "topk");
    return finish_op(ctx, "topk", err, err_len);
}

int ziggy_hip_normalize_topk_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *entries, uint32_t k, bool apply_softmax,
                                 bool normalize, float scale, char *err, size_t err_len) {
    ZH_N_CHECK(ctx && k > 0 && k <= 64 && buf_ok(entries, (size_t)k * 8));
    ZH_TRY(launch_normalize_topk(entries->ptr, (int)k, apply_softmax ? 1 : 0, normalize ? 1 : 0, scale, ctx->stream),
           "normalize_topk");
    return finish_op(ctx, "normalize_topk", err, err_len);
}

int ziggy_hip_weighted_sum_topk_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *d, const ZiggyHipBuffer *s,
                                    const ZiggyHipBuffer *entries, uint32_t n, uint32_t slot, char *err,
                                    size_t err_len) {
    ZH_N_CHECK(ctx && buf_ok(d, (size_t)n * 4) && buf_ok(s, (size_t)n * 4) && buf_ok(entries, (size_t)(slot + 1) * 8));
    ZH_TRY(launch_weighted_sum_topk((float *)d->ptr, (const float *)s->ptr, entries->ptr, (int)n, (int)slot,
                                    ctx->stream),
           "weighted_sum_topk");
    return finish_op(ctx, "weighted_sum_topk", err, err_len);
}

int ziggy_hip_sigmoid_scale_add_f32(ZiggyHipContext *ctx, ZiggyHipBuffer *d, const ZiggyHipBuffer *s,
                                    const ZiggyHipBuffer *scalar, uint32_t n, char *err, size_t err_len) {
    ZH_N_CHECK(ctx && buf_ok(d, (size_t)n * 4) && buf_ok(s, (size_t)n * 4) && buf_ok(scalar, 4));
    ZH_TRY(launch_sigmoid_scale_add((float *)d->ptr, (const float *)s->ptr, (const float *)scalar->ptr, (int)n,
                                    ctx->stream),
           "sigmoid_scale_add");
    return finish_op(ctx, "sigmoid_scale_add", err, err_len);
}

}  // extern "C"

extern "C" int ziggy_hip_time_matvec(ZiggyHipContext *ctx, uint32_t type, const ZiggyHipBuffer *m, uint32_t copies,
                                     size_t copy_stride, const ZiggyHipBuffer *in, ZiggyHipBuffer *out, uint32_t rows,
                                     uint32_t cols, uint32_t iterations, uint64_t *avg_ns, char *err,
                                     size_t err_len) {
    uint64_t stride;
    if (copies == 0 || iterations == 0 || !avg_ns) {
        set_err(err, err_len, "invalid time_matvec arguments");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    int st = check_matvec(ctx, type, m, (size_t)(copies - 1) * copy_stride, in, out, 0, rows, cols, &stride, err,
                          err_len, kMaxMatvecCols);
    if (st) return st;
    if (copy_stride < stride * rows) {
        set_err(err, err_len, "copy stride smaller than one matrix");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    hipEvent_t e0, e1;
    ZH_TRY(hipEventCreate(&e0), "time_matvec");
    if (hipEventCreate(&e1) != hipSuccess) {
        hipEventDestroy(e0);
        set_err(err, err_len, "event creation failed");
        return ZIGGY_HIP_EXECUTION_FAILED;
    }
    MvParams p{};
    p.nseg = 1;
    p.seg[0].stride = stride;
    p.seg[0].y = (float *)out->ptr;
    p.seg[0].rows = (int)rows;
    p.seg[0].fmt = (int)type;
    p.cols = (int)cols;
    p.x = (const float *)in->ptr;
    // back-to-back launches rotating over the copies, between one event pair
    float ms = 0.f;
    hipError_t e = hipEventRecord(e0, ctx->stream);
    for (uint32_t i = 0; i < iterations && e == hipSuccess; i++) {
        p.seg[0].w = (const uint8_t *)m->ptr + (size_t)(i % copies) * copy_stride;
        e = launch_matvec(p, IN_PLAIN, OUT_STORE, ctx->stream);
    }
    if (e == hipSuccess) e = hipEventRecord(e1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (e != hipSuccess) return hip_fail(e, "time_matvec", err, err_len);
    *avg_ns = (uint64_t)((double)ms * 1e6 / iterations);
    return ZIGGY_HIP_OK;
}
