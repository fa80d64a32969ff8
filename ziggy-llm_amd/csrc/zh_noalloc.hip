// zh_noalloc.hip -- the allocation-free variant of the bridge-level decode
// attention (ziggy_hip_attention_fused_f32_noalloc).
//
// The split-K attention kernel needs scratch beyond its inputs and output:
// the per-split partial outputs and (m, l) pairs, and one arrival counter per
// kv head.  The context entry point takes them from the context's scratch
// allocation; this one takes them from `scratch`, a file-scope device array
// of fixed size, so the call itself allocates nothing (for callers under
// graph capture or in loops that must not allocate).  Each device holds its
// own copy of the array until the process ends; its address on each device
// comes from hipGetSymbolAddress, taken once per device at context creation.
// Calls on one device share the array: calls that overlap on one device
// race, and every call clears the counters before its launch.
#include <mutex>

#include "zh_internal.h"

namespace {

constexpr size_t kScratchBytes = 4u << 20;          // counters + partials, per device
constexpr size_t kCounterBytes = 4096;              // up to 1024 kv heads' arrival counters
constexpr size_t kPartialBytes = kScratchBytes - kCounterBytes;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
unsigned char *g_ptr[kMaxDevices];  // scratch's address on each device (null until resolved)

}  // namespace

namespace zh {

int noalloc_init_device(int device, char *err, size_t err_len) {
    if (device < 0 || device >= kMaxDevices) {
        set_err(err, err_len, "device index %d beyond the %d devices the static scratch table holds", device,
                kMaxDevices);
        return ZIGGY_HIP_INITIALIZATION_FAILED;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[device]) return ZIGGY_HIP_OK;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        set_err(err, err_len, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
        return ZIGGY_HIP_INITIALIZATION_FAILED;
    }
    g_ptr[device] = static_cast<unsigned char *>(ptr);
    return ZIGGY_HIP_OK;
}

}  // namespace zh

using namespace zh;

extern "C" int ziggy_hip_attention_fused_f32_noalloc(ZiggyHipContext *ctx, const ZiggyHipBuffer *q,
                                                     const ZiggyHipBuffer *kc, const ZiggyHipBuffer *vc,
                                                     ZiggyHipBuffer *out, uint32_t heads, uint32_t heads_kv,
                                                     uint32_t hd, uint32_t kv_dim, uint32_t ctx_len, uint32_t pos,
                                                     uint32_t layer_base, uint32_t window_start, float scale,
                                                     float softcap, char *err, size_t err_len) {
    if (!ctx) {
        set_err(err, err_len, "null context");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    if ((size_t)heads_kv * sizeof(unsigned) > kCounterBytes) {
        set_err(err, err_len, "%u kv heads exceed the static scratch's %zu arrival counters", heads_kv,
                kCounterBytes / sizeof(unsigned));
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    AttnParams p{};
    const int st = attention_call_params(q, kc, vc, out, heads, heads_kv, hd, kv_dim, ctx_len, pos, layer_base,
                                         window_start, scale, softcap, &p, err, err_len);
    if (st != ZIGGY_HIP_OK) return st;
    // the kernel indexes partials [kv head][split][8][head_dim] and (m, l) pairs [kv head][split][8][2]
    const size_t slots = (size_t)heads_kv * p.max_splits * 8;
    const size_t part_o_bytes = slots * hd * 4, need = part_o_bytes + slots * 2 * 4;
    if (need > kPartialBytes) {
        set_err(err, err_len, "attention partials need %zu bytes, beyond the static scratch's %zu", need,
                kPartialBytes);
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    unsigned char *base = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        base = ctx->device >= 0 && ctx->device < kMaxDevices ? g_ptr[ctx->device] : nullptr;
    }
    if (!base) {
        set_err(err, err_len, "static scratch not resolved on device %d", ctx->device);
        return ZIGGY_HIP_INITIALIZATION_FAILED;
    }
    p.page_table = ctx->identity_pages;  // made at context creation: nothing allocated here
    p.page_shift = kKvPageShift;
    p.counters = reinterpret_cast<unsigned *>(base);
    p.part_o = reinterpret_cast<float *>(base + kCounterBytes);
    p.part_ml = reinterpret_cast<float *>(base + kCounterBytes + part_o_bytes);
    // the counters must start at zero: a fill kernel (no memset node, no allocation)
    ZH_TRY(launch_fill_u64(reinterpret_cast<unsigned long long *>(base), 0ull, (int)((heads_kv + 1) / 2),
                           ctx->stream),
           "attention counters");
    ZH_TRY(launch_attention(p, ctx->stream), "attention");
    return finish_op(ctx, "attention", err, err_len);
}
