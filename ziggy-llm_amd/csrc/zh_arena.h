// zh_arena.h -- host-side weight residency shared by the decode session and
// the MoE stack: every tensor of a model goes into one HBM arena, raw GGUF
// bytes, 256-byte aligned (DenseTensorStore.populate / prewarm,
// runtime/gpu/metal/tensor_store.zig:39-144).
#pragma once

#include <stdint.h>

#include <utility>
#include <vector>

#include "ziggy_hip.h"
#include "zh_internal.h"

namespace zh {

// One resident tensor: device rows of `stride` bytes.
struct DT {
    const uint8_t *p = nullptr;
    uint64_t rows = 0, cols = 0, stride = 0;
    int type = -1;
    bool present = false;
};

// Bytes per row of a tensor type (tensorRowByteSize, model/loader.zig:3325-3389,
// with the block sizes of gguf.zig:531-567); -1 for types off this path.
inline int row_bytes(uint32_t type, uint64_t cols, uint64_t *out) {
    switch (type) {
    case ZIGGY_HIP_TYPE_F32: *out = cols * 4; return 0;
    case ZIGGY_HIP_TYPE_F16: *out = cols * 2; return 0;
    case ZIGGY_HIP_TYPE_Q8_0: if (cols % 32) return -1; *out = cols / 32 * 34; return 0;
    case ZIGGY_HIP_TYPE_Q3_K: if (cols % 256) return -1; *out = cols / 256 * 110; return 0;
    case ZIGGY_HIP_TYPE_Q4_K: if (cols % 256) return -1; *out = cols / 256 * 144; return 0;
    case ZIGGY_HIP_TYPE_Q6_K: if (cols % 256) return -1; *out = cols / 256 * 210; return 0;
    case ZIGGY_HIP_TYPE_IQ4_XS: if (cols % 256) return -1; *out = cols / 256 * 136; return 0;
    default: return -1;
    }
}

using ArenaTodo = std::vector<std::pair<const ZiggyHipTensorDesc *, DT *>>;

// Reserves arena space for tensor d (want_rows / want_cols 0 = any): a missing
// tensor is accepted unless required; f32_only restricts the type; matvec
// operands need cols a multiple of 64 (the session limits the rows whose
// input is normed to one team; longer rows run as column windows).  The device
// address is an offset until the arena exists (fixed up by the caller).
inline bool take_tensor(const ZiggyHipTensorDesc *d, uint64_t want_rows, uint64_t want_cols, bool required,
                        bool f32_only, DT *out, size_t *arena_off, ArenaTodo &todo) {
    if (!d || !d->data) return !required;
    uint64_t stride;
    if (row_bytes(d->tensor_type, d->cols, &stride)) return false;
    if (f32_only && d->tensor_type != ZIGGY_HIP_TYPE_F32) return false;
    if ((want_rows && d->rows != want_rows) || (want_cols && d->cols != want_cols)) return false;
    if (!f32_only && (d->cols % 64 || d->cols > (uint64_t)kMaxMatvecRowLen)) return false;
    out->rows = d->rows;
    out->cols = d->cols;
    out->stride = stride;
    out->type = (int)d->tensor_type;
    out->present = true;
    out->p = reinterpret_cast<const uint8_t *>(*arena_off);  // fixed up after the arena is allocated
    *arena_off += (stride * d->rows + 255) & ~(size_t)255;
    todo.push_back({d, out});
    return true;
}

}  // namespace zh
