// zh_profile.cpp -- the decode profiler's summary (runtime/metal_profile.zig).
//
// A profiled decode (ziggy_hip_session_profile_decode) emits a stream of
// records: token markers and one record per timed piece of work, under the
// reference's Category names with its ShapeDesc fields.  This file folds such
// a stream as the reference's Profiler does (beginDecodeToken /
// endDecodeToken, record, recordWithShape, recordCommitWaitGpu,
// recordMoonQuantProjection: metal_profile.zig:120-199) and prints its
// renderSummary text (metal_profile.zig:201-316), key for key, so a reader of
// the reference's report parses this one unchanged.  Host code only.
#include <algorithm>
#include <cinttypes>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "ziggy_hip.h"

namespace {

constexpr int kCategories = 9;
const char *const kLabels[kCategories] = {"projections",     "attention",     "kv_writes",
                                          "normalization",   "elementwise_ops", "output_reduce",
                                          "commit_wait",     "host_readback", "cpu_sampling"};

// (category, rows, cols, depth, extra, tensor_type): the reference's ShapeKey
typedef std::tuple<int, uint64_t, uint64_t, uint64_t, uint64_t, uint32_t> ShapeKey;
struct Stats {
    uint64_t ns = 0, calls = 0;
};

struct Folded {
    Stats cat[kCategories];
    std::vector<std::vector<uint64_t>> tokens;  // per ended token: the nine category totals
    std::vector<uint64_t> moon_tokens, gpu_tokens;
    std::map<ShapeKey, Stats> shapes, moon_shapes;
    uint64_t cur[kCategories] = {};
    uint64_t cur_moon = 0, cur_gpu = 0, moon_ns = 0, moon_calls = 0, gpu_ns = 0;
    bool active = false;
};

ShapeKey key_of(int category, const ZiggyHipProfileRecord &r) {
    return ShapeKey(category, r.rows, r.cols, r.depth, r.extra, r.tensor_type);
}

// Returns false on a record kind the profiler does not know.
bool fold(Folded &f, const ZiggyHipProfileRecord &r) {
    switch (r.kind) {
    case ZIGGY_HIP_PROFILE_TOKEN_BEGIN:  // beginDecodeToken: a fresh breakdown, even over an open one
        std::fill(f.cur, f.cur + kCategories, 0);
        f.cur_moon = f.cur_gpu = 0;
        f.active = true;
        return true;
    case ZIGGY_HIP_PROFILE_TOKEN_END:  // endDecodeToken
        if (f.active) {
            f.tokens.emplace_back(f.cur, f.cur + kCategories);
            f.moon_tokens.push_back(f.cur_moon);
            f.gpu_tokens.push_back(f.cur_gpu);
            std::fill(f.cur, f.cur + kCategories, 0);
            f.cur_moon = f.cur_gpu = 0;
            f.active = false;
        }
        return true;
    case ZIGGY_HIP_PROFILE_COMMIT_WAIT_GPU:  // recordCommitWaitGpu: zero durations are not counted
        if (f.active && r.ns) {
            f.gpu_ns += r.ns;
            f.cur_gpu += r.ns;
        }
        return true;
    case ZIGGY_HIP_PROFILE_MOON_QUANT:  // recordMoonQuantProjection: its shapes key as projections
        if (f.active) {
            f.moon_ns += r.ns;
            f.moon_calls++;
            f.cur_moon += r.ns;
            Stats &s = f.moon_shapes[key_of(ZIGGY_HIP_PROFILE_PROJECTIONS, r)];
            s.ns += r.ns;
            s.calls++;
        }
        return true;
    default:
        if (r.kind >= (uint32_t)kCategories) return false;
        if (f.active) {  // record, then the shape of recordWithShape
            f.cat[r.kind].ns += r.ns;
            f.cat[r.kind].calls++;
            f.cur[r.kind] += r.ns;
            if (r.has_shape) {
                Stats &s = f.shapes[key_of((int)r.kind, r)];
                s.ns += r.ns;
                s.calls++;
            }
        }
        return true;
    }
}

double pct(uint64_t part, uint64_t whole) { return whole ? (double)part * 100.0 / (double)whole : 0.0; }

struct Out {
    std::string s;
    void add(const char *fmt, ...) __attribute__((format(printf, 2, 3))) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        const int n = vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        if (n > 0) s.append(buf, std::min((size_t)n, sizeof(buf) - 1));
    }
};

// lessShapeEntry: the larger total first, then the more calls (the key breaks
// the remaining ties, which the reference leaves to its hash map's order)
std::vector<std::pair<ShapeKey, Stats>> sorted(const std::map<ShapeKey, Stats> &m) {
    std::vector<std::pair<ShapeKey, Stats>> v(m.begin(), m.end());
    std::stable_sort(v.begin(), v.end(), [](const auto &a, const auto &b) {
        if (a.second.ns != b.second.ns) return a.second.ns > b.second.ns;
        return a.second.calls > b.second.calls;
    });
    return v;
}

std::string render(const Folded &f) {
    Out o;
    uint64_t total = 0;
    for (const Stats &c : f.cat) total += c.ns;
    o.add("metal_decode_profile_enabled=true\n");
    o.add("profiled_decode_tokens=%zu\n", f.tokens.size());
    o.add("profiled_decode_ns=%" PRIu64 "\n", total);
    o.add("moon_quant.profile.total_ns=%" PRIu64 "\n", f.moon_ns);
    o.add("moon_quant.profile.calls=%" PRIu64 "\n", f.moon_calls);
    o.add("moon_quant.profile.share_of_decode_pct=%.3f\n", pct(f.moon_ns, total));
    o.add("profile.commit_wait.gpu_ns=%" PRIu64 "\nprofile.commit_wait.gpu_share_of_decode_pct=%.3f\n", f.gpu_ns,
          pct(f.gpu_ns, total));
    for (int c = 0; c < kCategories; c++)
        o.add("profile.%s.ns=%" PRIu64 "\nprofile.%s.share_pct=%.3f\nprofile.%s.calls=%" PRIu64 "\n", kLabels[c],
              f.cat[c].ns, kLabels[c], pct(f.cat[c].ns, total), kLabels[c], f.cat[c].calls);
    // topCategoryBreakdown: three slots that start as (projections, 0); a
    // category takes the first slot it strictly exceeds, shifting the rest down
    int top_c[3] = {0, 0, 0};
    uint64_t top_ns[3] = {0, 0, 0};
    for (int c = 0; c < kCategories; c++) {
        for (int i = 0; i < 3; i++) {
            if (f.cat[c].ns > top_ns[i]) {
                for (int j = 2; j > i; j--) top_c[j] = top_c[j - 1], top_ns[j] = top_ns[j - 1];
                top_c[i] = c;
                top_ns[i] = f.cat[c].ns;
                break;
            }
        }
    }
    for (int i = 0; i < 3; i++)
        o.add("profile.top_bottleneck_%d=%s:%" PRIu64 "ns:%.3fpct\n", i + 1, kLabels[top_c[i]], top_ns[i],
              pct(top_ns[i], total));
    const auto shapes = sorted(f.shapes);
    for (size_t i = 0; i < shapes.size() && i < 8; i++) {
        const ShapeKey &k = shapes[i].first;
        o.add("profile.shape_%zu=%s:rows=%" PRIu64 ":cols=%" PRIu64 ":depth=%" PRIu64 ":extra=%" PRIu64
              ":tensor_type=%u:calls=%" PRIu64 ":ns=%" PRIu64 "\n",
              i + 1, kLabels[std::get<0>(k)], std::get<1>(k), std::get<2>(k), std::get<3>(k), std::get<4>(k),
              std::get<5>(k), shapes[i].second.calls, shapes[i].second.ns);
    }
    const auto moon = sorted(f.moon_shapes);
    for (size_t i = 0; i < moon.size() && i < 4; i++) {
        const ShapeKey &k = moon[i].first;
        o.add("moon_quant.profile.shape_%zu=rows=%" PRIu64 ":cols=%" PRIu64 ":depth=%" PRIu64 ":extra=%" PRIu64
              ":tensor_type=%u:calls=%" PRIu64 ":ns=%" PRIu64 "\n",
              i + 1, std::get<1>(k), std::get<2>(k), std::get<3>(k), std::get<4>(k), std::get<5>(k),
              moon[i].second.calls, moon[i].second.ns);
    }
    for (size_t t = 0; t < f.tokens.size(); t++) {
        uint64_t tt = 0;
        for (uint64_t v : f.tokens[t]) tt += v;
        o.add("profile.token_%zu.total_ns=%" PRIu64 "\n", t, tt);
        for (int c = 0; c < kCategories; c++)
            o.add("profile.token_%zu.%s.ns=%" PRIu64 "\n", t, kLabels[c], f.tokens[t][c]);
        o.add("moon_quant.profile.token_%zu.ns=%" PRIu64 "\n", t, f.moon_tokens[t]);
        o.add("profile.token_%zu.commit_wait.gpu_ns=%" PRIu64 "\n", t, f.gpu_tokens[t]);
    }
    return o.s;
}

}  // namespace

extern "C" int ziggy_hip_profile_render(const ZiggyHipProfileRecord *records, size_t count, char *out,
                                        size_t capacity, size_t *out_length) {
    if ((!records && count) || !out_length) return ZIGGY_HIP_INVALID_ARGUMENT;
    Folded f;
    for (size_t i = 0; i < count; i++)
        if (!fold(f, records[i])) return ZIGGY_HIP_INVALID_ARGUMENT;
    const std::string s = render(f);
    *out_length = s.size();  // without the terminating zero
    if (!out || capacity < s.size() + 1) return ZIGGY_HIP_INVALID_ARGUMENT;
    memcpy(out, s.c_str(), s.size() + 1);
    return ZIGGY_HIP_OK;
}
