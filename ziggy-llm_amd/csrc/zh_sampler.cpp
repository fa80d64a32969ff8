// zh_sampler.cpp -- the reference's CPU sampler, on the host side of the
// boundary: the device computes the logits and their top-k shortlist
// (zh_sample.hip); the draw itself runs here, as in the reference, where
// sampleShortlist (sampling.zig:31-45) runs on the CPU over the GPU session's
// shortlist (model/loader.zig:2140-2150).
//
// The policy is sampleCollectedCandidates (sampling.zig:54-110), in the same
// order and precision: repeat penalty in f32, weights exp((l - max) / T) and
// their sums in f64, min-p truncation in candidate order, top-p truncation
// after a stable sort by weight, and the draw `target = u * total` against
// the running sum.  The caller supplies u, the value random.float(f64) gives
// the reference, so runs are reproducible from the caller's generator.
#include <math.h>

#include <algorithm>
#include <vector>

#include "ziggy_hip.h"

namespace {

struct Cand {
    uint32_t id;
    float logit;
    double weight;
};

// applyRepeatPenalty (sampling.zig:121-128)
float repeat_penalty(float logit, uint32_t id, const uint32_t *recent, uint32_t n, float penalty) {
    if (penalty <= 1.0f) return logit;
    for (uint32_t i = 0; i < n; i++) {
        if (recent[i] != id) continue;
        return logit < 0 ? logit * penalty : logit / penalty;
    }
    return logit;
}

// fallbackToken (sampling.zig:112-119): the first candidate of the largest logit
uint32_t fallback(const Cand *c, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (c[i].logit > c[best].logit) best = i;
    return c[best].id;
}

double sum_weights(const Cand *c, size_t n) {
    double t = 0;
    for (size_t i = 0; i < n; i++) t += c[i].weight;
    return t;
}

// sampleCollectedCandidates (sampling.zig:54-110)
uint32_t sample_collected(Cand *c, size_t n, const uint32_t *recent, uint32_t nrecent, const ZiggyHipSamplingOptions &o,
                          double u) {
    if (n == 0) return 0;
    float max_logit = -INFINITY;
    uint32_t fb_token = c[0].id;
    float fb_logit = c[0].logit;
    for (size_t i = 0; i < n; i++) {
        const float a = repeat_penalty(c[i].logit, c[i].id, recent, nrecent, o.repeat_penalty);
        c[i].logit = a;
        if (a > fb_logit) {
            fb_logit = a;
            fb_token = c[i].id;
        }
        max_logit = fmaxf(max_logit, a);
    }
    double total = 0;
    for (size_t i = 0; i < n; i++) {
        const double shifted = ((double)c[i].logit - (double)max_logit) / (double)o.temperature;
        c[i].weight = exp(shifted);
        total += c[i].weight;
    }
    if (total <= 0 || !isfinite(total)) return fb_token;
    size_t active = n;
    if (o.min_p > 0) {
        // truncateByMinP (sampling.zig:176-190): keep weights >= max * min_p, in order; at least one
        double max_w = 0;
        for (size_t i = 0; i < active; i++) max_w = std::max(max_w, c[i].weight);
        const double threshold = max_w * (double)o.min_p;
        size_t kept = 0;
        for (size_t i = 0; i < active; i++)
            if (c[i].weight >= threshold) c[kept++] = c[i];
        active = std::max<size_t>(1, kept);
        total = sum_weights(c, active);
        if (total <= 0 || !isfinite(total)) return fallback(c, active);
    }
    if (o.top_p < 1.0f) {
        // a stable sort by descending weight (lessSampleCandidate, :192-194), then
        // truncateByTopP (:167-174): the shortest prefix whose share reaches top_p
        std::stable_sort(c, c + active, [](const Cand &a, const Cand &b) { return a.weight > b.weight; });
        double cum = 0;
        size_t kept = active;
        for (size_t i = 0; i < active; i++) {
            cum += c[i].weight;
            if (cum / total >= (double)o.top_p) {
                kept = i + 1;
                break;
            }
        }
        active = kept;
        total = sum_weights(c, active);
        if (total <= 0 || !isfinite(total)) return fallback(c, active);
    }
    const double target = u * total;
    double cum = 0;
    for (size_t i = 0; i < active; i++) {
        cum += c[i].weight;
        if (target <= cum) return c[i].id;
    }
    return c[active - 1].id;
}

bool options_ok(const ZiggyHipSamplingOptions *o, double u) { return o && u >= 0.0 && u < 1.0; }

}  // namespace

extern "C" uint32_t ziggy_hip_shortlist_len(const ZiggyHipSamplingOptions *o, uint32_t vocab) {
    // shortlistLenFor (sampling.zig:47-52)
    if (!o || vocab == 0 || o->temperature <= 0) return 0;
    const uint32_t k = o->top_k == 0 ? 64u : o->top_k;
    return std::min(vocab, std::min(k, 64u));
}

extern "C" int ziggy_hip_sample_shortlist(const ZiggyHipShortlistEntry *entries, uint32_t count, const uint32_t *recent,
                                          uint32_t recent_count, const ZiggyHipSamplingOptions *o, double u,
                                          uint32_t *out_token) {
    if (!out_token || !options_ok(o, u) || (count && !entries) || (recent_count && !recent))
        return ZIGGY_HIP_INVALID_ARGUMENT;
    // sampleShortlist (sampling.zig:31-45): an empty shortlist gives token 0
    if (count == 0) {
        *out_token = 0;
        return ZIGGY_HIP_OK;
    }
    std::vector<Cand> c(count);
    for (uint32_t i = 0; i < count; i++) c[i] = Cand{entries[i].token_id, entries[i].logit, 0.0};
    *out_token = sample_collected(c.data(), count, recent, recent_count, *o, u);
    return ZIGGY_HIP_OK;
}

extern "C" int ziggy_hip_sample_logits(const float *logits, uint32_t count, const uint32_t *recent,
                                       uint32_t recent_count, const ZiggyHipSamplingOptions *o, double u,
                                       uint32_t *out_token) {
    if (!out_token || !logits || count == 0 || !options_ok(o, u) || (recent_count && !recent))
        return ZIGGY_HIP_INVALID_ARGUMENT;
    // sampleToken (sampling.zig:11-29); argmax (:196-206) keeps the first maximum
    auto argmax = [&]() {
        uint32_t best = 0;
        for (uint32_t i = 1; i < count; i++)
            if (logits[i] > logits[best]) best = i;
        return best;
    };
    if (o->temperature <= 0) {
        *out_token = argmax();
        return ZIGGY_HIP_OK;
    }
    const uint32_t top_k = o->top_k == 0 ? count : std::min(o->top_k, count);
    std::vector<Cand> c;
    c.reserve(top_k);
    if (top_k < count) {
        // collectTopKCandidates (sampling.zig:139-164): descending logits by
        // insertion, a later equal logit behind an earlier one
        for (uint32_t i = 0; i < count; i++) {
            const Cand cand{i, logits[i], 0.0};
            size_t pos;
            if (c.size() < top_k) {
                c.push_back(cand);
                pos = c.size() - 1;
            } else {
                if (cand.logit <= c[top_k - 1].logit) continue;
                c[top_k - 1] = cand;
                pos = top_k - 1;
            }
            while (pos > 0 && c[pos].logit > c[pos - 1].logit) {
                std::swap(c[pos], c[pos - 1]);
                pos--;
            }
        }
    } else {
        for (uint32_t i = 0; i < count; i++) c.push_back(Cand{i, logits[i], 0.0});
    }
    if (c.empty()) {
        *out_token = argmax();
        return ZIGGY_HIP_OK;
    }
    *out_token = sample_collected(c.data(), c.size(), recent, recent_count, *o, u);
    return ZIGGY_HIP_OK;
}
