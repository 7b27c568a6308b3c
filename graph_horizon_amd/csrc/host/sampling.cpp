// Host token sampling for the graph driver's generation loop: a restatement of the engine's
// sampling.rs:1-203. The engine samples on the host; the device only reduces the logits to an
// argmax (greedy) or to k candidates (read_topk) first, and the full read-back remains the
// fallback. Filters in the reference's order: repeat penalty -> temperature -> top-k ->
// top-p -> min-p -> inverse-CDF draw, all in FP32 with sequential sums, so that a draw is
// reproducible for a seed.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "internal.h"

using namespace gh;

namespace {

// sampling.rs's total order for candidates: (logit desc by f32 total order, index asc)
struct Cand {
    uint32_t idx;
    float logit;
};

bool cand_before(const Cand& a, const Cand& b) {
    const int ka = total_key(a.logit), kb = total_key(b.logit);
    return ka != kb ? ka > kb : a.idx < b.idx;
}

// argmax, sampling.rs:196-204: strict `>` from -inf, so the lowest index wins and an
// all -inf / NaN vector gives 0
uint32_t argmax_host(const float* l, uint64_t n) {
    uint64_t best = 0;
    float best_val = -INFINITY;
    for (uint64_t i = 0; i < n; ++i)
        if (l[i] > best_val) {
            best_val = l[i];
            best = i;
        }
    return (uint32_t)best;
}

uint32_t tail(std::vector<Cand>& cand, const gh_sampling* p, uint64_t* rng) {
    if (cand.empty()) return 0;
    const float max = cand[0].logit;
    std::vector<float> probs(cand.size());
    for (size_t i = 0; i < cand.size(); ++i) probs[i] = std::exp(cand[i].logit - max);
    float sum = 0.0f;
    for (float pr : probs) sum += pr;
    for (float& pr : probs) pr /= sum;
    if (p->top_p < 1.0f) {  // nucleus: the shortest prefix whose mass reaches top_p
        float cum = 0.0f;
        size_t cut = probs.size();
        for (size_t i = 0; i < probs.size(); ++i) {
            cum += probs[i];
            if (cum >= p->top_p) {
                cut = i + 1;
                break;
            }
        }
        cand.resize(cut);
        probs.resize(cut);
    }
    if (p->min_p > 0.0f) {  // the leading run at or above min_p x the peak (at least one)
        const float thr = p->min_p * probs[0];
        size_t keep = 0;
        while (keep < probs.size() && probs[keep] >= thr) ++keep;
        keep = std::max<size_t>(keep, 1);
        cand.resize(keep);
        probs.resize(keep);
    }
    sum = 0.0f;
    for (float pr : probs) sum += pr;
    const float r = gh_rng_next_f32(rng) * sum;
    float acc = 0.0f;
    for (size_t i = 0; i < probs.size(); ++i) {
        acc += probs[i];
        if (r < acc) return cand[i].idx;
    }
    return cand.back().idx;
}

}  // namespace

uint64_t gh_rng_seed(uint64_t seed) { return (seed ^ 0x9E3779B97F4A7C15ull) | 1ull; }

float gh_rng_next_f32(uint64_t* state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return (float)((x * 0x2545F4914F6CDD1Dull) >> 40) / (float)(1ull << 24);
}

int gh_sampling_plan(const gh_sampling* p, uint32_t* k) {
    if (!p) return GH_E_INVALID;
    if (k) *k = 0;
    if (p->repeat_penalty != 1.0f) return GH_SAMPLE_FALLBACK;
    if (p->temperature <= 0.0f) return GH_SAMPLE_GREEDY;
    if (p->top_k > 0 && p->top_k <= GH_SAMPLE_MAX_DEVICE_K) {
        if (k) *k = p->top_k;
        return GH_SAMPLE_TOPK;
    }
    return GH_SAMPLE_FALLBACK;
}

int gh_sample_from_candidates(const uint32_t* idx, const float* logit, uint64_t n, const gh_sampling* p,
                              uint64_t* rng, uint32_t* token) {
    if (!p || !rng || !token || (n && (!idx || !logit))) return GH_E_INVALID;
    std::vector<Cand> cand(n);
    for (uint64_t i = 0; i < n; ++i) cand[i] = {idx[i], logit[i]};
    *token = tail(cand, p, rng);
    return GH_OK;
}

int gh_sample(float* logits, uint64_t vocab, const gh_sampling* p, const uint32_t* recent, uint64_t n_recent,
              uint64_t* rng, uint32_t* token) {
    if (!logits || !p || !rng || !token || (n_recent && !recent)) return GH_E_INVALID;
    if (p->repeat_penalty != 1.0f) {
        for (uint64_t i = 0; i < n_recent; ++i) {
            if (recent[i] >= vocab) continue;
            float& l = logits[recent[i]];
            l = l > 0.0f ? l / p->repeat_penalty : l * p->repeat_penalty;
        }
    }
    if (p->temperature <= 0.0f) {
        *token = argmax_host(logits, vocab);
        return GH_OK;
    }
    const float inv = 1.0f / p->temperature;
    std::vector<Cand> cand;
    cand.reserve(vocab);
    for (uint64_t i = 0; i < vocab; ++i)
        if (std::isfinite(logits[i])) cand.push_back({(uint32_t)i, logits[i] * inv});
    if (cand.empty()) {
        *token = argmax_host(logits, vocab);
        return GH_OK;
    }
    if (p->top_k > 0 && (size_t)p->top_k < cand.size()) {
        std::nth_element(cand.begin(), cand.begin() + (p->top_k - 1), cand.end(), cand_before);
        cand.resize(p->top_k);
    }
    std::sort(cand.begin(), cand.end(), cand_before);
    *token = tail(cand, p, rng);
    return GH_OK;
}
