// The CPU-choice decode: ocr-decode's choose on host logits and the generate loop around the one-token step
// (sampling.rs:23-89, 252-278; text.rs:524-537 TextModel::step). Host code only: the step runs on the device
// (htr_step), the choice on the calling thread, as the reference's engine does for presets the GPU choice does not
// take (sampled ones: temperature > 0, top-p on the host).
//
// Order of operations, as sampling.rs:38-89: the repetition penalty over the distinct ids of the history's last
// `window` (< 0: × rp, else ÷ rp, in f32), the frequency penalty (fp · count, in f32), then the first maximum
// (greedy), or: p_i = e^((l_i − max)/T) with (l_i − max)/T in f32 and the exponential in f64, normalised by their sum
// in index order; the descending order of p (ties by index: the order a stable sort gives); the smallest prefix whose
// running sum reaches top_p (all when top_p ≥ 1); r = next_f64 · Σ kept; the first kept token at which r minus the
// running sum is ≤ 0 (the last kept if none). The random source is SplitMix64 (sampling.rs:23-35).
#include <algorithm>
#include <cmath>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "htr_internal.h"

namespace {

double next_f64(uint64_t &state) {
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) / 9007199254740992.0;  // 2^53
}

// presets.rs:35-55 Preset::validate's ranges (the name aside)
int check_preset(const htr_preset *p) {
    const bool greedy = p->temperature == 0.0;
    if (!(p->temperature >= 0.0) || !(p->top_p > 0.0 && p->top_p <= 1.0) || (greedy && p->top_p != 1.0) ||
        !(p->repetition_penalty > 0.0) || p->repetition_window < 1 || !(p->frequency_penalty >= 0.0) ||
        p->max_new_tokens < 1)
        return htr_fail("preset: temperature %g, top_p %g, rp %g, window %zu, fp %g, max %zu (temperature ≥ 0, 0 < topP ≤ 1 "
                        "and 1 when greedy, rp > 0, window ≥ 1, fp ≥ 0, max ≥ 1)",
                        p->temperature, p->top_p, p->repetition_penalty, p->repetition_window, p->frequency_penalty,
                        p->max_new_tokens);
    return 0;
}

int32_t choose(float *logits, size_t n_vocab, const htr_preset &p, const int32_t *hist, size_t n_hist,
               const std::unordered_map<int32_t, uint32_t> &counts, uint64_t &rng, std::vector<std::pair<double, int32_t>> &probs) {
    if (p.repetition_penalty != 1.0) {
        const float rp = (float)p.repetition_penalty;
        std::unordered_set<int32_t> seen;
        for (size_t j = n_hist - std::min(p.repetition_window, n_hist); j < n_hist; j++)
            if (seen.insert(hist[j]).second) {
                float &l = logits[hist[j]];
                l = l < 0.0f ? l * rp : l / rp;
            }
    }
    if (p.frequency_penalty > 0.0)
        for (const auto &tc : counts) logits[tc.first] -= (float)p.frequency_penalty * (float)tc.second;
    if (p.temperature == 0.0) {
        size_t best = 0;
        for (size_t i = 0; i < n_vocab; i++)
            if (logits[i] > logits[best]) best = i;
        return (int32_t)best;
    }
    const float t = (float)p.temperature;
    float mx = -INFINITY;
    for (size_t i = 0; i < n_vocab; i++) mx = std::max(mx, logits[i]);
    probs.resize(n_vocab);
    double sum = 0.0;
    for (size_t i = 0; i < n_vocab; i++) {
        const double e = std::exp((double)((logits[i] - mx) / t));
        probs[i] = {e, (int32_t)i};
        sum += e;
    }
    for (auto &pr : probs) pr.first /= sum;
    std::stable_sort(probs.begin(), probs.end(), [](const auto &a, const auto &b) { return a.first > b.first; });
    size_t keep = probs.size();
    if (p.top_p < 1.0) {
        double acc = 0.0;
        for (size_t k = 0; k < probs.size(); k++) {
            acc += probs[k].first;
            if (acc >= p.top_p) {
                keep = k + 1;
                break;
            }
        }
    }
    double total = 0.0;
    for (size_t k = 0; k < keep; k++) total += probs[k].first;
    double r = next_f64(rng) * total;
    for (size_t k = 0; k < keep; k++) {
        r -= probs[k].first;
        if (r <= 0.0) return probs[k].second;
    }
    return probs[keep - 1].second;
}

}  // namespace

extern "C" int htr_choose_host(float *logits, size_t n_vocab, const htr_preset *p, const int32_t *history,
                               size_t n_history, const int32_t *count_ids, const uint32_t *counts, size_t n_counts,
                               uint64_t *rng, int32_t *out) {
    if (!logits || !p || !rng || !out || (n_history && !history) || (n_counts && (!count_ids || !counts)))
        return htr_fail("htr_choose_host: null argument");
    if (n_vocab == 0 || n_vocab > (size_t)INT32_MAX) return htr_fail("htr_choose_host: %zu logits", n_vocab);
    HTR_TRY(check_preset(p));
    std::unordered_map<int32_t, uint32_t> cnt;
    for (size_t i = 0; i < n_history; i++)
        if (history[i] < 0 || (size_t)history[i] >= n_vocab) return htr_fail("history token %d is outside the vocabulary", history[i]);
    for (size_t i = 0; i < n_counts; i++) {
        if (count_ids[i] < 0 || (size_t)count_ids[i] >= n_vocab) return htr_fail("counted token %d is outside the vocabulary", count_ids[i]);
        if (!cnt.emplace(count_ids[i], counts[i]).second) return htr_fail("token %d is counted twice", count_ids[i]);
    }
    std::vector<std::pair<double, int32_t>> probs;
    *out = choose(logits, n_vocab, *p, history, n_history, cnt, *rng, probs);
    return 0;
}

// sampling.rs:252-278 generate with TextModel::step as the Step (text.rs:524-537)
extern "C" int htr_generate(htr_session *s, const htr_preset *p, uint64_t seed, const int32_t *history,
                            size_t n_history, htr_token_cb on_token, void *user, size_t *n_out) {
    if (!s || !p || (n_history && !history)) return htr_fail("htr_generate: null argument");
    HTR_TRY(check_preset(p));
    const size_t nv = (size_t)session_n_vocab(s);
    std::vector<int32_t> hist(history, history + n_history);
    for (int32_t t : hist)
        if (t < 0 || (size_t)t >= nv) return htr_fail("history token %d is outside the vocabulary", t);
    std::unordered_map<int32_t, uint32_t> counts;
    uint64_t rng = seed;
    std::vector<float> logits(nv);
    std::vector<std::pair<double, int32_t>> probs;
    size_t out = 0;
    if (n_out) *n_out = 0;
    HTR_TRY(htr_session_logits(s, logits.data()));
    while (out < p->max_new_tokens) {
        const int32_t tok = choose(logits.data(), nv, *p, hist.data(), hist.size(), counts, rng, probs);
        out++;
        if (n_out) *n_out = out;
        if (on_token && !on_token(tok, user)) break;
        hist.push_back(tok);
        counts[tok]++;
        HTR_TRY(htr_step(s, tok, logits.data()));
    }
    return 0;
}
