// Sampler (src/model.rs:300-366). The arithmetic is f32 in the reference's order (differences,
// divisions by the temperature, expf, sums left to right), so a given seed draws the same tokens.
#include "sampler.hpp"

#include <algorithm>
#include <cmath>

namespace ls {

Sampler::Sampler(float temperature, size_t top_k, float top_p, uint64_t seed)
    : temperature_(temperature), top_p_(top_p), top_k_(top_k < 1 ? 1 : top_k), state_((seed * 0x9E3779B97F4A7C15ull) | 1) {}

float Sampler::uniform() {
    // xorshift64*, the top 24 bits of the product
    state_ ^= state_ >> 12;
    state_ ^= state_ << 25;
    state_ ^= state_ >> 27;
    const uint64_t r = state_ * 0x2545F4914F6CDD1Dull;
    return float(uint32_t(r >> 40)) / float(1u << 24);
}

uint32_t Sampler::sample(const float* logits, size_t n) {
    if (n == 0) return 0;
    if (temperature_ <= 0.0f) {
        size_t best = 0;  // the first maximum
        for (size_t i = 1; i < n; i++)
            if (logits[i] > logits[best]) best = i;
        return uint32_t(best);
    }
    // The k largest, largest first (equal logits: lower index first).
    const size_t k = std::min(top_k_, n);
    idx_.resize(n);
    for (size_t i = 0; i < n; i++) idx_[i] = uint32_t(i);
    std::partial_sort(idx_.begin(), idx_.begin() + k, idx_.end(),
                      [&](uint32_t a, uint32_t b) { return logits[a] > logits[b] || (logits[a] == logits[b] && a < b); });
    const float top = logits[idx_[0]];
    probs_.resize(k);
    float sum = 0.0f;
    for (size_t i = 0; i < k; i++) {
        probs_[i] = std::exp((logits[idx_[i]] - top) / temperature_);
        sum += probs_[i];
    }
    for (size_t i = 0; i < k; i++) probs_[i] /= sum;
    // The smallest prefix whose probability reaches top_p.
    size_t keep = k;
    float cum = 0.0f;
    for (size_t i = 0; i < k; i++) {
        cum += probs_[i];
        if (cum >= top_p_) {
            keep = i + 1;
            break;
        }
    }
    float total = 0.0f;
    for (size_t i = 0; i < keep; i++) total += probs_[i];
    float r = uniform() * total;
    for (size_t i = 0; i < keep; i++) {
        r -= probs_[i];
        if (r <= 0.0f) return idx_[i];
    }
    return idx_[keep - 1];
}

}  // namespace ls
