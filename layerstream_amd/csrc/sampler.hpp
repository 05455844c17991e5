// Logits to a token (Sampler, src/model.rs:300-366): greedy at temperature <= 0, else top-k,
// softmax at the temperature, a nucleus (top-p) cut and a draw from a seeded xorshift64* stream.
// Host code: it reads a row of logits the host already holds.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

namespace ls {

class Sampler {
public:
    Sampler(float temperature, size_t top_k, float top_p, uint64_t seed);
    uint32_t sample(const float* logits, size_t n);
    // The next uniform draw in [0, 1) (24 bits), as sample uses it.
    float uniform();

private:
    float temperature_, top_p_;
    size_t top_k_;
    uint64_t state_;
    std::vector<uint32_t> idx_;
    std::vector<float> probs_;
};

}  // namespace ls
