// Speculative decoding loop and drafters.
#pragma once

#include <vector>

#include "common.hpp"

namespace ls {

class Model;

// Scripted proposer: for output index i, greedy[i] with probability p_accept (SplitMix64
// counter stream keyed by seed and i), else a uniformly random different token.
struct Scripted {
    std::vector<uint32_t> greedy;
    double p_accept = 0;
    uint64_t seed = 0, vocab = 0;
    size_t len = 0;  // tokens emitted so far
    uint32_t token(size_t idx) const;
};

ls_drafter model_drafter(Model* m);
ls_drafter scripted_drafter(Scripted* s);
bool is_model_drafter(const ls_drafter& d);
bool is_scripted_drafter(const ls_drafter& d);

std::vector<uint32_t> speculative_greedy(Model& target, ls_drafter& d, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                                         size_t k, const uint32_t* eos, size_t n_eos, ls_spec_stats& st);
std::vector<uint32_t> greedy_generate(Model& m, const uint32_t* prompt, size_t n_prompt, size_t max_new, const uint32_t* eos,
                                      size_t n_eos);

}  // namespace ls
