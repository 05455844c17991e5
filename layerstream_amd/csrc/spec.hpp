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

// speculative_greedy (src/spec.rs:57-152) in resumable form.
class SpecRun {
public:
    SpecRun(Model& target, ls_drafter& d, const uint32_t* prompt, size_t n_prompt, size_t max_new, size_t k,
            const uint32_t* eos, size_t n_eos);
    bool done() const { return stop_ || out_.size() >= max_new_; }
    void step();  // one verify pass
    const std::vector<uint32_t>& tokens() const { return out_; }
    const ls_spec_stats& stats() const { return st_; }
    const std::vector<double>& step_ms() const { return step_ms_; }
    const std::vector<uint32_t>& step_m() const { return step_m_; }

private:
    Model& target_;
    ls_drafter d_;
    size_t max_new_, k_;
    std::vector<uint32_t> eos_, out_;
    uint32_t a_ = 0;
    bool stop_ = false;
    double t_dec_ = 0;
    ls_spec_stats st_{};
    std::vector<double> step_ms_;
    std::vector<uint32_t> step_m_;
};

std::vector<uint32_t> speculative_greedy(Model& target, ls_drafter& d, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                                         size_t k, const uint32_t* eos, size_t n_eos, ls_spec_stats& st);
std::vector<uint32_t> greedy_generate(Model& m, const uint32_t* prompt, size_t n_prompt, size_t max_new, const uint32_t* eos,
                                      size_t n_eos);

}  // namespace ls
