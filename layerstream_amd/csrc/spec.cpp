// Greedy speculative decoding (src/spec.rs:57-152) over the device Model, with pluggable
// drafters: a draft Model on the device (the reference's setup) or a scripted proposer.
#include <chrono>

#include "model.hpp"
#include "spec.hpp"

namespace ls {

static double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

static bool contains(const uint32_t* v, size_t n, uint32_t x) {
    for (size_t i = 0; i < n; i++)
        if (v[i] == x) return true;
    return false;
}

// ---- draft model ----------------------------------------------------------------------
static int md_prefill(void* ctx, const uint32_t* p, size_t n) {
    auto* m = static_cast<Model*>(ctx);
    uint32_t a;
    m->forward(p, n, nullptr, &a);
    return 1;
}

// kk single-token passes, each fed the argmax of the one before (src/spec.rs:100-107). Over
// resident weights they run as one chain on the device (one host wait for all kk tokens).
static int md_propose(void* ctx, uint32_t last, size_t kk, uint32_t* out) {
    auto* m = static_cast<Model*>(ctx);
    if (m->chains_on_device()) {
        m->draft_chain(last, kk, out);
        return int(kk);
    }
    uint32_t cur = last;
    for (size_t i = 0; i < kk; i++) {
        m->forward(&cur, 1, nullptr, &out[i]);
        cur = out[i];
    }
    return int(kk);
}

// Both models must end up having consumed [a, d_1 .. d_m] (src/spec.rs:137-147).
static int md_commit(void* ctx, const uint32_t* block, size_t p, size_t m) {
    auto* d = static_cast<Model*>(ctx);
    const size_t want = p + m + 1;
    if (d->pos() > want) {
        d->truncate(want);
        return 0;
    }
    if (d->pos() < want) {
        const size_t from = d->pos() - p;
        uint32_t a;
        d->forward(block + from, m + 1 - from, nullptr, &a);
        return 1;
    }
    return 0;
}

ls_drafter model_drafter(Model* m) {
    ls_drafter d{};
    d.ctx = m;
    d.prefill = md_prefill;
    d.propose = md_propose;
    d.commit = md_commit;
    return d;
}

bool is_model_drafter(const ls_drafter& d) { return d.propose == md_propose; }

// ---- scripted proposer ----------------------------------------------------------------
static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint32_t Scripted::token(size_t idx) const {
    const uint64_t h1 = mix64(seed ^ mix64(uint64_t(idx))), h2 = mix64(h1);
    const double u = double(h1 >> 11) * (1.0 / 9007199254740992.0);
    if (idx < greedy.size()) {
        const uint32_t g = greedy[idx];
        if (u < p_accept) return g;
        const uint64_t r = h2 % (vocab - 1);
        return uint32_t(r >= g ? r + 1 : r);
    }
    return uint32_t(h2 % vocab);
}

static int sc_prefill(void* ctx, const uint32_t*, size_t) {
    static_cast<Scripted*>(ctx)->len = 1;
    return 0;
}
static int sc_propose(void* ctx, uint32_t, size_t kk, uint32_t* out) {
    auto* s = static_cast<Scripted*>(ctx);
    for (size_t i = 0; i < kk; i++) out[i] = s->token(s->len + i);
    return 0;
}
static int sc_commit(void* ctx, const uint32_t*, size_t, size_t m) {
    static_cast<Scripted*>(ctx)->len += m + 1;
    return 0;
}

ls_drafter scripted_drafter(Scripted* s) {
    ls_drafter d{};
    d.ctx = s;
    d.prefill = sc_prefill;
    d.propose = sc_propose;
    d.commit = sc_commit;
    return d;
}

bool is_scripted_drafter(const ls_drafter& d) { return d.propose == sc_propose; }

// ---- the loop -------------------------------------------------------------------------
constexpr size_t MAX_DRAFT = 32;  // src/spec.rs:52

static void check_cb(int rc, const char* what) {
    if (rc < 0) fail(std::string("drafter ") + what + " failed");
}

SpecRun::SpecRun(Model& target, ls_drafter& d, const uint32_t* prompt, size_t n_prompt, size_t max_new, size_t k,
                 const uint32_t* eos, size_t n_eos)
    : target_(target), d_(d), max_new_(max_new), k_(k), eos_(eos, eos + n_eos) {
    if (k == 0 || k > MAX_DRAFT) fail("k must be between 1 and 32, not " + std::to_string(k));
    if (n_prompt == 0 || max_new == 0 || !prompt) fail("need a prompt and at least one token to generate");
    Model* dm = is_model_drafter(d) ? static_cast<Model*>(d.ctx) : nullptr;
    if (target.pos() != 0 || (dm && dm->pos() != 0)) fail("both models must start with an empty cache");
    if (dm && dm->cfg().vocab != target.cfg().vocab) fail("the draft and the target must share a vocabulary");
    const size_t need = n_prompt + max_new + k;
    if (need > target.max_ctx() || (dm && need > dm->max_ctx()))
        fail("prompt + max_new + k = " + std::to_string(need) + " tokens exceed the context limit");
    if (!d.prefill || !d.propose || !d.commit) fail("incomplete drafter");

    const double t0 = now_s();
    target.forward(prompt, n_prompt, nullptr, &a_);
    check_cb(d.prefill(d.ctx, prompt, n_prompt), "prefill");
    st_.first_secs = now_s() - t0;
    out_.reserve(max_new);
    out_.push_back(a_);
    stop_ = contains(eos_.data(), eos_.size(), a_);
    t_dec_ = now_s();
}

void SpecRun::step() {
    if (done()) return;
    const size_t kk = std::min(k_, max_new_ - out_.size() - 1);  // a pass yields at most kk + 1 tokens
    uint32_t block[MAX_DRAFT + 1];
    double ts = now_s();
    block[0] = a_;
    int f = d_.propose(d_.ctx, a_, kk, block + 1);
    check_cb(f, "propose");
    st_.draft_forwards += uint64_t(f);
    st_.draft_secs += now_s() - ts;

    const size_t p = target_.pos();
    ts = now_s();
    uint32_t m, next;
    target_.verify_greedy(block, kk + 1, &m, &next);  // one weight pass checks every guess
    st_.target_secs += now_s() - ts;
    st_.target_passes++;
    st_.drafted += kk;
    st_.accepted += m;
    step_ms_.push_back(target_.last_step_ms());
    step_m_.push_back(m);
    for (size_t i = 0; i <= m; i++) {
        const uint32_t tok = i < m ? block[i + 1] : next;
        out_.push_back(tok);
        if (contains(eos_.data(), eos_.size(), tok) || out_.size() == max_new_) {
            stop_ = true;
            break;
        }
    }
    ts = now_s();
    f = d_.commit(d_.ctx, block, p, m);
    check_cb(f, "commit");
    st_.draft_forwards += uint64_t(f);
    st_.draft_secs += now_s() - ts;
    a_ = next;
    st_.decode_secs = now_s() - t_dec_;
}

std::vector<uint32_t> speculative_greedy(Model& target, ls_drafter& d, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                                         size_t k, const uint32_t* eos, size_t n_eos, ls_spec_stats& st) {
    SpecRun run(target, d, prompt, n_prompt, max_new, k, eos, n_eos);
    while (!run.done()) run.step();
    st = run.stats();
    return run.tokens();
}

std::vector<uint32_t> greedy_generate(Model& m, const uint32_t* prompt, size_t n_prompt, size_t max_new, const uint32_t* eos,
                                      size_t n_eos) {
    std::vector<uint32_t> out;
    uint32_t t;
    m.forward(prompt, n_prompt, nullptr, &t);
    for (size_t i = 0; i < max_new; i++) {
        out.push_back(t);
        if (contains(eos, n_eos, t) || i + 1 == max_new) break;
        m.forward(&t, 1, nullptr, &t);
    }
    return out;
}

}  // namespace ls
