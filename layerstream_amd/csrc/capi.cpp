// The extern "C" boundary (include/layerstream.h). Every entry point catches C++ errors and
// turns them into a negative code plus a thread-local message, as the reference turns bad
// requests into Err(String) instead of panics.
#include <memory>
#include <new>

#include <cstring>

#include "model.hpp"
#include "sampler.hpp"
#include "spec.hpp"
#include "static_mm.hpp"
#include "tokenizer.hpp"

struct ls_source {
    std::unique_ptr<ls::Source> s;
};

struct ls_model {
    std::unique_ptr<ls::Model> m;
};

struct ls_spec {
    std::unique_ptr<ls::SpecRun> r;
};

struct ls_tokenizer {
    std::unique_ptr<ls::Tokenizer> t;
};

struct ls_stream_decoder {
    ls::StreamDecoder d;
};

struct ls_sampler {
    std::unique_ptr<ls::Sampler> s;
};

namespace {

template <class F>
int guard(F&& f) {
    try {
        f();
        ls::set_last_error("");
        return LS_OK;
    } catch (const ls::Error& e) {
        ls::set_last_error(e.what());
        return e.code;
    } catch (const std::bad_alloc&) {
        ls::set_last_error("out of host memory");
        return LS_E_INVALID;
    } catch (const std::exception& e) {
        ls::set_last_error(e.what());
        return std::string(e.what()).rfind("HIP", 0) == 0 ? LS_E_DEVICE : LS_E_INVALID;
    }
}

void need(const void* p, const char* what) {
    if (!p) ls::fail(std::string("null ") + what);
}

// A variable-length result: its size always, the data when it fits.
template <class T>
void give(const std::vector<T>& v, T* out, size_t cap, size_t* n) {
    need(n, "size output");
    *n = v.size();
    if (out && cap >= v.size() && !v.empty()) std::memcpy(out, v.data(), v.size() * sizeof(T));
}
void give(const std::string& v, char* out, size_t cap, size_t* n) {
    need(n, "size output");
    *n = v.size();
    if (out && cap >= v.size() && !v.empty()) std::memcpy(out, v.data(), v.size());
}

}  // namespace

extern "C" {

const char* ls_last_error(void) { return ls::last_error().c_str(); }
const char* ls_version(void) { return "layerstream_amd 0.1 (gfx950)"; }

size_t ls_row_bytes(ls_format f, size_t cols) { return ls::Format::from(f).row_bytes(cols); }

int ls_format_validate(ls_format f, const size_t* cols, size_t n) {
    return guard([&] { ls::Format::from(f).validate(std::vector<size_t>(cols, cols + n)); });
}

int ls_config_from_json(const char* text, ls_config* out) {
    return guard([&] {
        need(text, "config text");
        need(out, "output");
        *out = ls::Config::from_json(text).c();
    });
}

size_t ls_layer_layout(const ls_config* cfg, size_t ranges[24]) {
    size_t total = 0;
    int rc = guard([&] {
        need(cfg, "config");
        ls::LayerLayout L = ls::Config::from(*cfg).layout();
        for (int s = 0; s < ls::N_TENSORS; s++) {
            ranges[2 * s] = L.off[s];
            ranges[2 * s + 1] = L.len[s];
        }
        total = L.total;
    });
    return rc == LS_OK ? total : 0;
}

int ls_inject_quant(const char* text, int bits, int group, int eb, int eg, char* out, size_t cap, size_t* out_len) {
    return guard([&] {
        need(text, "config text");
        std::string s = ls::inject_quant(text, bits, group, eb, eg);
        if (out_len) *out_len = s.size();
        if (out) {
            if (cap < s.size() + 1) ls::fail("output buffer too small");
            std::memcpy(out, s.c_str(), s.size() + 1);
        }
    });
}

int ls_quantize_row(ls_format f, const float* row, size_t cols, int clip, uint8_t* out, double* err, double* norm) {
    return guard([&] {
        need(row, "row");
        need(out, "output");
        ls::quantize_row(ls::Format::from(f), row, cols, clip != 0, out, err, norm);
    });
}

int ls_quantize_model(const char* text, const uint8_t* layers, const uint8_t* embed, const uint8_t* norm, ls_format fmt,
                      ls_format efmt, int clip, int threads, uint8_t* out, size_t cap, size_t* out_len, double* rel) {
    return guard([&] {
        need(text, "config text");
        need(out_len, "out_len");
        ls::Config c = ls::Config::from_json(text);
        if (!out) {
            // Size only: header text + parts.
            ls::Format f = ls::Format::from(fmt), e = ls::Format::from(efmt);
            if (f.is_bf16() || e.is_bf16()) ls::fail("quantize needs a quantized target format");
            bool same = f == e;
            std::string q = ls::inject_quant(text, f.bits, f.group, same ? 0 : e.bits, same ? 0 : e.group);
            ls::Config qc = ls::Config::from_json(q);
            ls::QuantHeader h;
            h.config_text = q;
            h.layer_bytes = qc.layout().total;
            h.embed_bytes = qc.vocab * qc.row_bytes();
            h.norm_bytes = qc.hidden * 2;
            *out_len = h.to_bytes().size() + qc.layers * h.layer_bytes + h.embed_bytes + h.norm_bytes;
            return;
        }
        need(layers, "layers");
        need(embed, "embedding");
        need(norm, "final norm");
        (void)c;
        std::vector<uint8_t> img = ls::quantize_model(text, layers, embed, norm, ls::Format::from(fmt), ls::Format::from(efmt),
                                                      clip != 0, threads, rel);
        *out_len = img.size();
        if (cap < img.size()) ls::fail("output buffer too small");
        std::memcpy(out, img.data(), img.size());
    });
}

int ls_synth_bf16_model(const ls_config* cfg, uint64_t seed, float std_dev, uint8_t* layers, uint8_t* embed, uint8_t* norm,
                        int threads) {
    return guard([&] {
        need(cfg, "config");
        need(layers, "layers");
        need(embed, "embedding");
        need(norm, "final norm");
        ls::synth_bf16_model(ls::Config::from(*cfg), seed, std_dev, layers, embed, norm, threads);
    });
}

int ls_source_from_memory(const char* text, const uint8_t* layers, size_t ll, const uint8_t* embed, size_t el,
                          const uint8_t* norm, size_t nl, ls_source** out) {
    return guard([&] {
        need(text, "config text");
        need(out, "output");
        auto s = std::make_unique<ls_source>();
        s->s = std::make_unique<ls::MemorySource>(text, layers, ll, embed, el, norm, nl);
        *out = s.release();
    });
}

int ls_source_open_lsq(const char* path, ls_source** out) {
    return guard([&] {
        need(path, "path");
        need(out, "output");
        auto s = std::make_unique<ls_source>();
        s->s = std::make_unique<ls::LsqFileSource>(path);
        *out = s.release();
    });
}

int ls_source_from_lsq_image(const uint8_t* image, size_t len, ls_source** out) {
    return guard([&] {
        need(out, "output");
        auto s = std::make_unique<ls_source>();
        s->s = std::make_unique<ls::LsqImageSource>(image, len);
        *out = s.release();
    });
}

int ls_source_pinned_copy(const ls_source* src, ls_source** out) {
    return guard([&] {
        need(src, "source");
        need(out, "output");
        auto s = std::make_unique<ls_source>();
        s->s = std::make_unique<ls::PinnedSource>(*src->s);
        *out = s.release();
    });
}

void ls_source_free(ls_source* s) { delete s; }

int ls_source_config(const ls_source* s, ls_config* out) {
    return guard([&] {
        need(s, "source");
        need(out, "output");
        *out = s->s->cfg().c();
    });
}

uint64_t ls_source_bytes_read(const ls_source* s) { return s ? s->s->bytes_read() : 0; }

int ls_model_create(ls_source* src, int mode, int slots, size_t max_ctx, int device, ls_model** out) {
    return guard([&] {
        need(src, "source");
        need(out, "output");
        auto m = std::make_unique<ls_model>();
        m->m = std::make_unique<ls::Model>(*src->s, mode, slots, max_ctx, device);
        *out = m.release();
    });
}

void ls_model_free(ls_model* m) {
    try {
        delete m;
    } catch (...) {
    }
}

int ls_model_create_batch(ls_source* src, int mode, int slots, size_t max_ctx, int device, int n_seq, ls_model** out) {
    return guard([&] {
        need(src, "source");
        need(out, "output");
        auto m = std::make_unique<ls_model>();
        m->m = std::make_unique<ls::Model>(*src->s, mode, slots, max_ctx, device, n_seq);
        *out = m.release();
    });
}

int ls_model_select(ls_model* m, int seq) {
    return guard([&] {
        need(m, "model");
        m->m->select(seq);
    });
}

int ls_model_n_seq(const ls_model* m) { return m ? m->m->n_seq() : 0; }

int ls_model_verify_greedy_batch(ls_model* m, const uint32_t* blocks, const size_t* lens, int n_seq, uint32_t* accepted,
                                 uint32_t* next) {
    return guard([&] {
        need(m, "model");
        need(blocks, "blocks");
        need(lens, "lens");
        need(accepted, "accepted");
        need(next, "next");
        if (n_seq != m->m->n_seq())
            ls::fail("the model holds " + std::to_string(m->m->n_seq()) + " sequences, not " + std::to_string(n_seq));
        m->m->verify_greedy_batch(blocks, lens, accepted, next);
    });
}

size_t ls_model_pos(const ls_model* m) { return m ? m->m->pos() : 0; }
size_t ls_model_max_ctx(const ls_model* m) { return m ? m->m->max_ctx() : 0; }
void ls_model_reset(ls_model* m) {
    if (m) m->m->reset();
}

int ls_model_truncate(ls_model* m, size_t pos) {
    return guard([&] {
        need(m, "model");
        m->m->truncate(pos);
    });
}

int ls_model_forward(ls_model* m, const uint32_t* tok, size_t n, float* logits, uint32_t* argmax) {
    return guard([&] {
        need(m, "model");
        m->m->forward(tok, n, logits, argmax);
    });
}

int ls_model_forward_multi(ls_model* m, const uint32_t* tok, size_t n, size_t n_logits, float* logits, uint32_t* argmax) {
    return guard([&] {
        need(m, "model");
        m->m->forward_multi(tok, n, n_logits, logits, argmax);
    });
}

int ls_model_verify_greedy(ls_model* m, const uint32_t* block, size_t n, uint32_t* accepted, uint32_t* next) {
    return guard([&] {
        need(m, "model");
        need(accepted, "accepted");
        need(next, "next");
        m->m->verify_greedy(block, n, accepted, next);
    });
}

int ls_model_draft_chain(ls_model* m, uint32_t first, size_t k, uint32_t* out) {
    return guard([&] {
        need(m, "model");
        need(out, "output");
        if (k < 1 || k > 32) ls::fail("a draft chain takes 1 to 32 passes, not " + std::to_string(k));
        m->m->draft_chain(first, k, out);
    });
}

int ls_model_report(const ls_model* m, ls_report* out) {
    return guard([&] {
        need(m, "model");
        need(out, "output");
        *out = m->m->report();
    });
}

double ls_model_last_step_ms(const ls_model* m) { return m ? m->m->last_step_ms() : 0.0; }

int ls_drafter_from_model(ls_model* draft, ls_drafter* out) {
    return guard([&] {
        need(draft, "model");
        need(out, "output");
        *out = ls::model_drafter(draft->m.get());
    });
}

int ls_drafter_scripted(const uint32_t* greedy, size_t n, double p, uint64_t seed, uint64_t vocab, ls_drafter* out) {
    return guard([&] {
        need(out, "output");
        if (vocab < 2) ls::fail("vocab must hold at least two tokens");
        if (n && !greedy) ls::fail("null greedy sequence");
        auto* s = new ls::Scripted;
        s->greedy.assign(greedy, greedy + n);
        s->p_accept = p;
        s->seed = seed;
        s->vocab = vocab;
        *out = ls::scripted_drafter(s);
    });
}

uint32_t ls_drafter_scripted_token(const ls_drafter* d, size_t i) {
    if (!d || !ls::is_scripted_drafter(*d)) return 0;
    return static_cast<const ls::Scripted*>(d->ctx)->token(i);
}

void ls_drafter_free(ls_drafter* d) {
    if (d && ls::is_scripted_drafter(*d)) {
        delete static_cast<ls::Scripted*>(d->ctx);
        d->ctx = nullptr;
    }
}

int ls_speculative_greedy(ls_model* target, ls_drafter* d, const uint32_t* prompt, size_t n_prompt, size_t max_new, size_t k,
                          const uint32_t* eos, size_t n_eos, uint32_t* out, size_t* out_len, ls_spec_stats* stats) {
    return guard([&] {
        need(target, "target");
        need(d, "drafter");
        need(out, "output");
        need(out_len, "out_len");
        ls_spec_stats st{};
        *out_len = 0;
        std::vector<uint32_t> toks = ls::speculative_greedy(*target->m, *d, prompt, n_prompt, max_new, k, eos, n_eos, st);
        std::memcpy(out, toks.data(), toks.size() * 4);
        *out_len = toks.size();
        if (stats) *stats = st;
    });
}

int ls_spec_begin(ls_model* target, ls_drafter* d, const uint32_t* prompt, size_t n_prompt, size_t max_new, size_t k,
                  const uint32_t* eos, size_t n_eos, ls_spec** out) {
    return guard([&] {
        need(target, "target");
        need(d, "drafter");
        need(out, "output");
        auto s = std::make_unique<ls_spec>();
        s->r = std::make_unique<ls::SpecRun>(*target->m, *d, prompt, n_prompt, max_new, k, eos, n_eos);
        *out = s.release();
    });
}

int ls_spec_step(ls_spec* s, size_t max_steps, int* done) {
    return guard([&] {
        need(s, "run");
        for (size_t i = 0; (max_steps == 0 || i < max_steps) && !s->r->done(); i++) s->r->step();
        if (done) *done = s->r->done() ? 1 : 0;
    });
}

int ls_spec_result(const ls_spec* s, uint32_t* out, size_t cap, size_t* out_len, ls_spec_stats* stats) {
    return guard([&] {
        need(s, "run");
        const auto& t = s->r->tokens();
        if (out_len) *out_len = t.size();
        if (out) std::memcpy(out, t.data(), std::min(cap, t.size()) * 4);
        if (stats) *stats = s->r->stats();
    });
}

size_t ls_spec_step_log(const ls_spec* s, double* ms, uint32_t* accepted, size_t cap) {
    if (!s) return 0;
    const auto& a = s->r->step_ms();
    const auto& b = s->r->step_m();
    for (size_t i = 0; i < std::min(cap, a.size()); i++) {
        if (ms) ms[i] = a[i];
        if (accepted) accepted[i] = b[i];
    }
    return a.size();
}

void ls_spec_free(ls_spec* s) { delete s; }

int ls_model_profile(ls_model* m, int enable) {
    return guard([&] {
        need(m, "model");
        m->m->set_profiling(enable == 2 ? 2 : (enable != 0 ? 1 : 0));
    });
}

int ls_model_use_graphs(ls_model* m, int enable) {
    return guard([&] {
        need(m, "model");
        m->m->set_graphs(enable != 0);
    });
}

int ls_model_debug_fail_next(ls_model* m) {
    return guard([&] {
        need(m, "model");
        m->m->debug_fail_next();
    });
}

size_t ls_model_debug_timeline(ls_model* m, uint64_t* out, size_t cap) {
    size_t n = 0;
    guard([&] {
        need(m, "model");
        n = m->m->debug_timeline(out, cap);
    });
    return n;
}

size_t ls_model_debug_read(ls_model* m, const char* name, void* out, size_t cap) {
    size_t n = 0;
    guard([&] {
        need(m, "model");
        n = m->m->debug_read(name, out, cap);
    });
    return n;
}

int ls_model_profile_read(ls_model* m, ls_kernel_stat* out) {
    return guard([&] {
        need(m, "model");
        need(out, "output");
        *out = m->m->read_profile();
    });
}

int ls_greedy_generate(ls_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new, const uint32_t* eos, size_t n_eos,
                       uint32_t* out, size_t* out_len) {
    return guard([&] {
        need(m, "model");
        need(out, "output");
        need(out_len, "out_len");
        *out_len = 0;
        if (max_new == 0) return;
        std::vector<uint32_t> toks = ls::greedy_generate(*m->m, prompt, n_prompt, max_new, eos, n_eos);
        std::memcpy(out, toks.data(), toks.size() * 4);
        *out_len = toks.size();
    });
}

int ls_matmul(ls_format f, const void* w_dev, size_t rows, size_t cols, const float* x_dev, size_t t, float* y_dev, void* stream) {
    return guard([&] {
        need(w_dev, "weights");
        need(x_dev, "input");
        need(y_dev, "output");
        ls::Format F = ls::Format::from(f);
        F.validate({cols});
        if (t == 0 || t > 128) ls::fail("t must be between 1 and 128");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const ls::TMat shape = ls::tile_shape(F.bits, F.group, int(rows), int(cols));
        ls::DevBuf data(ls::tile_data_bytes(shape));
        ls::DevBuf scales(std::max<size_t>(16, ls::tile_scale_bytes(shape)));
        const ls::TMat W = ls::tile_bind(shape, data.as<uint8_t>(), scales.as<uint16_t>());
        ls::tile_clear(W, s);
        ls::tile_repack(static_cast<const uint8_t*>(w_dev), int(rows), W, 0, int(rows), int(rows), s);
        HIPC(hipMemsetAsync(y_dev, 0, t * rows * 4, s));
        // y = W x through the residual kernel (y starts at zero), inputs as fragments.
        const size_t tiles = (t + ls::FTOK - 1) / ls::FTOK;
        ls::DevBuf frags(ls::frag_tile_bytes(int(cols)) * tiles);
        HIPC(hipMemsetAsync(frags.p, 0, frags.n, s));
        ls::x_frags(x_dev, int(t), int(cols), nullptr, frags.as<uint8_t>(), nullptr, s);
        const ls::MMPlan plan = ls::mm_plan(W, 1, 8, int(t), 1);
        ls::DevBuf part(std::max<size_t>(1, ls::mm_part_floats(plan)) * 4);
        ls::DevBuf cnt(std::max<size_t>(1, ls::mm_counters(plan)) * 4);
        HIPC(hipMemsetAsync(cnt.p, 0, cnt.n, s));
        ls::MMArgs a;
        a.W = W;
        a.frags = frags.as<uint8_t>();
        a.frag_stride = ls::frag_tile_bytes(int(cols));
        a.n = int(t);
        a.out = y_dev;
        a.ldo = int(rows);
        ls::mm_residual(a, plan, ls::MMScratch{part.as<float>(), cnt.as<int>()}, s);
        HIPC(hipStreamSynchronize(s));
    });
}

int ls_tokenizer_load(const char* dir, ls_tokenizer** out) {
    return guard([&] {
        need(dir, "directory");
        need(out, "output");
        auto t = std::make_unique<ls_tokenizer>();
        t->t = std::make_unique<ls::Tokenizer>(dir);
        *out = t.release();
    });
}

void ls_tokenizer_free(ls_tokenizer* t) { delete t; }

size_t ls_tokenizer_vocab_size(const ls_tokenizer* t) { return t ? t->t->vocab_size() : 0; }

int ls_tokenizer_encode(const ls_tokenizer* t, const char* text, size_t len, uint32_t* out, size_t cap, size_t* n) {
    return guard([&] {
        need(t, "tokenizer");
        if (len) need(text, "text");
        give(t->t->encode(std::string(text ? text : "", len)), out, cap, n);
    });
}

int ls_tokenizer_decode(const ls_tokenizer* t, const uint32_t* ids, size_t n, char* out, size_t cap, size_t* len) {
    return guard([&] {
        need(t, "tokenizer");
        if (n) need(ids, "ids");
        give(t->t->decode(ids, n), out, cap, len);
    });
}

int ls_tokenizer_token_bytes(const ls_tokenizer* t, uint32_t id, int show_special, char* out, size_t cap, size_t* len) {
    return guard([&] {
        need(t, "tokenizer");
        give(t->t->token_bytes(id, show_special != 0), out, cap, len);
    });
}

int ls_tokenizer_token_id(const ls_tokenizer* t, const char* token, uint32_t* id) {
    if (!t || !token || !id) return 0;
    return t->t->token_id(token, id) ? 1 : 0;
}

int ls_tokenizer_is_special(const ls_tokenizer* t, uint32_t id) { return t && t->t->is_special(id) ? 1 : 0; }

int ls_tokenizer_pretokens(const char* text, size_t len, uint32_t* ends, size_t cap, size_t* n) {
    return guard([&] {
        if (len) need(text, "text");
        const std::vector<uint32_t> cps = ls::utf8_to_cps(std::string(text ? text : "", len));
        std::vector<uint32_t> e;
        for (size_t i = 0; i < cps.size();) {
            i = ls::Tokenizer::pretoken_end(cps, i);
            e.push_back(uint32_t(i));
        }
        give(e, ends, cap, n);
    });
}

int ls_stream_decoder_new(ls_stream_decoder** out) {
    return guard([&] {
        need(out, "output");
        *out = new ls_stream_decoder();
    });
}

void ls_stream_decoder_free(ls_stream_decoder* d) { delete d; }

int ls_stream_decoder_push(ls_stream_decoder* d, const char* bytes, size_t n, char* out, size_t cap, size_t* len) {
    return guard([&] {
        need(d, "decoder");
        need(out, "output");
        if (n) need(bytes, "bytes");
        if (cap < 3 * (n + 4)) ls::fail("the output buffer must hold 3 * (n + 4) bytes");
        give(d->d.push(std::string(bytes ? bytes : "", n)), out, cap, len);
    });
}

int ls_stream_decoder_finish(ls_stream_decoder* d, char* out, size_t cap, size_t* len) {
    return guard([&] {
        need(d, "decoder");
        need(out, "output");
        if (cap < 12) ls::fail("the output buffer must hold 12 bytes");
        give(d->d.finish(), out, cap, len);
    });
}

int ls_sampler_new(float temperature, size_t top_k, float top_p, uint64_t seed, ls_sampler** out) {
    return guard([&] {
        need(out, "output");
        auto s = std::make_unique<ls_sampler>();
        s->s = std::make_unique<ls::Sampler>(temperature, top_k, top_p, seed);
        *out = s.release();
    });
}

void ls_sampler_free(ls_sampler* s) { delete s; }

int ls_sampler_sample(ls_sampler* s, const float* logits, size_t n, uint32_t* token) {
    return guard([&] {
        need(s, "sampler");
        need(token, "token");
        if (n == 0) ls::fail("no logits to sample from");
        need(logits, "logits");
        *token = s->s->sample(logits, n);
    });
}

int ls_matmul_noalloc(ls_format f, const void* w_dev, size_t rows, size_t cols, const float* x_dev, size_t t, float* y_dev,
                      void* stream) {
    return guard([&] {
        need(w_dev, "weights");
        need(x_dev, "input");
        need(y_dev, "output");
        ls::Format F = ls::Format::from(f);
        F.validate({cols});
        if (t == 0 || t > 128) ls::fail("t must be between 1 and 128");
        if (rows == 0 || rows > (1u << 24) || cols > (1u << 24)) ls::fail("matrix shape out of range");
        ls::matmul_static(F.bits, F.group, static_cast<const uint8_t*>(w_dev), int(rows), int(cols), x_dev, int(t), y_dev,
                          static_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
