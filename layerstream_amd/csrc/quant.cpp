// Weight quantizer (the reference's src/quant.rs) and the synthetic-weight generator.
//
// The quantizer must produce the reference's bytes exactly, so this file is compiled without
// floating-point contraction: every expression below rounds after each operation, like Rust.
#pragma clang fp contract(off)

#include <atomic>
#include <cmath>
#include <functional>
#include <thread>

#include "common.hpp"

namespace ls {

// Run body(i) for i in [0, n) on `threads` threads handing out indices from a counter.
void parallel_for(size_t n, int threads, const std::function<void(size_t)>& body) {
    if (threads <= 0) threads = default_threads();
    if (threads == 1 || n <= 1) {
        for (size_t i = 0; i < n; i++) body(i);
        return;
    }
    std::atomic<size_t> next{0};
    auto work = [&] {
        for (;;) {
            size_t i = next.fetch_add(1, std::memory_order_relaxed);
            if (i >= n) break;
            body(i);
        }
    };
    std::vector<std::thread> pool;
    int nt = int(std::min<size_t>(size_t(threads), n));
    for (int k = 1; k < nt; k++) pool.emplace_back(work);
    work();
    for (auto& t : pool) t.join();
}

static const float CLIPS[9] = {1.0f, 0.95f, 0.9f, 0.85f, 0.8f, 0.75f, 0.7f, 0.65f, 0.6f};

static inline float round_clamp(float v, float qmax) {
    float r = std::round(v);  // half away from zero, as Rust's f32::round
    return r < -qmax ? -qmax : (r > qmax ? qmax : r);
}

// One group (src/quant.rs:39-75): the first clip ratio with the least squared error wins.
static float quant_group(int bits, const float* w, size_t n, bool clip, int8_t* q, double& err) {
    const float qmax = bits == 8 ? 127.0f : 7.0f;
    float amax = 0.0f;
    for (size_t i = 0; i < n; i++) amax = std::fmax(amax, std::fabs(w[i]));
    auto zeros = [&]() {
        double e = -0.0;
        for (size_t i = 0; i < n; i++) e = e + double(w[i] * w[i]);
        std::memset(q, 0, n);
        err = e;
        return 0.0f;
    };
    if (amax == 0.0f || !std::isfinite(amax)) return zeros();
    double best_err = INFINITY;
    float best_s = 0.0f;
    for (int ci = 0; ci < (clip ? 9 : 1); ci++) {
        float s = bf16_round(CLIPS[ci] * amax / qmax);
        if (s == 0.0f) continue;
        float inv = 1.0f / s;
        double e = 0.0;
        for (size_t i = 0; i < n; i++) {
            float d = w[i] - round_clamp(w[i] * inv, qmax) * s;
            e = e + double(d * d);
        }
        if (e < best_err) {
            best_err = e;
            best_s = s;
        }
    }
    if (best_s == 0.0f) return zeros();
    float inv = 1.0f / best_s;
    for (size_t i = 0; i < n; i++) q[i] = int8_t(round_clamp(w[i] * inv, qmax));
    err = best_err;
    return best_s;
}

// quantize_row (src/quant.rs:79-104): packed integers, then one bf16 scale per group.
void quantize_row(const Format& f, const float* row, size_t cols, bool clip, uint8_t* out, double* err_out, double* norm_out) {
    if (f.is_bf16()) fail("quantize_row needs a quantized format");
    if (f.group > 256 || cols % size_t(f.group) != 0) fail("row width must be a multiple of the group size");
    const size_t G = size_t(f.group);
    uint8_t* scales = out + f.data_bytes(cols);
    int8_t q[256];
    double err = 0.0, norm = 0.0;
    for (size_t g = 0; g < cols / G; g++) {
        const float* wg = row + g * G;
        double e;
        float s = quant_group(f.bits, wg, G, clip, q, e);
        err = err + e;
        double nn = -0.0;
        for (size_t i = 0; i < G; i++) nn = nn + double(wg[i] * wg[i]);
        norm = norm + nn;
        uint16_t sb = f32_to_bf16_bits(s);
        scales[2 * g] = uint8_t(sb);
        scales[2 * g + 1] = uint8_t(sb >> 8);
        if (f.bits == 8) {
            for (size_t j = 0; j < G; j++) out[g * G + j] = uint8_t(q[j]);
        } else {
            const size_t half = G / 2;
            for (size_t j = 0; j < half; j++) out[g * half + j] = uint8_t(uint8_t(q[j] + 8) | uint8_t(q[j + half] + 8) << 4);
        }
    }
    if (err_out) *err_out = err;
    if (norm_out) *norm_out = norm;
}

// Quantize `rows` bf16 rows of `cols` into dst; returns (squared error, squared norm).
static void quantize_matrix(const uint8_t* src, size_t rows, size_t cols, const Format& f, bool clip, uint8_t* dst,
                            int threads, double& err, double& norm) {
    const size_t rb = f.row_bytes(cols), blocks = (rows + 63) / 64;
    std::vector<double> e(blocks), n(blocks);
    parallel_for(blocks, threads, [&](size_t b) {
        std::vector<float> row(cols);
        double eb = 0, nb = 0;
        for (size_t r = b * 64; r < std::min(rows, b * 64 + 64); r++) {
            for (size_t i = 0; i < cols; i++) row[i] = bf16_at(src + r * cols * 2, i);
            double er, nr;
            quantize_row(f, row.data(), cols, clip, dst + r * rb, &er, &nr);
            eb += er;
            nb += nr;
        }
        e[b] = eb;
        n[b] = nb;
    });
    for (size_t b = 0; b < blocks; b++) {
        err += e[b];
        norm += n[b];
    }
}

// quantize_model (src/quant.rs:158-251) over in-memory parts.
std::vector<uint8_t> quantize_model(const std::string& bf16_text, const uint8_t* layers, const uint8_t* embed,
                                    const uint8_t* norm_raw, const Format& fmt, const Format& efmt, bool clip, int threads,
                                    double* rel_rmse) {
    if (fmt.is_bf16()) fail("quantize needs a quantized target format");
    if (efmt.is_bf16()) fail("the embedding table needs a quantized format too");
    Config src = Config::from_json(bf16_text);
    if (!src.format.is_bf16()) fail("the source model is already quantized");
    bool same = fmt == efmt;
    std::string qtext = inject_quant(bf16_text, fmt.bits, fmt.group, same ? 0 : efmt.bits, same ? 0 : efmt.group);
    Config q = Config::from_json(qtext);
    Config as_bf16 = q;
    as_bf16.format = Format{};
    as_bf16.embed_format = Format{};
    if (!as_bf16.same_shape(src)) fail("the config text does not describe the model being quantized");
    LayerLayout sl = src.layout(), dl = q.layout();
    QuantHeader h;
    h.config_text = qtext;
    h.layer_bytes = dl.total;
    h.embed_bytes = q.vocab * q.row_bytes();
    h.norm_bytes = q.hidden * 2;
    std::vector<uint8_t> out = h.to_bytes();
    size_t hl = out.size();
    out.resize(hl + q.layers * dl.total + h.embed_bytes + h.norm_bytes);
    uint8_t* w = out.data() + hl;
    double err = 0, norm = 0;
    for (size_t l = 0; l < q.layers; l++) {
        const uint8_t* in = layers + l * sl.total;
        for (int s = 0; s < N_TENSORS; s++) {
            size_t rows, cols;
            q.slot_shape(s, rows, cols);
            if (!rows) {
                if (sl.len[s] != dl.len[s]) fail("tensor changed size");
                std::memcpy(w + dl.off[s], in + sl.off[s], sl.len[s]);
            } else {
                quantize_matrix(in + sl.off[s], rows, cols, fmt, clip, w + dl.off[s], threads, err, norm);
            }
        }
        w += dl.total;
    }
    quantize_matrix(embed, q.vocab, q.hidden, efmt, clip, w, threads, err, norm);
    w += h.embed_bytes;
    std::memcpy(w, norm_raw, h.norm_bytes);
    if (rel_rmse) *rel_rmse = norm > 0 ? std::sqrt(err / norm) : 0.0;
    return out;
}

// ---------------------------------------------------------------------------------------
// Synthetic weights: SplitMix64 counter stream -> Box-Muller normals -> bf16.
// ---------------------------------------------------------------------------------------
static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Element e of stream `stream`: the pair e/2 gives two normals (cos and sin branches).
static inline double synth_normal(uint64_t seed, uint64_t stream, uint64_t e) {
    uint64_t key = (stream << 40) | (e >> 1);
    uint64_t h1 = mix64(seed ^ mix64(key)), h2 = mix64(h1);
    double u1 = double((h1 >> 11) + 1) * (1.0 / 9007199254740992.0);  // (0, 1]
    double u2 = double(h2 >> 11) * (1.0 / 9007199254740992.0);        // [0, 1)
    double r = std::sqrt(-2.0 * std::log(u1));
    double a = 6.283185307179586 * u2;
    return (e & 1) ? r * std::sin(a) : r * std::cos(a);
}

static void synth_tensor(uint64_t seed, uint64_t stream, size_t n, float std_dev, bool is_norm, uint8_t* out, int threads) {
    const size_t chunk = 1 << 16, nchunks = (n + chunk - 1) / chunk;
    parallel_for(nchunks, threads, [&](size_t c) {
        for (size_t e = c * chunk; e < std::min(n, (c + 1) * chunk); e++) {
            double z = synth_normal(seed, stream, e) * double(std_dev);
            float v = is_norm ? float(1.0 + z) : float(z);
            uint16_t b = f32_to_bf16_bits(bf16_round(v));
            out[2 * e] = uint8_t(b);
            out[2 * e + 1] = uint8_t(b >> 8);
        }
    });
}

void synth_bf16_model(const Config& c, uint64_t seed, float std_dev, uint8_t* layers, uint8_t* embed, uint8_t* norm, int threads) {
    if (!c.format.is_bf16() || !c.embed_format.is_bf16()) fail("synthetic weights are generated as bf16");
    LayerLayout L = c.layout();
    for (size_t l = 0; l < c.layers; l++)
        for (int s = 0; s < N_TENSORS; s++) {
            bool is_norm = s == T_INPUT_NORM || s == T_POST_NORM;
            synth_tensor(seed, l * N_TENSORS + s, L.len[s] / 2, std_dev, is_norm, layers + l * L.total + L.off[s], threads);
        }
    synth_tensor(seed, c.layers * N_TENSORS, c.vocab * c.hidden, std_dev, false, embed, threads);
    synth_tensor(seed, c.layers * N_TENSORS + 1, c.hidden, std_dev, true, norm, threads);
}

}  // namespace ls
