// Shared host-side types of the engine: errors, bf16 helpers, model config and formats.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "layerstream.h"

namespace ls {

// An error that crosses the C ABI as a negative code plus a thread-local message (the
// reference's `Err(String)`).
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] inline void fail(const std::string& m, int code = LS_E_INVALID) { throw Error(code, m); }

void set_last_error(const std::string& m);

inline float bf16_to_f32(uint16_t b) {
    uint32_t u = uint32_t(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline float bf16_at(const uint8_t* p, size_t i) { return bf16_to_f32(uint16_t(p[2 * i] | (p[2 * i + 1] << 8))); }

// Round to the nearest bf16, ties to even; NaN passes through (src/quant.rs:26-33).
inline float bf16_round(float v) {
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return v;
    uint32_t r = (bits + 0x7fffu + ((bits >> 16) & 1u)) & 0xffff0000u;
    float f;
    std::memcpy(&f, &r, 4);
    return f;
}

inline uint16_t f32_to_bf16_bits(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    return uint16_t(u >> 16);
}

struct Format {
    int bits = 16;  // 16 (bf16), 8 or 4
    int group = 0;
    bool is_bf16() const { return bits == 16; }
    size_t row_bytes(size_t cols) const {
        return is_bf16() ? cols * 2 : cols * size_t(bits) / 8 + cols / size_t(group) * 2;
    }
    // Bytes of the packed integers (or bf16 values) of one row.
    size_t data_bytes(size_t cols) const { return is_bf16() ? cols * 2 : cols * size_t(bits) / 8; }
    void validate(const std::vector<size_t>& cols) const;
    bool operator==(const Format& o) const { return bits == o.bits && (is_bf16() || group == o.group); }
    bool operator!=(const Format& o) const { return !(*this == o); }
    ls_format c() const { return ls_format{bits, group}; }
    static Format from(ls_format f) { return Format{f.bits, f.group}; }
};

// Tensor slots of a layer block in storage order (src/weights.rs:158-171).
enum Slot { T_INPUT_NORM, T_DOWN, T_GATE, T_UP, T_POST_NORM, T_K_B, T_K_W, T_O_W, T_Q_B, T_Q_W, T_V_B, T_V_W, N_TENSORS };

struct LayerLayout {
    size_t off[N_TENSORS] = {};
    size_t len[N_TENSORS] = {};
    size_t total = 0;
};

struct Config {
    Format format, embed_format;
    size_t hidden = 0, inter = 0, layers = 0, heads = 0, kv_heads = 0, head_dim = 0, vocab = 0, max_pos = 0;
    float eps = 0, rope_theta = 0;

    size_t kv_dim() const { return kv_heads * head_dim; }
    size_t row_bytes() const { return embed_format.row_bytes(hidden); }  // one embedding row
    // (rows, cols) of a matrix slot, or (0, len) for a vector slot (src/weights.rs:188-211).
    void slot_shape(int slot, size_t& rows, size_t& cols) const;
    LayerLayout layout() const;  // layer_layout_for (src/weights.rs:215-227)
    ls_config c() const;
    static Config from(const ls_config& c);
    static Config from_json(const std::string& text);  // src/weights.rs:77-141
    bool same_shape(const Config& o) const;
};

// .lsq header (src/weights.rs:327-387).
struct QuantHeader {
    std::string config_text;
    size_t layer_bytes = 0, embed_bytes = 0, norm_bytes = 0;
    size_t data_start = 0;
    std::vector<uint8_t> to_bytes() const;
    static QuantHeader parse(const uint8_t* data, size_t avail, size_t file_len);
};

std::string inject_quant(const std::string& config_text, int bits, int group, int embed_bits, int embed_group);
std::string json_escape(const std::string& s);

int default_threads();
const std::string& last_error();

// quant.cpp
void parallel_for(size_t n, int threads, const std::function<void(size_t)>& body);
void quantize_row(const Format& f, const float* row, size_t cols, bool clip, uint8_t* out, double* err, double* norm);
std::vector<uint8_t> quantize_model(const std::string& bf16_text, const uint8_t* layers, const uint8_t* embed,
                                    const uint8_t* norm_raw, const Format& fmt, const Format& efmt, bool clip, int threads,
                                    double* rel_rmse);
void synth_bf16_model(const Config& c, uint64_t seed, float std_dev, uint8_t* layers, uint8_t* embed, uint8_t* norm,
                      int threads);

}  // namespace ls
