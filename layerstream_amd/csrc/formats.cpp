// Config parsing, weight formats, the layer-block layout and the `.lsq` header: the byte-level
// contracts of src/weights.rs, src/quant.rs:137-145 and src/json.rs that the engine reads.
#include <algorithm>
#include <cmath>
#include <map>
#include <memory>
#include <thread>

#include "common.hpp"
#include "json.hpp"

namespace ls {

static thread_local std::string g_last_error;
void set_last_error(const std::string& m) { g_last_error = m; }
const std::string& last_error() { return g_last_error; }

int default_threads() {
    unsigned n = std::thread::hardware_concurrency();
    return n ? int(n) : 4;
}

// Json::as_u64 (src/json.rs:50-55): a non-negative integral number below 9e15.
static bool as_u64(const Json* j, uint64_t& out) {
    if (!j || j->kind != Json::Num) return false;
    double n = j->num;
    if (!(n >= 0.0) || std::floor(n) != n || n >= 9.0e15) return false;
    out = uint64_t(n);
    return true;
}

// Json::Str(..).to_text() (src/json.rs:84-99).
std::string json_escape(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        switch (c) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            default:
                if (c < 0x20) {
                    char b[8];
                    snprintf(b, sizeof b, "\\u%04x", c);
                    o += b;
                } else {
                    o += char(c);
                }
        }
    }
    return o + "\"";
}

// ---------------------------------------------------------------------------------------
// Formats and config
// ---------------------------------------------------------------------------------------
void Format::validate(const std::vector<size_t>& cols) const {
    if (is_bf16()) return;
    if (bits != 8 && bits != 4) fail("quantization supports 8 or 4 bits, not " + std::to_string(bits));
    if (group < 16 || group > 256 || group % 16 != 0)
        fail("group size must be a multiple of 16 between 16 and 256, not " + std::to_string(group));
    for (size_t c : cols)
        if (c % size_t(group) != 0)
            fail("group size " + std::to_string(group) + " does not divide a matrix width of " + std::to_string(c));
}

void Config::slot_shape(int slot, size_t& rows, size_t& cols) const {
    size_t h = hidden, i = inter, kv = kv_dim();
    switch (slot) {
        case T_INPUT_NORM: case T_POST_NORM: case T_Q_B: rows = 0; cols = h; break;
        case T_K_B: case T_V_B: rows = 0; cols = kv; break;
        case T_DOWN: rows = h; cols = i; break;
        case T_GATE: case T_UP: rows = i; cols = h; break;
        case T_K_W: case T_V_W: rows = kv; cols = h; break;
        default: rows = h; cols = h; break;  // T_O_W, T_Q_W
    }
}

LayerLayout Config::layout() const {
    LayerLayout L;
    size_t off = 0;
    for (int s = 0; s < N_TENSORS; s++) {
        size_t rows, cols;
        slot_shape(s, rows, cols);
        size_t len = rows ? rows * format.row_bytes(cols) : cols * 2;
        L.off[s] = off;
        L.len[s] = len;
        off += len;
    }
    L.total = off;
    return L;
}

ls_config Config::c() const {
    ls_config o{};
    o.format = format.c();
    o.embed_format = embed_format.c();
    o.hidden = int64_t(hidden);
    o.inter = int64_t(inter);
    o.layers = int64_t(layers);
    o.heads = int64_t(heads);
    o.kv_heads = int64_t(kv_heads);
    o.head_dim = int64_t(head_dim);
    o.vocab = int64_t(vocab);
    o.max_pos = int64_t(max_pos);
    o.eps = eps;
    o.rope_theta = rope_theta;
    return o;
}

Config Config::from(const ls_config& c) {
    Config o;
    o.format = Format::from(c.format);
    o.embed_format = Format::from(c.embed_format);
    if (c.hidden <= 0 || c.inter <= 0 || c.layers <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.vocab <= 0)
        fail("config sizes must be positive");
    o.hidden = size_t(c.hidden);
    o.inter = size_t(c.inter);
    o.layers = size_t(c.layers);
    o.heads = size_t(c.heads);
    o.kv_heads = size_t(c.kv_heads);
    o.head_dim = c.head_dim > 0 ? size_t(c.head_dim) : o.hidden / o.heads;
    o.vocab = size_t(c.vocab);
    o.max_pos = c.max_pos > 0 ? size_t(c.max_pos) : 0;
    o.eps = c.eps;
    o.rope_theta = c.rope_theta;
    if (o.hidden % o.heads != 0 || o.heads % o.kv_heads != 0 || o.head_dim * o.heads != o.hidden)
        fail("inconsistent head configuration");
    if (o.head_dim % 2 != 0) fail("head dimension must be even for rotary embeddings");
    o.format.validate({o.hidden, o.inter});
    o.embed_format.validate({o.hidden});
    return o;
}

bool Config::same_shape(const Config& o) const {
    return hidden == o.hidden && inter == o.inter && layers == o.layers && heads == o.heads && kv_heads == o.kv_heads &&
           head_dim == o.head_dim && vocab == o.vocab && eps == o.eps && rope_theta == o.rope_theta && max_pos == o.max_pos;
}

Config Config::from_json(const std::string& text) {
    Json j = JsonParser(text).parse();
    auto u = [&](const char* k) -> size_t {
        uint64_t v;
        if (!as_u64(j.get(k), v)) fail(std::string("config.json: missing integer ") + k, LS_E_FORMAT);
        return size_t(v);
    };
    auto f = [&](const char* k) -> float {
        const Json* v = j.get(k);
        if (!v || v->kind != Json::Num) fail(std::string("config.json: missing number ") + k, LS_E_FORMAT);
        return float(v->num);
    };
    auto str_is = [&](const char* k, const char* want) {
        const Json* v = j.get(k);
        return v && v->kind == Json::Str && v->str == want;
    };
    if (!str_is("model_type", "qwen2")) fail("only Qwen2-architecture models are supported", LS_E_FORMAT);
    if (!str_is("hidden_act", "silu")) fail("only SiLU activations are supported", LS_E_FORMAT);
    const Json* tie = j.get("tie_word_embeddings");
    if (!tie || tie->kind != Json::Bool || !tie->b)
        fail("only models with tied input/output embeddings are supported", LS_E_FORMAT);
    Config c;
    c.hidden = u("hidden_size");
    c.heads = u("num_attention_heads");
    c.kv_heads = u("num_key_value_heads");
    if (c.heads == 0 || c.kv_heads == 0 || c.hidden % c.heads != 0 || c.heads % c.kv_heads != 0)
        fail("inconsistent head configuration", LS_E_FORMAT);
    c.head_dim = c.hidden / c.heads;
    if (c.head_dim % 2 != 0) fail("head dimension must be even for rotary embeddings", LS_E_FORMAT);
    c.inter = u("intermediate_size");
    const Json* q = j.get("layerstream_quant");
    if (q) {
        auto get = [&](const char* k) -> uint64_t {
            uint64_t v;
            if (!as_u64(q->get(k), v)) fail(std::string("config: layerstream_quant is missing ") + k, LS_E_FORMAT);
            return v;
        };
        auto quant = [&](const char* bk, const char* gk) -> Format {
            uint64_t bits = get(bk), group = get(gk);
            if (bits > 255 || group > 4096) fail("config: implausible layerstream_quant values", LS_E_FORMAT);
            return Format{int(bits), int(group)};
        };
        c.format = quant("bits", "group");
        bool eb = q->get("embed_bits") != nullptr, eg = q->get("embed_group") != nullptr;
        if (!eb && !eg) c.embed_format = c.format;
        else if (eb && eg) c.embed_format = quant("embed_bits", "embed_group");
        else fail("config: layerstream_quant needs embed_bits and embed_group together", LS_E_FORMAT);
        if (c.format.is_bf16() || c.embed_format.is_bf16())
            fail("quantization supports 8 or 4 bits, not 16", LS_E_FORMAT);
    }
    try {
        c.format.validate({c.hidden, c.inter});
        c.embed_format.validate({c.hidden});
    } catch (const Error& e) {
        throw Error(LS_E_FORMAT, e.what());
    }
    c.layers = u("num_hidden_layers");
    c.vocab = u("vocab_size");
    c.eps = f("rms_norm_eps");
    c.rope_theta = f("rope_theta");
    c.max_pos = u("max_position_embeddings");
    if (c.layers == 0 || c.vocab == 0) fail("config: a model needs layers and a vocabulary", LS_E_FORMAT);
    return c;
}

// ---------------------------------------------------------------------------------------
// .lsq header (src/weights.rs:340-387)
// ---------------------------------------------------------------------------------------
static const char* QUANT_FORMAT = "layerstream-quant-1";

std::vector<uint8_t> QuantHeader::to_bytes() const {
    std::string json = std::string("{\"format\":\"") + QUANT_FORMAT + "\",\"config_json\":" + json_escape(config_text) +
                       ",\"layer_bytes\":" + std::to_string(layer_bytes) + ",\"embed_bytes\":" + std::to_string(embed_bytes) +
                       ",\"norm_bytes\":" + std::to_string(norm_bytes) + "}";
    std::vector<uint8_t> out(8 + json.size());
    std::memcpy(out.data(), "LSQ1", 4);
    uint32_t n = uint32_t(json.size());
    for (int k = 0; k < 4; k++) out[4 + k] = uint8_t(n >> (8 * k));
    std::memcpy(out.data() + 8, json.data(), json.size());
    return out;
}

QuantHeader QuantHeader::parse(const uint8_t* data, size_t avail, size_t file_len) {
    if (file_len < 8 || avail < 8) fail("file too short to be a quantized model", LS_E_FORMAT);
    if (std::memcmp(data, "LSQ1", 4) != 0) fail("not a quantized layerstream model (bad magic bytes)", LS_E_FORMAT);
    uint32_t len = uint32_t(data[4]) | uint32_t(data[5]) << 8 | uint32_t(data[6]) << 16 | uint32_t(data[7]) << 24;
    if (len == 0 || len > (1u << 20)) fail("implausible quantized header length", LS_E_FORMAT);
    if (8 + size_t(len) > avail) fail("quantized header: file too short", LS_E_FORMAT);
    std::string text(reinterpret_cast<const char*>(data + 8), len);
    Json j = JsonParser(text).parse();
    const Json* fm = j.get("format");
    if (!fm || fm->kind != Json::Str || fm->str != QUANT_FORMAT) fail("unknown quantized file format", LS_E_FORMAT);
    auto u = [&](const char* k) -> size_t {
        uint64_t v;
        if (!as_u64(j.get(k), v)) fail(std::string("quantized header: missing ") + k, LS_E_FORMAT);
        return size_t(v);
    };
    QuantHeader h;
    const Json* cj = j.get("config_json");
    if (!cj || cj->kind != Json::Str) fail("quantized header: missing config", LS_E_FORMAT);
    h.config_text = cj->str;
    h.layer_bytes = u("layer_bytes");
    h.embed_bytes = u("embed_bytes");
    h.norm_bytes = u("norm_bytes");
    h.data_start = 8 + len;
    return h;
}

std::string inject_quant(const std::string& text, int bits, int group, int embed_bits, int embed_group) {
    size_t end = text.rfind('}');
    if (end == std::string::npos) fail("config.json has no closing brace", LS_E_FORMAT);
    std::string head = text.substr(0, end);
    while (!head.empty() && (head.back() == ' ' || head.back() == '\n' || head.back() == '\r' || head.back() == '\t')) head.pop_back();
    std::string extra;
    if (embed_bits) extra = ",\"embed_bits\":" + std::to_string(embed_bits) + ",\"embed_group\":" + std::to_string(embed_group);
    return head + ",\"layerstream_quant\":{\"bits\":" + std::to_string(bits) + ",\"group\":" + std::to_string(group) + extra + "}}";
}

}  // namespace ls
