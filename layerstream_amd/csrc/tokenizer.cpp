// Qwen2 byte-level BPE (src/tokenizer.rs): the files, the pre-token split, rank-ordered merges,
// and UTF-8 handling. Host code only; it never touches the device.
#include "tokenizer.hpp"

#include <algorithm>
#include <cstring>
#include <fstream>
#include <sstream>

#include "common.hpp"
#include "json.hpp"

namespace ls {

#include "unicode_classes.inc"

namespace {

bool in_ranges(const uint32_t (*r)[2], size_t n, uint32_t cp) {
    size_t lo = 0, hi = n;  // first range whose end >= cp
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (r[mid][1] < cp) lo = mid + 1;
        else hi = mid;
    }
    return lo < n && r[lo][0] <= cp;
}

bool is_letter(uint32_t cp) { return in_ranges(kLetterRanges, sizeof kLetterRanges / sizeof kLetterRanges[0], cp); }
bool is_number(uint32_t cp) { return in_ranges(kNumberRanges, sizeof kNumberRanges / sizeof kNumberRanges[0], cp); }
bool is_nl(uint32_t cp) { return cp == '\r' || cp == '\n'; }
// The Unicode White_Space property (the pattern's \s).
bool is_space(uint32_t cp) {
    return (cp >= 0x09 && cp <= 0x0D) || cp == 0x20 || cp == 0x85 || cp == 0xA0 || cp == 0x1680 || (cp >= 0x2000 && cp <= 0x200A) ||
           cp == 0x2028 || cp == 0x2029 || cp == 0x202F || cp == 0x205F || cp == 0x3000;
}

// One UTF-8 sequence at s[i]: its length (> 0, code point in *cp), -k for an invalid maximal
// subpart of k bytes, or 0 when the bytes so far are a valid start that the input cuts short.
int utf8_scan(const std::string& s, size_t i, uint32_t* cp) {
    const auto u = [&](size_t k) { return uint8_t(s[k]); };
    const uint8_t b = u(i);
    if (b < 0x80) {
        *cp = b;
        return 1;
    }
    int len;
    uint8_t lo = 0x80, hi = 0xBF;  // range of the second byte
    uint32_t v;
    if (b >= 0xC2 && b <= 0xDF) {
        len = 2;
        v = b & 0x1F;
    } else if (b >= 0xE0 && b <= 0xEF) {
        len = 3;
        v = b & 0x0F;
        if (b == 0xE0) lo = 0xA0;
        if (b == 0xED) hi = 0x9F;
    } else if (b >= 0xF0 && b <= 0xF4) {
        len = 4;
        v = b & 0x07;
        if (b == 0xF0) lo = 0x90;
        if (b == 0xF4) hi = 0x8F;
    } else {
        return -1;
    }
    for (int k = 1; k < len; k++) {
        if (i + k >= s.size()) return 0;
        const uint8_t c = u(i + k);
        if (k == 1 ? (c < lo || c > hi) : (c < 0x80 || c > 0xBF)) return -k;
        v = (v << 6) | (c & 0x3F);
    }
    *cp = v;
    return len;
}

void put_cp(std::string& o, uint32_t cp) {
    if (cp < 0x80) {
        o += char(cp);
    } else if (cp < 0x800) {
        o += char(0xC0 | (cp >> 6));
        o += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        o += char(0xE0 | (cp >> 12));
        o += char(0x80 | ((cp >> 6) & 0x3F));
        o += char(0x80 | (cp & 0x3F));
    } else {
        o += char(0xF0 | (cp >> 18));
        o += char(0x80 | ((cp >> 12) & 0x3F));
        o += char(0x80 | ((cp >> 6) & 0x3F));
        o += char(0x80 | (cp & 0x3F));
    }
}

const char* const kReplacement = "\xEF\xBF\xBD";  // U+FFFD

std::string read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) fail("cannot read " + path, LS_E_IO);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

bool as_id(const Json& j, uint32_t* id) {
    if (j.kind != Json::Num || !(j.num >= 0) || j.num != double(uint32_t(j.num))) return false;
    *id = uint32_t(j.num);
    return true;
}

}  // namespace

std::vector<uint32_t> utf8_to_cps(const std::string& s) {
    std::vector<uint32_t> out;
    out.reserve(s.size());
    for (size_t i = 0; i < s.size();) {
        uint32_t cp = 0;
        const int r = utf8_scan(s, i, &cp);
        if (r <= 0) fail("text is not valid UTF-8 (byte " + std::to_string(i) + ")");
        out.push_back(cp);
        i += size_t(r);
    }
    return out;
}

std::string cps_to_utf8(const std::vector<uint32_t>& cps, size_t a, size_t b) {
    std::string o;
    for (size_t k = a; k < b; k++) put_cp(o, cps[k]);
    return o;
}

std::string utf8_lossy(const std::string& bytes) {
    std::string o;
    for (size_t i = 0; i < bytes.size();) {
        uint32_t cp = 0;
        const int r = utf8_scan(bytes, i, &cp);
        if (r > 0) {
            o.append(bytes, i, size_t(r));
            i += size_t(r);
        } else {
            o += kReplacement;
            if (r == 0) break;  // a sequence the input cuts short: one replacement for it
            i += size_t(-r);
        }
    }
    return o;
}

std::string StreamDecoder::push(const std::string& bytes) {
    pending_ += bytes;
    std::string out;
    size_t i = 0;
    while (i < pending_.size()) {
        uint32_t cp = 0;
        const int r = utf8_scan(pending_, i, &cp);
        if (r == 0) break;  // incomplete: wait for more bytes
        if (r > 0) {
            out.append(pending_, i, size_t(r));
            i += size_t(r);
        } else {
            out += kReplacement;
            i += size_t(-r);
        }
    }
    pending_.erase(0, i);
    return out;
}

std::string StreamDecoder::finish() {
    std::string out = utf8_lossy(pending_);
    pending_.clear();
    return out;
}

Tokenizer::Tokenizer(const std::string& dir) {
    const std::string base = dir.empty() || dir.back() == '/' ? dir : dir + "/";
    // The GPT-2 byte table: printable bytes stand for themselves, the others for 256, 257, ...
    // in byte order.
    uint32_t next = 256;
    for (uint32_t b = 0; b < 256; b++) {
        const bool printable = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
        byte_cp_[b] = printable ? b : next++;
        cp_byte_[byte_cp_[b]] = uint8_t(b);
    }
    // Vocabulary.
    {
        const std::string text = read_file(base + "vocab.json");
        const Json v = JsonParser(text).parse();
        if (v.kind != Json::Obj) fail("vocab.json: expected an object", LS_E_FORMAT);
        for (const auto& kv : v.obj) {
            uint32_t id;
            if (!as_id(kv.second, &id)) fail("vocab.json: bad id for " + kv.first, LS_E_FORMAT);
            if (id >= strs_.size()) strs_.resize(size_t(id) + 1);
            strs_[id] = kv.first;
        }
    }
    // Added tokens (specials and others), matched literally in text.
    {
        const std::string text = read_file(base + "tokenizer_config.json");
        const Json c = JsonParser(text).parse();
        const Json* dec = c.get("added_tokens_decoder");
        if (dec && dec->kind == Json::Obj) {
            for (const auto& kv : dec->obj) {
                char* end = nullptr;
                const unsigned long id = std::strtoul(kv.first.c_str(), &end, 10);
                if (kv.first.empty() || *end || id > 0xFFFFFFFFul) fail("tokenizer_config.json: bad added token id " + kv.first, LS_E_FORMAT);
                const Json* content = kv.second.get("content");
                if (!content || content->kind != Json::Str) fail("tokenizer_config.json: added token without content", LS_E_FORMAT);
                const Json* sp = kv.second.get("special");
                if (id >= strs_.size()) strs_.resize(size_t(id) + 1);
                strs_[id] = content->str;
                if (is_added_.size() < strs_.size()) is_added_.resize(strs_.size(), false);
                if (special_.size() < strs_.size()) special_.resize(strs_.size(), false);
                is_added_[id] = true;
                special_[id] = sp && sp->kind == Json::Bool && sp->b;
                if (!content->str.empty()) added_.emplace_back(content->str, uint32_t(id));
            }
        }
        std::sort(added_.begin(), added_.end(), [](const auto& a, const auto& b) {
            return a.first.size() != b.first.size() ? a.first.size() > b.first.size() : a.second < b.second;
        });
        is_added_.resize(strs_.size(), false);
        special_.resize(strs_.size(), false);
    }
    // String -> id over the vocabulary (added tokens never come out of merges); the lowest id wins
    // when two share a string.
    ids_.reserve(strs_.size() * 2);
    for (uint32_t id = 0; id < strs_.size(); id++)
        if (!strs_[id].empty() && !is_added_[id]) ids_.emplace(strs_[id], id);
    for (uint32_t b = 0; b < 256; b++) {
        std::string s;
        put_cp(s, byte_cp_[b]);
        auto it = ids_.find(s);
        if (it == ids_.end()) fail("vocab.json: a single-byte token is missing", LS_E_FORMAT);
        byte_id_[b] = it->second;
    }
    // Merges by rank (line order, the version line and empty lines skipped); a repeated pair keeps
    // its first (lowest) rank.
    {
        const std::string text = read_file(base + "merges.txt");
        uint32_t rank = 0;
        size_t at = 0;
        while (at < text.size()) {
            size_t eol = text.find('\n', at);
            if (eol == std::string::npos) eol = text.size();
            std::string line = text.substr(at, eol - at);
            at = eol + 1;
            if (!line.empty() && line.back() == '\r') line.pop_back();
            if (line.empty() || line.compare(0, 8, "#version") == 0) continue;
            const size_t sp = line.find(' ');
            if (sp == std::string::npos) fail("merges.txt: bad line " + line, LS_E_FORMAT);
            const std::string a = line.substr(0, sp), b = line.substr(sp + 1);
            const auto ia = ids_.find(a), ib = ids_.find(b), im = ids_.find(a + b);
            if (ia == ids_.end() || ib == ids_.end()) fail("merges.txt: a merge token is missing from the vocabulary", LS_E_FORMAT);
            if (im == ids_.end()) fail("merges.txt: a merged token is missing from the vocabulary", LS_E_FORMAT);
            merges_.emplace((uint64_t(ia->second) << 32) | ib->second, std::make_pair(rank, im->second));
            rank++;
        }
    }
}

size_t Tokenizer::pretoken_end(const std::vector<uint32_t>& c, size_t i) {
    const size_t n = c.size();
    // (?i:'s|'t|'re|'ve|'m|'ll|'d)
    if (c[i] == '\'') {
        const auto low = [&](size_t k) -> uint32_t { return k < n && c[k] < 128 ? uint32_t(std::tolower(int(c[k]))) : 0; };
        const uint32_t a = low(i + 1), b = low(i + 2);
        if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) return i + 3;
        if (a == 's' || a == 't' || a == 'm' || a == 'd') return i + 2;
    }
    // [^\r\n\p{L}\p{N}]?\p{L}+
    {
        size_t j = i;
        if (!is_nl(c[j]) && !is_letter(c[j]) && !is_number(c[j])) j++;
        if (j < n && is_letter(c[j])) {
            while (j < n && is_letter(c[j])) j++;
            return j;
        }
    }
    // \p{N}
    if (is_number(c[i])) return i + 1;
    // ' '?[^\s\p{L}\p{N}]+[\r\n]*
    {
        const auto symbol = [](uint32_t ch) { return !is_space(ch) && !is_letter(ch) && !is_number(ch); };
        size_t j = i + (c[i] == ' ' ? 1 : 0);
        if (j < n && symbol(c[j])) {
            while (j < n && symbol(c[j])) j++;
            while (j < n && is_nl(c[j])) j++;
            return j;
        }
    }
    if (is_space(c[i])) {
        size_t m = i;
        while (m < n && is_space(c[m])) m++;
        // \s*[\r\n]+: the run up to and including its last newline
        for (size_t k = m; k-- > i;)
            if (is_nl(c[k])) return k + 1;
        // \s+(?!\S): all of it at the end of the text, else all but the last character
        if (m == n) return m;
        if (m - i >= 2) return m - 1;
        // \s+
        return m;
    }
    return i + 1;
}

void Tokenizer::bpe(const std::string& bytes, std::vector<uint32_t>& out) const {
    std::vector<uint32_t> ids(bytes.size()), next;
    for (size_t k = 0; k < bytes.size(); k++) ids[k] = byte_id_[uint8_t(bytes[k])];
    while (ids.size() > 1) {
        // the adjacent pair of lowest rank, then every non-overlapping occurrence of it, left to right
        uint32_t best_rank = UINT32_MAX, left = 0, right = 0, merged = 0;
        for (size_t k = 0; k + 1 < ids.size(); k++) {
            const auto it = merges_.find((uint64_t(ids[k]) << 32) | ids[k + 1]);
            if (it != merges_.end() && it->second.first < best_rank) {
                best_rank = it->second.first;
                left = ids[k];
                right = ids[k + 1];
                merged = it->second.second;
            }
        }
        if (best_rank == UINT32_MAX) break;
        next.clear();
        for (size_t k = 0; k < ids.size();) {
            if (k + 1 < ids.size() && ids[k] == left && ids[k + 1] == right) {
                next.push_back(merged);
                k += 2;
            } else {
                next.push_back(ids[k++]);
            }
        }
        ids.swap(next);
    }
    out.insert(out.end(), ids.begin(), ids.end());
}

void Tokenizer::encode_plain(const std::string& text, std::vector<uint32_t>& out) const {
    const std::vector<uint32_t> cps = utf8_to_cps(text);
    for (size_t i = 0; i < cps.size();) {
        const size_t e = pretoken_end(cps, i);
        bpe(cps_to_utf8(cps, i, e), out);
        i = e;
    }
}

std::vector<uint32_t> Tokenizer::encode(const std::string& text) const {
    std::vector<uint32_t> out;
    size_t pos = 0;
    while (pos < text.size()) {
        // the earliest added token in the rest of the text (the longest of those starting there)
        size_t at = std::string::npos;
        const std::pair<std::string, uint32_t>* hit = nullptr;
        for (const auto& a : added_) {
            const size_t p = text.find(a.first, pos);
            if (p != std::string::npos && p < at) {
                at = p;
                hit = &a;
            }
        }
        if (!hit) {
            encode_plain(text.substr(pos), out);
            break;
        }
        encode_plain(text.substr(pos, at - pos), out);
        out.push_back(hit->second);
        pos = at + hit->first.size();
    }
    return out;
}

std::string Tokenizer::token_bytes(uint32_t id, bool show_special) const {
    if (id >= strs_.size() || strs_[id].empty()) return std::string();
    if (special_[id]) return show_special ? strs_[id] : std::string();
    if (is_added_[id]) return strs_[id];
    std::string o;
    for (uint32_t cp : utf8_to_cps(strs_[id])) {
        const auto it = cp_byte_.find(cp);
        if (it != cp_byte_.end()) o += char(it->second);
    }
    return o;
}

std::string Tokenizer::decode(const uint32_t* ids, size_t n) const {
    std::string bytes;
    for (size_t k = 0; k < n; k++) bytes += token_bytes(ids[k], false);
    return utf8_lossy(bytes);
}

bool Tokenizer::token_id(const std::string& token, uint32_t* id) const {
    for (const auto& a : added_)
        if (a.first == token) {
            *id = a.second;
            return true;
        }
    const auto it = ids_.find(token);
    if (it == ids_.end()) return false;
    *id = it->second;
    return true;
}

}  // namespace ls
