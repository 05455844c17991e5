// Qwen2 byte-level BPE tokenizer (src/tokenizer.rs:56-354) and the incremental UTF-8 decoder
// (src/tokenizer.rs:292-331), host side: text in and token ids out around the device engine.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace ls {

class Tokenizer {
public:
    // vocab.json, merges.txt and tokenizer_config.json (added tokens) of a model directory
    // (src/tokenizer.rs:67-180). Errors: LS_E_IO for a missing file, LS_E_FORMAT for bad content.
    explicit Tokenizer(const std::string& dir);

    // Text (UTF-8) to ids: added tokens such as <|im_start|> matched literally, the rest split
    // into pre-tokens and merged by rank (src/tokenizer.rs:208-280).
    std::vector<uint32_t> encode(const std::string& text) const;
    // Ids to text: special tokens hidden, invalid UTF-8 replaced by U+FFFD (src/tokenizer.rs:282-306).
    std::string decode(const uint32_t* ids, size_t n) const;
    // The bytes a token stands for; special tokens give none unless show_special.
    std::string token_bytes(uint32_t id, bool show_special) const;
    bool token_id(const std::string& token, uint32_t* id) const;
    bool is_special(uint32_t id) const { return id < special_.size() && special_[id]; }
    size_t vocab_size() const { return strs_.size(); }

    // End (exclusive, in code points) of the pre-token starting at cps[i] (the Qwen2 split
    // pattern, src/tokenizer.rs:356-437). Exposed for tests.
    static size_t pretoken_end(const std::vector<uint32_t>& cps, size_t i);

private:
    void encode_plain(const std::string& text, std::vector<uint32_t>& out) const;
    void bpe(const std::string& bytes, std::vector<uint32_t>& out) const;

    std::vector<std::string> strs_;                  // id -> token string (vocabulary and added tokens)
    std::unordered_map<std::string, uint32_t> ids_;  // vocabulary string -> id (not added tokens)
    std::unordered_map<uint64_t, std::pair<uint32_t, uint32_t>> merges_;  // (left << 32 | right) -> (rank, merged)
    uint32_t byte_id_[256] = {};    // id of each single-byte token
    uint32_t byte_cp_[256] = {};    // the printable code point standing for each byte
    std::unordered_map<uint32_t, uint8_t> cp_byte_;  // and back
    std::vector<std::pair<std::string, uint32_t>> added_;  // longest first, then by id
    std::vector<bool> special_, is_added_;
};

// Feed token bytes, get back the text complete so far (src/tokenizer.rs:311-346).
class StreamDecoder {
public:
    std::string push(const std::string& bytes);
    std::string finish();

private:
    std::string pending_;
};

// UTF-8 helpers shared with tests.
std::vector<uint32_t> utf8_to_cps(const std::string& s);  // fails on invalid UTF-8
std::string cps_to_utf8(const std::vector<uint32_t>& cps, size_t a, size_t b);
// Bytes to valid UTF-8, each maximal invalid subsequence replaced by U+FFFD.
std::string utf8_lossy(const std::string& bytes);

}  // namespace ls
