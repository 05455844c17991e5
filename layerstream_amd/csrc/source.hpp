// Byte sources (trait Source, src/source.rs:23-33): where layer blocks and embedding rows come
// from. A Source knows nothing about device memory; providers decide what to keep resident.
#pragma once

#include <atomic>
#include <string>
#include <vector>

#include "common.hpp"

namespace ls {

class Source {
public:
    virtual ~Source() = default;
    const Config& cfg() const { return cfg_; }
    const LayerLayout& layout() const { return layout_; }
    const std::vector<float>& final_norm() const { return final_norm_; }
    // Fill buf (layout().total bytes) with layer l's block (src/source.rs:26).
    virtual void read_layer(size_t l, uint8_t* buf) const = 0;
    // Fill buf (rows * row_bytes) with embedding rows first..first+rows (src/source.rs:28).
    virtual void read_embed_rows(size_t first, size_t rows, uint8_t* buf) const = 0;
    // Zero-copy views when the bytes already sit in memory (nullptr otherwise).
    virtual const uint8_t* layer_view(size_t) const { return nullptr; }
    virtual const uint8_t* embed_view() const { return nullptr; }
    // True when the views are pinned host memory (direct DMA to the device).
    virtual bool pinned() const { return false; }
    uint64_t bytes_read() const { return bytes_read_.load(std::memory_order_relaxed); }
    void count_read(uint64_t n) const { bytes_read_.fetch_add(n, std::memory_order_relaxed); }
    virtual std::string describe() const = 0;

protected:
    void init(const Config& c, const uint8_t* norm_raw);
    void check_layer(size_t l) const;
    void check_rows(size_t first, size_t rows) const;
    Config cfg_;
    LayerLayout layout_;
    std::vector<float> final_norm_;
    mutable std::atomic<uint64_t> bytes_read_{0};
};

// Borrowed in-memory parts: layer blocks, embedding table, final norm.
class MemorySource : public Source {
public:
    MemorySource(const std::string& config_json, const uint8_t* layers, size_t layers_len, const uint8_t* embed,
                 size_t embed_len, const uint8_t* norm, size_t norm_len);
    void read_layer(size_t l, uint8_t* buf) const override;
    void read_embed_rows(size_t first, size_t rows, uint8_t* buf) const override;
    const uint8_t* layer_view(size_t l) const override { return layers_ + l * layout_.total; }
    const uint8_t* embed_view() const override { return embed_; }
    std::string describe() const override { return "memory"; }

protected:
    MemorySource() = default;
    const uint8_t* layers_ = nullptr;
    const uint8_t* embed_ = nullptr;
};

// A `.lsq` image in memory (src/weights.rs:389-424 checks).
class LsqImageSource : public MemorySource {
public:
    LsqImageSource(const uint8_t* image, size_t len);
    std::string describe() const override { return "lsq image"; }
};

// A copy of another source's bytes in pinned host memory (hipHostMalloc), so streamed layers
// reach the device by DMA straight from it.
class PinnedSource : public MemorySource {
public:
    explicit PinnedSource(const Source& src);
    ~PinnedSource() override;
    bool pinned() const override { return true; }
    std::string describe() const override { return "pinned host memory"; }

private:
    void* mem_ = nullptr;
};

// A `.lsq` file read with positioned reads (FileSource, src/source.rs:90-182).
class LsqFileSource : public Source {
public:
    explicit LsqFileSource(const std::string& path);
    ~LsqFileSource() override;
    void read_layer(size_t l, uint8_t* buf) const override;
    void read_embed_rows(size_t first, size_t rows, uint8_t* buf) const override;
    std::string describe() const override { return "lsq file " + path_; }

private:
    void read_at(uint8_t* buf, size_t len, size_t off) const;
    std::string path_;
    int fd_ = -1;
    size_t data_start_ = 0, embed_start_ = 0;
};

}  // namespace ls
