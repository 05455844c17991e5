// Byte sources: in-memory parts, `.lsq` images and `.lsq` files.
#include "source.hpp"

#include <hip/hip_runtime.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

namespace ls {

void Source::init(const Config& c, const uint8_t* norm_raw) {
    cfg_ = c;
    layout_ = c.layout();
    final_norm_.resize(c.hidden);
    for (size_t i = 0; i < c.hidden; i++) final_norm_[i] = bf16_at(norm_raw, i);
}

void Source::check_layer(size_t l) const {
    if (l >= cfg_.layers) fail("layer " + std::to_string(l) + " out of range");
}

void Source::check_rows(size_t first, size_t rows) const {
    if (first + rows > cfg_.vocab) fail("embedding range out of bounds");
}

MemorySource::MemorySource(const std::string& config_json, const uint8_t* layers, size_t layers_len, const uint8_t* embed,
                           size_t embed_len, const uint8_t* norm, size_t norm_len) {
    Config c = Config::from_json(config_json);
    LayerLayout L = c.layout();
    if (!layers || !embed || !norm) fail("memory source needs layers, embedding and final norm");
    if (layers_len != c.layers * L.total) fail("layer bytes do not match the config", LS_E_FORMAT);
    if (embed_len != c.vocab * c.row_bytes()) fail("embedding bytes do not match the config", LS_E_FORMAT);
    if (norm_len != c.hidden * 2) fail("final norm bytes do not match the config", LS_E_FORMAT);
    layers_ = layers;
    embed_ = embed;
    init(c, norm);
}

void MemorySource::read_layer(size_t l, uint8_t* buf) const {
    check_layer(l);
    std::memcpy(buf, layers_ + l * layout_.total, layout_.total);
    bytes_read_.fetch_add(layout_.total, std::memory_order_relaxed);
}

void MemorySource::read_embed_rows(size_t first, size_t rows, uint8_t* buf) const {
    check_rows(first, rows);
    size_t rb = cfg_.row_bytes();
    std::memcpy(buf, embed_ + first * rb, rows * rb);
    bytes_read_.fetch_add(rows * rb, std::memory_order_relaxed);
}

// ModelFiles::open_quantized checks (src/weights.rs:391-407).
static Config check_quantized(const QuantHeader& h, size_t file_len) {
    Config c = Config::from_json(h.config_text);
    if (c.format.is_bf16()) fail("this file does not describe quantized weights", LS_E_FORMAT);
    LayerLayout L = c.layout();
    if (L.total != h.layer_bytes || c.vocab * c.row_bytes() != h.embed_bytes || c.hidden * 2 != h.norm_bytes)
        fail("quantized header does not match the model's shape", LS_E_FORMAT);
    size_t want = h.data_start + c.layers * L.total + h.embed_bytes + h.norm_bytes;
    if (file_len != want)
        fail("file is " + std::to_string(file_len) + " bytes but its header implies " + std::to_string(want), LS_E_FORMAT);
    return c;
}

LsqImageSource::LsqImageSource(const uint8_t* image, size_t len) {
    if (!image) fail("no image");
    QuantHeader h = QuantHeader::parse(image, len, len);
    Config c = check_quantized(h, len);
    layers_ = image + h.data_start;
    embed_ = layers_ + c.layers * c.layout().total;
    init(c, embed_ + h.embed_bytes);
}

PinnedSource::PinnedSource(const Source& src) {
    const Config& c = src.cfg();
    size_t lb = c.layers * src.layout().total, eb = c.vocab * c.row_bytes();
    if (hipHostMalloc(&mem_, lb + eb, hipHostMallocDefault) != hipSuccess || !mem_)
        fail("cannot allocate pinned host memory for the model", LS_E_DEVICE);
    uint8_t* m = static_cast<uint8_t*>(mem_);
    for (size_t l = 0; l < c.layers; l++) src.read_layer(l, m + l * src.layout().total);
    for (size_t first = 0; first < c.vocab; first += 4096) {
        size_t rows = std::min<size_t>(4096, c.vocab - first);
        src.read_embed_rows(first, rows, m + lb + first * c.row_bytes());
    }
    layers_ = m;
    embed_ = m + lb;
    cfg_ = c;
    layout_ = src.layout();
    final_norm_ = src.final_norm();
}

PinnedSource::~PinnedSource() {
    if (mem_) (void)hipHostFree(mem_);
}

LsqFileSource::LsqFileSource(const std::string& path) : path_(path) {
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) fail(path + ": cannot open", LS_E_IO);
    struct stat st {};
    if (fstat(fd_, &st) != 0) fail(path + ": cannot stat", LS_E_IO);
    size_t len = size_t(st.st_size);
    std::vector<uint8_t> head(std::min<size_t>(len, 8 + (1u << 20)));
    ssize_t got = pread(fd_, head.data(), head.size(), 0);
    if (got < 0) fail(path + ": read failed", LS_E_IO);
    QuantHeader h = QuantHeader::parse(head.data(), size_t(got), len);
    Config c = check_quantized(h, len);
    data_start_ = h.data_start;
    embed_start_ = data_start_ + c.layers * c.layout().total;
    std::vector<uint8_t> norm(h.norm_bytes);
    read_at(norm.data(), norm.size(), embed_start_ + h.embed_bytes);
    init(c, norm.data());
    bytes_read_.store(0);
}

LsqFileSource::~LsqFileSource() {
    if (fd_ >= 0) ::close(fd_);
}

void LsqFileSource::read_at(uint8_t* buf, size_t len, size_t off) const {
    size_t done = 0;
    while (done < len) {
        ssize_t n = pread(fd_, buf + done, len - done, off_t(off + done));
        if (n <= 0) fail("read at " + std::to_string(off + done) + " failed", LS_E_IO);
        done += size_t(n);
    }
    bytes_read_.fetch_add(len, std::memory_order_relaxed);
}

void LsqFileSource::read_layer(size_t l, uint8_t* buf) const {
    check_layer(l);
    read_at(buf, layout_.total, data_start_ + l * layout_.total);
}

void LsqFileSource::read_embed_rows(size_t first, size_t rows, uint8_t* buf) const {
    check_rows(first, rows);
    size_t rb = cfg_.row_bytes();
    read_at(buf, rows * rb, embed_start_ + first * rb);
}

}  // namespace ls
