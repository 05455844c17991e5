// The device Model (src/model.rs) and its providers (src/provider.rs) on one MI355X.
//
// HBM layout: per layer one arena holding the fused q|k|v matrix (q and k rows with each head's
// RoPE pairs adjacent), o, the fused gate|up matrix (32-row blocks of gate and up interleaved)
// and down in the tile layout (fused.hpp), then the q|k|v bias and the two RMSNorm weight
// vectors as f32. The tied embedding table is one tile-layout matrix used both for the
// embedding gather and as the output head. The KV cache is f32 [layer][max_ctx][kv_dim] for K
// and for V, as the reference's (src/model.rs:67-68); rollback is O(1) (only `pos` moves).
//
// A forward pass over t tokens (every 16-token tile in each launch) runs per layer: QKV (1/rms,
// bias, RoPE and K/V append in the epilogue), attention (chunks and their combine in one
// launch), O projection (+ residual, then the fragments of x * post_norm), gate|up (1/rms and
// SiLU(g) * u into fragments) and down (+ residual, then the fragments of x * the next norm);
// then the head (persistent, argmax partials) and the argmax reduction. Every kernel reads its
// input as fragments written by the one before; the verify step is replayed from a HIP graph.
#include "model.hpp"

#include <chrono>
#include <cmath>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <thread>
#include <cstdio>
#include <cstdlib>

namespace ls {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(LS_E_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

DevBuf::DevBuf(size_t bytes) : n(bytes) {
    if (bytes) HIPC(hipMalloc(&p, bytes));
}
DevBuf::~DevBuf() {
    if (p) (void)hipFree(p);
}
DevBuf& DevBuf::operator=(DevBuf&& o) noexcept {
    if (this != &o) {
        if (p) (void)hipFree(p);
        p = o.p;
        n = o.n;
        o.p = nullptr;
        o.n = 0;
    }
    return *this;
}

PinnedBuf::PinnedBuf(size_t bytes) : n(bytes) {
    if (bytes) HIPC(hipHostMalloc(&p, bytes, hipHostMallocDefault));
}
PinnedBuf::~PinnedBuf() {
    if (p) (void)hipHostFree(p);
}
PinnedBuf& PinnedBuf::operator=(PinnedBuf&& o) noexcept {
    if (this != &o) {
        if (p) (void)hipHostFree(p);
        p = o.p;
        n = o.n;
        o.p = nullptr;
        o.n = 0;
    }
    return *this;
}

static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

static void mat_region(size_t& off, size_t& d, size_t& s, const TMat& m) {
    d = off;
    off = align256(off + tile_data_bytes(m));
    s = off;
    off = align256(off + tile_scale_bytes(m));
}

LayerArena layer_arena(const Config& c) {
    LayerArena a{};
    const int h = int(c.hidden), kv = int(c.kv_dim()), in = int(c.inter), b = c.format.bits, g = c.format.group;
    a.qkv = tile_shape(b, g, h + 2 * kv, h);
    a.o = tile_shape(b, g, h, h);
    a.gu = tile_shape(b, g, 2 * in, h);
    a.down = tile_shape(b, g, h, in);
    size_t off = 0;
    mat_region(off, a.qkv_d, a.qkv_s, a.qkv);
    mat_region(off, a.o_d, a.o_s, a.o);
    mat_region(off, a.gu_d, a.gu_s, a.gu);
    mat_region(off, a.down_d, a.down_s, a.down);
    a.b_qkv = off;
    off = align256(off + 4 * size_t(h + 2 * kv));
    a.in_norm = off;
    off = align256(off + 4 * size_t(h));
    a.post_norm = off;
    off = align256(off + 4 * size_t(h));
    a.total = off;
    return a;
}

DevLayer bind_layer(const LayerArena& a, uint8_t* b) {
    DevLayer L;
    L.qkv = tile_bind(a.qkv, b + a.qkv_d, reinterpret_cast<uint16_t*>(b + a.qkv_s));
    L.o = tile_bind(a.o, b + a.o_d, reinterpret_cast<uint16_t*>(b + a.o_s));
    L.gu = tile_bind(a.gu, b + a.gu_d, reinterpret_cast<uint16_t*>(b + a.gu_s));
    L.down = tile_bind(a.down, b + a.down_d, reinterpret_cast<uint16_t*>(b + a.down_s));
    L.b_qkv = reinterpret_cast<const float*>(b + a.b_qkv);
    L.in_norm = reinterpret_cast<const float*>(b + a.in_norm);
    L.post_norm = reinterpret_cast<const float*>(b + a.post_norm);
    return L;
}

void clear_layer(const LayerArena& a, uint8_t* b, hipStream_t s) {
    HIPC(hipMemsetAsync(b, 0, a.total, s));
    DevLayer L = bind_layer(a, b);
    tile_clear(L.qkv, s);
    tile_clear(L.o, s);
    tile_clear(L.gu, s);
    tile_clear(L.down, s);
}

void build_layer_device(const Config& c, const LayerLayout& L, const uint8_t* raw, const LayerArena& a, uint8_t* b,
                        hipStream_t s) {
    const int h = int(c.hidden), kv = int(c.kv_dim()), in = int(c.inter);
    const DevLayer D = bind_layer(a, b);
    const int hd = int(c.head_dim), gb = 16 * GU_STRIPS;
    tile_repack(raw + L.off[T_Q_W], h, D.qkv, 0, h, h, s, hd);
    tile_repack(raw + L.off[T_K_W], kv, D.qkv, h, kv, kv, s, hd);
    tile_repack(raw + L.off[T_V_W], kv, D.qkv, h + kv, kv, kv, s);
    tile_repack(raw + L.off[T_O_W], h, D.o, 0, h, h, s);
    tile_repack(raw + L.off[T_GATE], in, D.gu, 0, gb, 2 * gb, s);
    tile_repack(raw + L.off[T_UP], in, D.gu, gb, gb, 2 * gb, s);
    tile_repack(raw + L.off[T_DOWN], h, D.down, 0, h, h, s);
    float* bq = reinterpret_cast<float*>(b + a.b_qkv);
    Widen w;
    w.add(raw + L.off[T_Q_B], h, bq);
    w.add(raw + L.off[T_K_B], kv, bq + h);
    w.add(raw + L.off[T_V_B], kv, bq + h + kv);
    w.add(raw + L.off[T_INPUT_NORM], h, reinterpret_cast<float*>(b + a.in_norm));
    w.add(raw + L.off[T_POST_NORM], h, reinterpret_cast<float*>(b + a.post_norm));
    bf16_to_f32_dev(w, s);
}

// ---------------------------------------------------------------------------------------
// Resident: every layer and the whole table in HBM (ResidentProvider, src/provider.rs:61-137)
// ---------------------------------------------------------------------------------------
class ResidentProvider : public DeviceProvider {
public:
    ResidentProvider(const Source& src, hipStream_t s) : src_(src), c_(src.cfg()), a_(layer_arena(c_)), s_(s) {
        const LayerLayout L = src.layout();
        arena_ = DevBuf(a_.total * c_.layers);
        const size_t rb = c_.row_bytes();
        const size_t stage_bytes = std::max(L.total, HEAD_ROWS * rb);
        PinnedBuf stage(stage_bytes);
        DevBuf raw(stage_bytes);
        for (size_t l = 0; l < c_.layers; l++) {
            uint8_t* b = arena_.as<uint8_t>() + l * a_.total;
            clear_layer(a_, b, s_);
            src.read_layer(l, stage.as<uint8_t>());
            HIPC(hipMemcpyAsync(raw.p, stage.p, L.total, hipMemcpyHostToDevice, s_));
            build_layer_device(c_, L, raw.as<uint8_t>(), a_, b, s_);
            HIPC(hipStreamSynchronize(s_));
            layers_.push_back(bind_layer(a_, b));
        }
        const Format ef = c_.embed_format;
        const int V = int(c_.vocab), h = int(c_.hidden);
        const TMat shape = tile_shape(ef.bits, ef.group, V, h, 256);
        edata_ = DevBuf(tile_data_bytes(shape));
        escales_ = DevBuf(std::max<size_t>(16, tile_scale_bytes(shape)));
        E_ = tile_bind(shape, edata_.as<uint8_t>(), escales_.as<uint16_t>());
        tile_clear(E_, s_);
        for (size_t first = 0; first < c_.vocab; first += HEAD_ROWS) {
            const size_t rows = std::min(HEAD_ROWS, c_.vocab - first);
            src.read_embed_rows(first, rows, stage.as<uint8_t>());
            HIPC(hipMemcpyAsync(raw.p, stage.p, rows * rb, hipMemcpyHostToDevice, s_));
            tile_repack(raw.as<uint8_t>(), int(rows), E_, int(first), int(rows), int(rows), s_);
            HIPC(hipStreamSynchronize(s_));
        }
    }
    const char* name() const override { return "resident"; }
    void begin_forward(bool) override {}
    const DevLayer& layer(size_t l) override {
        if (l >= layers_.size()) fail("layer " + std::to_string(l) + " out of range");
        return layers_[l];
    }
    void release_layer(size_t) override {}
    size_t n_head_chunks() const override { return 1; }
    HeadChunk head_chunk(size_t c) override {
        if (c != 0) fail("head chunk out of range");
        return HeadChunk{0, c_.vocab, E_};
    }
    void release_head_chunk(size_t) override {}
    void end_forward() override {}
    bool resident() const override { return true; }
    void embed(const uint32_t*, const uint32_t* dev_tokens, int t, float* x, const float* w, uint8_t* frags, float* ss,
               const StageMirror& mirror) override {
        tile_embed(E_, dev_tokens, t, x, w, frags, ss, s_, mirror);
    }
    ls_report report() const override {
        ls_report r{};
        r.resident_weight_bytes = arena_.n + edata_.n + escales_.n;
        r.bytes_read = src_.bytes_read();
        return r;
    }

private:
    const Source& src_;
    Config c_;
    LayerArena a_;
    hipStream_t s_;
    DevBuf arena_, edata_, escales_;
    std::vector<DevLayer> layers_;
    TMat E_;
};

// ---------------------------------------------------------------------------------------
// Streaming: `slots` device slots fed in schedule order (StreamProvider, src/provider.rs:161-352).
// A slot holds the raw block (copied host -> device on a copy stream), the arena it is
// rearranged into (on a build stream, so one item's rearrangement overlaps the next one's
// copy), and events: `copied` (its host staging buffer may be refilled), `ready` (the arena
// may be computed on and the raw buffer refilled) and `freed` (the compute stream is done with
// the arena). With a
// pinned source the copy goes straight from the source's memory; otherwise the host reads
// into a pinned staging buffer first.
// ---------------------------------------------------------------------------------------
class StreamProvider : public DeviceProvider {
    enum Kind { LAYER, HEAD };
    struct Item {
        Kind kind;
        size_t idx;
        bool operator==(const Item& o) const { return kind == o.kind && idx == o.idx; }
    };
    // A device slot: an item in the tile layout, as compute reads it.
    struct Slot {
        DevBuf arena, hdata, hscales;
        hipEvent_t ready = nullptr, freed = nullptr;
        bool used = false;
    };
    // A landing buffer for one item's bytes as the source holds them (reference layout). There is
    // one more than there are slots, so a copy never waits for the rearrangement of the item just
    // before it.
    struct Landing {
        DevBuf raw;
        PinnedBuf stage;
        hipEvent_t copied = nullptr, consumed = nullptr;
        bool used = false;
        uint64_t read_seq = 0;  // the read-ahead request that fills stage with the next item
    };
    // A read of one item's bytes into a landing buffer's pinned stage, by the I/O thread.
    struct Read {
        Item it;
        size_t landing;
        uint64_t seq;
    };

public:
    StreamProvider(const Source& src, int slots, size_t max_rows, hipStream_t compute)
        : src_(src), c_(src.cfg()), L_(src.layout()), a_(layer_arena(c_)), compute_(compute), max_rows_(max_rows) {
        if (slots < 1) slots = 1;
        HIPC(hipStreamCreateWithFlags(&copy_, hipStreamNonBlocking));
        HIPC(hipStreamCreateWithFlags(&build_, hipStreamNonBlocking));
        const size_t rb = c_.row_bytes();
        buf_size_ = std::max(L_.total, std::min(STREAM_HEAD_ROWS, c_.vocab) * rb);
        const Format ef = c_.embed_format;
        hshape_ = tile_shape(ef.bits, ef.group, int(STREAM_HEAD_ROWS), int(c_.hidden), 256);
        slots_.resize(size_t(slots));
        for (auto& s : slots_) {
            s.arena = DevBuf(a_.total);
            clear_layer(a_, s.arena.as<uint8_t>(), copy_);
            s.hdata = DevBuf(tile_data_bytes(hshape_));
            s.hscales = DevBuf(std::max<size_t>(16, tile_scale_bytes(hshape_)));
            tile_clear(tile_bind(hshape_, s.hdata.as<uint8_t>(), s.hscales.as<uint16_t>()), copy_);
            HIPC(hipEventCreateWithFlags(&s.ready, hipEventDisableTiming));
            HIPC(hipEventCreateWithFlags(&s.freed, hipEventDisableTiming));
        }
        landing_.resize(size_t(slots) + 1);
        for (auto& d : landing_) {
            d.raw = DevBuf(buf_size_);
            if (!src_.pinned()) d.stage = PinnedBuf(buf_size_);
            HIPC(hipEventCreateWithFlags(&d.copied, hipEventDisableTiming));
            HIPC(hipEventCreateWithFlags(&d.consumed, hipEventDisableTiming));
        }
        HIPC(hipStreamSynchronize(copy_));
        embed_stage_ = PinnedBuf(max_rows_ * rb);
        embed_raw_ = DevBuf(max_rows_ * rb);
        HIPC(hipEventCreateWithFlags(&embed_copied_, hipEventDisableTiming));
        // Bytes already in pinned memory: a pinned mirror of every item in the tile layout,
        // built once here, so that each pass copies straight into the slots (LS_STREAM_TILED=0:
        // copy the source's bytes and rearrange them on the device every pass).
        if (src_.pinned()) {
            tiled_on_ = true;
            if (const char* e = std::getenv("LS_STREAM_TILED")) tiled_on_ = std::atoi(e) != 0;
            if (tiled_on_) build_tiled();
        }
        // Bytes that are not already in pinned memory are read by an I/O thread, ahead of the
        // copies in schedule order (src/provider.rs:187-206, 288-305).
        if (!src_.pinned()) {
            HIPC(hipGetDevice(&device_));
            reader_ = std::thread([this] { read_loop(); });
        }
    }
    ~StreamProvider() override {
        if (reader_.joinable()) {
            {
                std::lock_guard<std::mutex> g(mu_);
                stop_ = true;
            }
            cv_.notify_all();
            reader_.join();
        }
        (void)hipStreamSynchronize(copy_);
        (void)hipStreamSynchronize(build_);
        (void)hipStreamSynchronize(compute_);
        for (auto& s : slots_) {
            (void)hipEventDestroy(s.ready);
            (void)hipEventDestroy(s.freed);
        }
        for (auto& d : landing_) {
            (void)hipEventDestroy(d.copied);
            (void)hipEventDestroy(d.consumed);
        }
        (void)hipEventDestroy(embed_copied_);
        (void)hipStreamDestroy(build_);
        (void)hipStreamDestroy(copy_);
    }
    const char* name() const override { return "stream"; }

    void begin_forward(bool with_head) override {
        // Items the previous pass issued ahead for this one (its first layers) are in flight;
        // otherwise (an earlier pass stopped early) wait for whatever copies are.
        if (!ahead_) {
            HIPC(hipStreamSynchronize(copy_));
            HIPC(hipStreamSynchronize(build_));
        }
        schedule_.clear();
        for (size_t l = 0; l < c_.layers; l++) schedule_.push_back({LAYER, l});
        if (with_head)
            for (size_t c = 0; c < n_head_chunks(); c++) schedule_.push_back({HEAD, c});
        next_issue_ = ahead_;
        next_take_ = 0;
        ahead_ = 0;
        holding_ = false;
        if (reader_.joinable()) {
            // Each pass reads its own items (as the reference counts them); reads a pass that did
            // not end normally requested finish first and are forgotten.
            {
                std::unique_lock<std::mutex> g(mu_);
                cv_.wait(g, [&] { return (reads_.empty() && done_seq_ == read_seq_) || !read_error_.empty(); });
            }
            next_read_ = 0;
            read_ahead();
        }
        while (next_issue_ < schedule_.size() && next_issue_ < slots_.size()) issue();
    }

    const DevLayer& layer(size_t l) override {
        Slot& s = take({LAYER, l});
        cur_layer_ = bind_layer(a_, s.arena.as<uint8_t>());
        return cur_layer_;
    }
    void release_layer(size_t) override { release(); }
    size_t n_head_chunks() const override { return (c_.vocab + STREAM_HEAD_ROWS - 1) / STREAM_HEAD_ROWS; }
    size_t head_rows(size_t c) const { return std::min(STREAM_HEAD_ROWS, c_.vocab - c * STREAM_HEAD_ROWS); }
    HeadChunk head_chunk(size_t c) override {
        Slot& s = take({HEAD, c});
        const size_t first = c * STREAM_HEAD_ROWS, rows = std::min(STREAM_HEAD_ROWS, c_.vocab - first);
        TMat m = tile_bind(hshape_, s.hdata.as<uint8_t>(), s.hscales.as<uint16_t>());
        m.rows = int(rows);
        return HeadChunk{first, rows, m};
    }
    void release_head_chunk(size_t) override { release(); }
    void end_forward() override {
        if (holding_) release();
        if (next_take_ != schedule_.size())
            fail("forward pass ended before every scheduled item was consumed", LS_E_STATE);
        // Every pass starts with the same layers, whatever it asks for: with the bytes already in
        // pinned host memory, their copies start now instead of after the host has seen this
        // pass's result. (Other sources read from storage, counted at the read: they wait.)
        if (src_.pinned()) {
            schedule_.clear();
            for (size_t l = 0; l < c_.layers && l < slots_.size(); l++) schedule_.push_back({LAYER, l});
            next_issue_ = 0;
            while (next_issue_ < schedule_.size()) issue();
            ahead_ = next_issue_;
        }
    }

    bool resident() const override { return false; }
    void embed(const uint32_t* host_tokens, const uint32_t*, int t, float* x, const float* w, uint8_t* frags, float* ss,
               const StageMirror& mirror) override {
        if (mirror.host) fail("a streamed table takes its tokens from the host call", LS_E_STATE);
        // Rows come from the source on every pass, as src/provider.rs:284-286.
        const size_t rb = c_.row_bytes();
        if (size_t(t) > max_rows_) fail("more embedding rows than the staging buffer holds", LS_E_STATE);
        HIPC(hipEventSynchronize(embed_copied_));
        for (int i = 0; i < t; i++) src_.read_embed_rows(host_tokens[i], 1, embed_stage_.as<uint8_t>() + size_t(i) * rb);
        HIPC(hipMemcpyAsync(embed_raw_.p, embed_stage_.p, size_t(t) * rb, hipMemcpyHostToDevice, compute_));
        HIPC(hipEventRecord(embed_copied_, compute_));
        embed_raw_rows(embed_raw_.as<uint8_t>(), c_.embed_format.bits, c_.embed_format.group, int(c_.hidden), t, x, compute_);
        if (frags) x_frags(x, t, int(c_.hidden), w, frags, ss, compute_);
    }

    ls_report report() const override {
        ls_report r{};
        for (auto& s : slots_) r.resident_weight_bytes += s.arena.n + s.hdata.n + s.hscales.n;
        for (auto& d : landing_) r.resident_weight_bytes += d.raw.n;
        r.bytes_read = src_.bytes_read();
        r.wait_ns = wait_ns_;
        r.h2d_bytes = h2d_bytes_;
        return r;
    }

private:
    size_t head_data_bytes() const { return tile_data_bytes(hshape_); }
    size_t head_scale_bytes() const { return std::max<size_t>(16, tile_scale_bytes(hshape_)); }
    size_t tiled_head_off() const { return c_.layers * a_.total; }

    // The pinned mirror: each layer's arena, then each head chunk's tile data and scales, made by
    // the same device rearrangement a pass would run (so the slots get the same bytes).
    void build_tiled() {
        const size_t hd = head_data_bytes(), hs = head_scale_bytes(), rb = c_.row_bytes();
        tiled_ = PinnedBuf(tiled_head_off() + n_head_chunks() * (hd + hs));
        Slot& s = slots_[0];
        Landing& d = landing_[0];
        uint8_t* dst = tiled_.as<uint8_t>();
        for (size_t l = 0; l < c_.layers; l++) {
            HIPC(hipMemcpyAsync(d.raw.p, src_.layer_view(l), L_.total, hipMemcpyHostToDevice, copy_));
            build_layer_device(c_, L_, d.raw.as<uint8_t>(), a_, s.arena.as<uint8_t>(), copy_);
            HIPC(hipMemcpyAsync(dst + l * a_.total, s.arena.p, a_.total, hipMemcpyDeviceToHost, copy_));
        }
        for (size_t c = 0; c < n_head_chunks(); c++) {
            const size_t first = c * STREAM_HEAD_ROWS, rows = head_rows(c);
            HIPC(hipMemcpyAsync(d.raw.p, src_.embed_view() + first * rb, rows * rb, hipMemcpyHostToDevice, copy_));
            TMat m = tile_bind(hshape_, s.hdata.as<uint8_t>(), s.hscales.as<uint16_t>());
            tile_repack(d.raw.as<uint8_t>(), int(rows), m, 0, int(rows), int(rows), copy_);
            uint8_t* at = dst + tiled_head_off() + c * (hd + hs);
            HIPC(hipMemcpyAsync(at, s.hdata.p, hd, hipMemcpyDeviceToHost, copy_));
            HIPC(hipMemcpyAsync(at + hd, s.hscales.p, hs, hipMemcpyDeviceToHost, copy_));
        }
        HIPC(hipStreamSynchronize(copy_));
    }

    void issue() {
        const Item it = schedule_[next_issue_];
        Slot& s = slots_[next_issue_ % slots_.size()];
        if (tiled_on_) {
            // Straight from the pinned mirror into the slot, once compute is done with it.
            if (s.used) HIPC(hipStreamWaitEvent(copy_, s.freed, 0));
            const uint8_t* mirror = tiled_.as<uint8_t>();
            if (it.kind == LAYER) {
                HIPC(hipMemcpyAsync(s.arena.p, mirror + it.idx * a_.total, a_.total, hipMemcpyHostToDevice, copy_));
                h2d_bytes_ += a_.total;
            } else {
                const size_t hd = head_data_bytes(), hs = head_scale_bytes();
                const uint8_t* at = mirror + tiled_head_off() + it.idx * (hd + hs);
                HIPC(hipMemcpyAsync(s.hdata.p, at, hd, hipMemcpyHostToDevice, copy_));
                HIPC(hipMemcpyAsync(s.hscales.p, at + hd, hs, hipMemcpyHostToDevice, copy_));
                h2d_bytes_ += hd + hs;
            }
            HIPC(hipEventRecord(s.ready, copy_));
            s.used = true;
            next_issue_++;
            return;
        }
        Landing& d = landing_[next_issue_ % landing_.size()];
        const size_t rb = c_.row_bytes();
        size_t bytes, first = 0, rows = 0;
        if (it.kind == LAYER) {
            bytes = L_.total;
        } else {
            first = it.idx * STREAM_HEAD_ROWS;
            rows = std::min(STREAM_HEAD_ROWS, c_.vocab - first);
            bytes = rows * rb;
        }
        const uint8_t* from;
        if (src_.pinned()) {
            from = it.kind == LAYER ? src_.layer_view(it.idx) : src_.embed_view() + first * rb;
        } else {
            // The I/O thread has this item's read (requested read-ahead items back); wait for it.
            read_ahead();
            auto t0 = std::chrono::steady_clock::now();
            {
                std::unique_lock<std::mutex> g(mu_);
                cv_.wait(g, [&] { return done_seq_ >= d.read_seq || !read_error_.empty(); });
                if (!read_error_.empty()) fail("streamed read failed: " + read_error_, LS_E_IO);
            }
            wait_ns_ += uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0).count());
            from = d.stage.as<uint8_t>();
        }
        // The landing buffer is free once the rearrangement of its previous item has read it
        // (slots + 1 items back); the slot's arena once the compute stream is done with its
        // previous item. The copy waits only for the former.
        if (d.used) HIPC(hipStreamWaitEvent(copy_, d.consumed, 0));
        HIPC(hipMemcpyAsync(d.raw.p, from, bytes, hipMemcpyHostToDevice, copy_));
        h2d_bytes_ += bytes;
        HIPC(hipEventRecord(d.copied, copy_));
        // The tile layout is built on a stream of its own, so the next item's PCIe copy runs
        // meanwhile.
        HIPC(hipStreamWaitEvent(build_, d.copied, 0));
        if (s.used) HIPC(hipStreamWaitEvent(build_, s.freed, 0));
        if (it.kind == LAYER) {
            build_layer_device(c_, L_, d.raw.as<uint8_t>(), a_, s.arena.as<uint8_t>(), build_);
        } else {
            TMat m = tile_bind(hshape_, s.hdata.as<uint8_t>(), s.hscales.as<uint16_t>());
            tile_repack(d.raw.as<uint8_t>(), int(rows), m, 0, int(rows), int(rows), build_);
        }
        HIPC(hipEventRecord(s.ready, build_));
        HIPC(hipEventRecord(d.consumed, build_));
        s.used = true;
        d.used = true;
        next_issue_++;
    }

    // Requests reads for the schedule's items up to one landing buffer per item ahead of the next
    // copy (a landing's stage is refilled once its previous copy has landed).
    void read_ahead() {
        bool any = false;
        {
            std::lock_guard<std::mutex> g(mu_);
            while (next_read_ < schedule_.size() && next_read_ < next_issue_ + landing_.size()) {
                Landing& d = landing_[next_read_ % landing_.size()];
                d.read_seq = ++read_seq_;
                reads_.push_back({schedule_[next_read_], next_read_ % landing_.size(), d.read_seq});
                next_read_++;
                any = true;
            }
        }
        if (any) cv_.notify_all();
    }

    void read_loop() {
        (void)hipSetDevice(device_);
        for (;;) {
            Read r;
            {
                std::unique_lock<std::mutex> g(mu_);
                cv_.wait(g, [&] { return stop_ || !reads_.empty(); });
                if (stop_) return;
                r = reads_.front();
                reads_.pop_front();
            }
            Landing& d = landing_[r.landing];
            std::string err;
            try {
                // the stage's previous copy has landed before it is overwritten
                if (hipEventSynchronize(d.copied) != hipSuccess) throw std::runtime_error("waiting for a staging copy failed");
                if (r.it.kind == LAYER) {
                    src_.read_layer(r.it.idx, d.stage.as<uint8_t>());
                } else {
                    const size_t first = r.it.idx * STREAM_HEAD_ROWS;
                    src_.read_embed_rows(first, std::min(STREAM_HEAD_ROWS, c_.vocab - first), d.stage.as<uint8_t>());
                }
            } catch (const std::exception& e) {
                err = e.what();
            }
            {
                std::lock_guard<std::mutex> g(mu_);
                if (!err.empty() && read_error_.empty()) read_error_ = err;
                done_seq_ = r.seq;
            }
            cv_.notify_all();
        }
    }

    Slot& take(const Item& want) {
        if (holding_) release();
        if (next_take_ >= schedule_.size() || !(schedule_[next_take_] == want))
            fail(std::string("provider asked for ") + (want.kind == LAYER ? "layer " : "head chunk ") + std::to_string(want.idx) +
                     " out of schedule order",
                 LS_E_STATE);
        Slot& s = slots_[next_take_ % slots_.size()];
        HIPC(hipStreamWaitEvent(compute_, s.ready, 0));
        // Pinned bytes are counted when the pass takes them (they may be copied a pass ahead).
        if (src_.pinned()) src_.count_read(want.kind == LAYER ? L_.total : head_rows(want.idx) * c_.row_bytes());
        holding_ = true;
        return s;
    }

    void release() {
        if (!holding_) return;
        Slot& s = slots_[next_take_ % slots_.size()];
        HIPC(hipEventRecord(s.freed, compute_));
        holding_ = false;
        next_take_++;
        while (next_issue_ < schedule_.size() && next_issue_ < next_take_ + slots_.size()) issue();
    }

    const Source& src_;
    Config c_;
    LayerLayout L_;
    LayerArena a_;
    TMat hshape_;
    hipStream_t compute_, copy_ = nullptr, build_ = nullptr;
    std::vector<Slot> slots_;
    std::vector<Landing> landing_;
    std::vector<Item> schedule_;
    size_t next_issue_ = 0, next_take_ = 0, buf_size_ = 0;
    size_t ahead_ = 0;  // items of the next pass issued at the end of the last one
    bool holding_ = false;
    DevLayer cur_layer_;
    size_t max_rows_;
    PinnedBuf embed_stage_;
    DevBuf embed_raw_;
    hipEvent_t embed_copied_ = nullptr;
    uint64_t wait_ns_ = 0, h2d_bytes_ = 0;
    bool tiled_on_ = false;  // copies from the pinned tile-layout mirror
    PinnedBuf tiled_;
    // the I/O thread (sources not in pinned memory)
    std::thread reader_;
    int device_ = 0;
    std::mutex mu_;
    std::condition_variable cv_;
    std::deque<Read> reads_;
    size_t next_read_ = 0;  // the next schedule item whose read is requested
    uint64_t read_seq_ = 0, done_seq_ = 0;
    bool stop_ = false;
    std::string read_error_;
};

std::unique_ptr<DeviceProvider> make_resident(const Source& src, hipStream_t s) {
    return std::make_unique<ResidentProvider>(src, s);
}
std::unique_ptr<DeviceProvider> make_stream(const Source& src, int slots, size_t max_rows, hipStream_t s) {
    return std::make_unique<StreamProvider>(src, slots, max_rows, s);
}

// ---------------------------------------------------------------------------------------
// Model
// ---------------------------------------------------------------------------------------
constexpr size_t PREFILL_CHUNK = 128;  // src/model.rs:14
constexpr size_t MAX_BLOCK = 33;       // a verify block: 1 + MAX_DRAFT (src/spec.rs:52) tokens
constexpr size_t MAX_CHAIN = 32;       // a draft chain: at most MAX_DRAFT passes
constexpr int MAX_SEQ = 1024;

Model::Model(const Source& src, int mode, int slots, size_t max_ctx, int device, int n_seq)
    : cfg_(src.cfg()), device_(device), max_ctx_(max_ctx), n_seq_(n_seq) {
    if (max_ctx == 0) fail("max_ctx must be positive");
    if (n_seq < 1 || n_seq > MAX_SEQ) fail("a model holds 1 to " + std::to_string(MAX_SEQ) + " sequences");
    if (size_t(n_seq) * max_ctx > size_t(INT32_MAX / 2)) fail("sequences x max_ctx is too large");
    seq_pos_.assign(size_t(n_seq), 0);
    // Launch rows: a prefill chunk, or one block of up to MAX_BLOCK tokens per sequence.
    rows_cap_ = (std::max(PREFILL_CHUNK, size_t(n_seq) * MAX_BLOCK) + FTOK - 1) / FTOK * FTOK;
    const Config& c = cfg_;
    if (c.inter % 64 != 0) fail("the intermediate size must be a multiple of 64");
    if (c.head_dim != 16 && c.head_dim != 32 && c.head_dim != 64 && c.head_dim != 128)
        fail("head_dim must be 16, 32, 64 or 128");
    HIPC(hipSetDevice(device));
    (void)device_cu_count();  // cached before any graph capture
    HIPC(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    HIPC(hipEventCreate(&ev0_));
    HIPC(hipEventCreate(&ev1_));
    if (mode == LS_MODE_RESIDENT) prov_ = make_resident(src, stream_);
    else if (mode == LS_MODE_STREAM) prov_ = make_stream(src, slots, rows_cap_, stream_);
    else fail("unknown mode " + std::to_string(mode) + " (use resident or stream)");

    const size_t h = c.hidden, kv = c.kv_dim(), in = c.inter, T = rows_cap_;
    const size_t tiles = T / FTOK, max_segs = tiles + size_t(n_seq);
    // K/V caches [layer][sequence][position][kv_dim].
    kcache_ = DevBuf(c.layers * n_seq * max_ctx * kv * 4);
    vcache_ = DevBuf(c.layers * n_seq * max_ctx * kv * 4);
    HIPC(hipMemsetAsync(kcache_.p, 0, kcache_.n, stream_));
    HIPC(hipMemsetAsync(vcache_.p, 0, vcache_.n, stream_));

    // RoPE table on the host with glibc, as the reference computes each angle (src/model.rs:63-65,
    // src/kernels.rs:246-247): inv_freq in f64 cast to f32, angle = (pos as f32) * inv_freq.
    const size_t half = c.head_dim / 2;
    std::vector<float> inv(half), cs(max_ctx * half), sn(max_ctx * half);
    for (size_t i = 0; i < half; i++)
        inv[i] = float(1.0 / std::pow(double(c.rope_theta), double(2 * i) / double(c.head_dim)));
    for (size_t p = 0; p < max_ctx; p++)
        for (size_t i = 0; i < half; i++) {
            float ang = float(p) * inv[i];
            cs[p * half + i] = cosf(ang);
            sn[p * half + i] = sinf(ang);
        }
    rope_cos_ = DevBuf(cs.size() * 4);
    rope_sin_ = DevBuf(sn.size() * 4);
    HIPC(hipMemcpy(rope_cos_.p, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    HIPC(hipMemcpy(rope_sin_.p, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    fnorm_ = DevBuf(h * 4);
    HIPC(hipMemcpy(fnorm_.p, src.final_norm().data(), h * 4, hipMemcpyHostToDevice));

    vpad_ = (c.vocab + 63) / 64 * 64;
    if (c.hidden % 8) fail("hidden size must be a multiple of 8");
    const size_t hq = c.heads * c.head_dim;
    fb_h_ = frag_tile_bytes(int(h));
    fb_q_ = frag_tile_bytes(int(hq));
    fb_in_ = frag_tile_bytes(int(in));
    slots_h_ = ss_slots(int(h));
    if (h > 4096) fail("hidden sizes above 4096 are not supported");
    if ((c.heads + c.kv_heads) * c.head_dim % 16) fail("q and k heads must fill whole 16-row strips");
    {
        const TMat e_res = tile_shape(c.embed_format.bits, c.embed_format.group, int(c.vocab), int(h), 256);
        const size_t n_chunks = (c.vocab + STREAM_HEAD_ROWS - 1) / STREAM_HEAD_ROWS;
        head_blocks_ = std::max(e_res.n_strips / 4, int(n_chunks * STREAM_HEAD_ROWS / 64));
    }
    // Wide rows (3B: 32 int8 chunks): 256-column K shares, so 8 wavefronts cover a row of 2048
    // with no split and every role of a layer fits the layer stack's 512-thread workgroups
    // (LS_WIDE=0: 128-column shares, 16 wavefronts; not for weights in groups of 16). The head has
    // its own plan.
    const bool g16w = c.format.bits != 16 && c.format.group == 16;
    if (c.hidden >= 2048) {
        wide_ = g16w ? 1 : 2;
        if (const char* e = std::getenv("LS_WIDE"); e && std::atoi(e) == 0) wide_ = 1;
        kw_qkv_ = kw_o_ = kw_gu_ = kw_down_ = wide_ == 2 ? 8 : 16;
        kw_head_ = 16;
        // Down in four strips per wavefront: half the workgroups of two (192 for 3B), each reading
        // its input fragments once for 64 rows; the layer stack's down stage measured 13 us
        // against 17 us. q|k|v and o stay at one strip per wavefront (four measured slower: 8.5
        // against 6.7 us, the products of a wavefront's four strips run one after another).
        if (wide_ == 2 && c.hidden % 64 == 0) ds_ = 4;
    }
    {
        // Launches over several token tiles (prefill chunks, batches): more rows per wavefront, so
        // each workgroup reads its tile's fragments once for more rows (q|k|v 4, o 2, down 4
        // strips: 16 sequences x 9 rows of the 0.5B int8 shape, 2.76 -> 2.47 ms per batched verify
        // step; a 512-token prefill, 8.60 -> 8.08 ms). Strips do
        // not change any sum, so every launch keeps the bits of the one-tile plans.
        const LayerArena la = layer_arena(c);
        mqs_ = la.qkv.n_strips % 4 == 0 ? 4 : qs_;
        mos_ = la.o.n_strips % 2 == 0 ? std::max(2, os_) : os_;
        mds_ = la.down.n_strips % 4 == 0 ? 4 : ds_;
    }
    if (const char* e = std::getenv("LS_MT_STRIPS")) {
        // Strips per wavefront of q|k|v, o and down in launches over several token tiles.
        int v[3];
        if (std::sscanf(e, "%d,%d,%d", &v[0], &v[1], &v[2]) != 3) fail("LS_MT_STRIPS needs three integers");
        for (int x : v)
            if (x != 1 && x != 2 && x != 4) fail("LS_MT_STRIPS values must be 1, 2 or 4");
        mqs_ = v[0];
        mos_ = v[1];
        mds_ = v[2];
    }
    plan_kw_from_env();
    if (const char* e = std::getenv("LS_FUSE")) fuse_on_ = std::atoi(e) != 0;  // fused launches (default on)
    if (const char* e = std::getenv("LS_FUSE_QKV")) fuse_qkv_ = std::atoi(e) != 0;
    if (const char* e = std::getenv("LS_PF")) pf_on_ = std::atoi(e) != 0;  // weight prefetch in fused launches (default on)
    if (const char* e = std::getenv("LS_STACK")) stack_on_ = std::atoi(e) != 0;  // layer-stack launch (default on)
    if (const char* e = std::getenv("LS_PIPE")) pipe_on_ = std::atoi(e) != 0;  // pipelined large gate|up (default on)
    if (const char* e = std::getenv("LS_DIRECT")) direct_on_ = std::atoi(e) != 0;  // verify staging without copies (default on)
    if (const char* e = std::getenv("LS_STEP_EVENTS")) step_events_ = std::atoi(e) != 0;  // device events around each step (default off)
    x_ = DevBuf(T * h * 4);
    q_ = DevBuf(T * hq * 4);
    // Fragment buffers start at zero: padding columns are never written and must stay finite.
    xf_ = DevBuf(fb_h_ * tiles);
    ss_ = DevBuf(tiles * slots_h_ * FTOK * 4);
    af_ = DevBuf(fb_q_ * tiles);
    actf_ = DevBuf(fb_in_ * tiles);
    HIPC(hipMemsetAsync(xf_.p, 0, xf_.n, stream_));
    HIPC(hipMemsetAsync(ss_.p, 0, ss_.n, stream_));
    HIPC(hipMemsetAsync(af_.p, 0, af_.n, stream_));
    HIPC(hipMemsetAsync(actf_.p, 0, actf_.n, stream_));
    {
        // Split-K scratch for the largest launch of each matrix (T rows).
        const LayerArena la = layer_arena(c);
        const TMat e_res = tile_shape(c.embed_format.bits, c.embed_format.group, int(c.vocab), int(h), 256);
        const int n = int(T);
        const TMat e_chunk = tile_shape(c.embed_format.bits, c.embed_format.group, int(STREAM_HEAD_ROWS), int(h), 256);
        const MMPlan plans[] = {mm_plan(la.qkv, 1, kw_qkv_, n, qs_, wide_),  mm_plan(la.o, 1, kw_o_, n, os_, wide_),
                                gu_plan(la.gu, kw_gu_, n, wide_), mm_plan(la.down, 1, kw_down_, n, ds_, wide_),
                                mm_plan(e_res, 1, kw_head_, n, 4),       mm_plan(e_chunk, 1, kw_head_, n, 4)};
        size_t pf = 0, nc = 0;
        for (const MMPlan& pl : plans) {
            pf = std::max(pf, mm_part_floats(pl));
            nc = std::max(nc, mm_counters(pl));
        }
        for (const MMPlan& pl : {mm_plan(la.qkv, 1, kw_qkv_, n, mqs_, wide_), mm_plan(la.o, 1, kw_o_, n, mos_, wide_),
                                 mm_plan(la.down, 1, kw_down_, n, mds_, wide_)}) {
            pf = std::max(pf, mm_part_floats(pl));
            nc = std::max(nc, mm_counters(pl));
        }
        part_ = DevBuf(std::max<size_t>(pf, 1) * 4);
        cnt_ = DevBuf(std::max<size_t>(nc, 1) * 4);
        HIPC(hipMemsetAsync(cnt_.p, 0, cnt_.n, stream_));
    }
    attn_scratch_ = DevBuf(attention_scratch_floats(int(T), int(c.heads), int(c.head_dim), int(max_ctx)) * 4);
    attn_cnt_ = DevBuf(max_segs * c.heads * 4);
    HIPC(hipMemsetAsync(attn_cnt_.p, 0, attn_cnt_.n, stream_));
    logits_ = DevBuf(PREFILL_CHUNK * vpad_ * 4);  // logits are returned for at most one chunk
    hpv_ = DevBuf(tiles * head_blocks_ * FTOK * 4);
    hpi_ = DevBuf(tiles * head_blocks_ * FTOK * 4);
    row0_ = DevBuf(T * 4);
    amax_ = DevBuf(T * 4);
    // Staging (ints): a call's chunk positions and tokens, or a batch's segments, rows and blocks.
    const size_t stage_words = std::max(max_ctx / PREFILL_CHUNK + 2 + max_ctx, 4 * max_segs + 3 * T + 2 * size_t(n_seq));
    stage_ = DevBuf(stage_words * 4);
    ctl_ = DevBuf(flow_words(int(c.layers)) * 4);
    HIPC(hipMemsetAsync(ctl_.p, 0, ctl_.n, stream_));
    bacc_ = DevBuf((1 + 2 * size_t(n_seq)) * 4);
    chain_out_ = DevBuf((MAX_CHAIN + 1) * 4);
    h_stage_ = PinnedBuf(stage_words * 4);
    h_out_ = PinnedBuf(PREFILL_CHUNK * 4);
    h_ctl_ = PinnedBuf(CTL_BACK * 4);
    h_bacc_ = PinnedBuf((1 + 2 * size_t(n_seq)) * 4);
    if (prov_->resident()) {
        // Layer pointers for the layer-stack launch; caches of sequence 0 (a selected sequence
        // adds its offset at launch).
        std::vector<LayerPtrs> lp(c.layers);
        for (size_t l = 0; l < c.layers; l++) {
            const DevLayer& L = prov_->layer(l);
            LayerPtrs& P = lp[l];
            P.qkv = L.qkv;
            P.o = L.o;
            P.gu = L.gu;
            P.down = L.down;
            P.b_qkv = L.b_qkv;
            P.post_norm = L.post_norm;
            P.next_norm = l + 1 < c.layers ? prov_->layer(l + 1).in_norm : fnorm_.as<float>();
            P.kc = kcache_.as<float>() + l * size_t(n_seq) * max_ctx * kv;
            P.vc = vcache_.as<float>() + l * size_t(n_seq) * max_ctx * kv;
        }
        layer_ptrs_ = DevBuf(lp.size() * sizeof(LayerPtrs));
        HIPC(hipMemcpyAsync(layer_ptrs_.p, lp.data(), layer_ptrs_.n, hipMemcpyHostToDevice, stream_));
        // The persistent pass, when its plans fit (the plans of a one-tile pass do not depend on
        // its token count).
        const DevLayer& L0 = prov_->layer(0);
        const MMPlan pq = mm_plan(L0.qkv, 1, kw_qkv_, 1, qs_, wide_), po = mm_plan(L0.o, 1, kw_o_, 1, os_, wide_);
        const MMPlan pg = gu_plan(L0.gu, kw_gu_, 1, wide_), pd = mm_plan(L0.down, 1, kw_down_, 1, ds_, wide_);
        if (const char* e = std::getenv("LS_STACK_TIMELINE"); e && std::atoi(e) != 0 && !layer_stack_unfit(1, int(c.heads), int(c.kv_heads), int(c.head_dim), pq, po, pg, pd)) {
            // Per-workgroup stamps of the layer stack (entry, input there, done), for profiling.
            stack_tl_ = DevBuf(size_t(c.layers) * layer_stack_workgroups(int(c.heads), pq, po, pg, pd) * 8 * 8);
            HIPC(hipMemsetAsync(stack_tl_.p, 0, stack_tl_.n, stream_));
        }
        if (const char* e = std::getenv("LS_PASS")) pass_on_ = std::atoi(e) != 0;  // persistent pass (default off)
        if (pass_on_ && !layer_pass_unfit(1, int(c.heads), int(c.kv_heads), int(c.head_dim), pq, po, pg, pd) && c.layers < 64) {
            int repl = 1;  // copies of the exchange buffers that many units read at once (LS_PASS_COPIES)
            if (const char* e = std::getenv("LS_PASS_COPIES")) repl = std::atoi(e);
            pass_shape_ = pass_area_shape(int(c.hidden), int(c.heads), int(c.kv_heads), int(c.head_dim), int(c.inter), pd, repl);
            pass_area_ = DevBuf(2 * pass_shape_.set_bytes);
            pass_flags_ = DevBuf(pass_shape_.flag_bytes);
            epoch_ = DevBuf(256);
            HIPC(hipMemsetAsync(pass_area_.p, 0, pass_area_.n, stream_));
            HIPC(hipMemsetAsync(pass_flags_.p, 0, pass_flags_.n, stream_));
            HIPC(hipMemsetAsync(epoch_.p, 0, epoch_.n, stream_));
            if (const char* e = std::getenv("LS_PASS_TIMELINE"); e && std::atoi(e) != 0) {
                pass_tl_ = DevBuf(pass_timeline_words(int(c.layers)) * 8);
                HIPC(hipMemsetAsync(pass_tl_.p, 0, pass_tl_.n, stream_));
            }
        } else {
            pass_on_ = false;
        }
    }
    HIPC(hipStreamSynchronize(stream_));
}

Model::~Model() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (auto& kv : graphs_) (void)hipGraphExecDestroy(kv.second);
    for (auto& kv : batch_graphs_) (void)hipGraphExecDestroy(kv.second);
    for (auto& kv : chain_graphs_) (void)hipGraphExecDestroy(kv.second);
    for (hipEvent_t e : prof_ev_) (void)hipEventDestroy(e);
    prov_.reset();
    if (ev0_) (void)hipEventDestroy(ev0_);
    if (ev1_) (void)hipEventDestroy(ev1_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

void Model::select(int seq) {
    if (seq < 0 || seq >= n_seq_) fail("sequence " + std::to_string(seq) + " is not in [0, " + std::to_string(n_seq_) + ")");
    seq_pos_[size_t(cur_)] = pos_;
    cur_ = seq;
    pos_ = seq_pos_[size_t(seq)];
}

void Model::truncate(size_t pos) {
    if (pos > pos_) fail("cannot truncate to " + std::to_string(pos) + ": only " + std::to_string(pos_) + " tokens are cached");
    pos_ = pos;
}

void Model::check_request(const uint32_t* tok, size_t n) const {
    if (n == 0) fail("no tokens to process");
    if (!tok) fail("no token buffer");
    if (pos_ + n > max_ctx_)
        fail("context is full: " + std::to_string(pos_) + " cached + " + std::to_string(n) + " new tokens exceeds the limit of " +
             std::to_string(max_ctx_));
    for (size_t i = 0; i < n; i++)
        if (tok[i] >= cfg_.vocab) fail("token id " + std::to_string(tok[i]) + " is outside the vocabulary");
}

// ---- profiling of the weight-streaming kernels ------------------------------------------
// The next matrix launch records its own start and end (no marker packets in between).
void Model::prof_begin() {
    if (!prof_ || prof_skip_) return;
    while (prof_ev_.size() < prof_used_ + 2) {
        hipEvent_t e;
        HIPC(hipEventCreate(&e));
        prof_ev_.push_back(e);
    }
    mm_time_next_launch(prof_ev_[prof_used_], prof_ev_[prof_used_ + 1]);
}

void Model::prof_end(const TMat& W, int nt, bool launch, double extra_bytes) {
    if (!prof_ || prof_skip_) return;
    const Format f{W.bits, W.group};
    if (launch) {
        prof_used_ += 2;
        prof_acc_.launches++;
    }
    prof_acc_.bytes += double(W.rows) * double(f.row_bytes(size_t(W.cols))) + 4.0 * nt * (double(W.cols) + double(W.rows)) + extra_bytes;
    prof_acc_.flops += 2.0 * nt * double(W.rows) * double(W.cols);
}

void Model::harvest() {
    for (size_t i = 0; i + 1 < prof_used_; i += 2) {
        float ms = 0;
        HIPC(hipEventElapsedTime(&ms, prof_ev_[i], prof_ev_[i + 1]));
        prof_acc_.ms += ms;
    }
    prof_used_ = 0;
}

void Model::set_graphs(bool on) {
    HIPC(hipStreamSynchronize(stream_));
    graphs_on_ = on;
}

void Model::set_profiling(int on) {
    HIPC(hipStreamSynchronize(stream_));
    harvest();
    prof_ = on;
    prof_acc_ = ls_kernel_stat{};
}

ls_kernel_stat Model::read_profile() {
    HIPC(hipStreamSynchronize(stream_));
    harvest();
    ls_kernel_stat r = prof_acc_;
    prof_acc_ = ls_kernel_stat{};
    return r;
}

// Workgroup shapes along K can be overridden for tuning: LS_MM_KW="qkv,o,gate_up,down,head".
void Model::plan_kw_from_env() {
    const char* e = std::getenv("LS_MM_KW");
    if (!e || !*e) return;
    int v[5];
    if (std::sscanf(e, "%d,%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3], &v[4]) != 5) fail("LS_MM_KW needs five integers");
    for (int x : v)
        if (x < 1 || x > 16) fail("LS_MM_KW values must be between 1 and 16");
    kw_qkv_ = v[0];
    kw_o_ = v[1];
    kw_gu_ = v[2];
    kw_down_ = v[3];
    kw_head_ = v[4];
}

// Copy a call's tokens (and the position of each 128-token chunk) to the device once. The
// pinned staging buffers are only rewritten by the next call, after this call has drained.
//
// Staging layout, host (pinned) and device alike: [position of each 128-token chunk][tokens],
// moved by one copy.
const uint32_t* Model::stage_tokens(const uint32_t* tok, size_t n) {
    const size_t chunks = (n + PREFILL_CHUNK - 1) / PREFILL_CHUNK;
    int* hp = h_stage_.as<int>();
    for (size_t ci = 0; ci < chunks; ci++) hp[ci] = int(pos_ + ci * PREFILL_CHUNK);
    std::memcpy(hp + chunks, tok, n * 4);
    HIPC(hipMemcpyAsync(stage_.p, h_stage_.p, (chunks + n) * 4, hipMemcpyHostToDevice, stream_));
    stage_pos_ = stage_.as<int>();
    return reinterpret_cast<const uint32_t*>(stage_.as<int>() + chunks);
}

// forward_chunk (src/model.rs:161-220), all on the compute stream.
void Model::forward_chunk(const uint32_t* tok, const uint32_t* dtok, size_t t, size_t n_logits, bool want_logits,
                          const uint32_t* accept_block, const BatchView* bv) {
    const Config& c = cfg_;
    const int h = int(c.hidden), kv = int(c.kv_dim()), T = int(t);
    const int heads = int(c.heads), kvh = int(c.kv_heads), hd = int(c.head_dim);
    const int hq = heads * hd;
    hipStream_t s = stream_;
    float* x = x_.as<float>();
    float* ss = ss_.as<float>();
    uint8_t* xf = xf_.as<uint8_t>();
    const int* pos_dev = stage_pos_ + chunk_index_;  // this chunk's first position
    const MMScratch scr{part_.as<float>(), cnt_.as<int>()};
    const bool res = prov_->resident();
    prov_->begin_forward(n_logits > 0);
    // Resident layers: the embedding kernel and every down epilogue write the fragments of the
    // next layer's input directly. Streamed layers: each layer's fragments are made once it has
    // arrived.
    const DevLayer* L0 = res ? &prov_->layer(0) : nullptr;
    // A one-tile pass over resident layers runs as the persistent pass (its epoch moves first).
    const bool use_pass = res && !bv && stack_on_ && fuse_on_ && layer_ptrs_.p && pass_on_ && T <= int(FTOK);
    StageMirror em = mirror_;
    if (use_pass) em.epoch = epoch_.as<int>();
    prov_->embed(tok, dtok, T, x, L0 ? L0->in_norm : nullptr, L0 ? xf : nullptr, L0 ? ss : nullptr, em);
    bool stacked = false;
    prof_skip_ = false;
    if (res && !bv && stack_on_ && fuse_on_ && layer_ptrs_.p) {
        // One launch for every layer: the same plans (so the same bits) as the per-layer
        // launches below.
        const MMPlan pq = mm_plan(L0->qkv, 1, kw_qkv_, T, qs_, wide_), po = mm_plan(L0->o, 1, kw_o_, T, os_, wide_);
        const MMPlan pg = gu_plan(L0->gu, kw_gu_, T, wide_), pd = mm_plan(L0->down, 1, kw_down_, T, ds_, wide_);
        if (!layer_stack_unfit(T, heads, kvh, hd, pq, po, pg, pd)) {
            MMArgs qa;
            qa.W = L0->qkv;
            qa.frags = xf;
            qa.frag_stride = fb_h_;
            qa.ss = ss;
            qa.ss_slots = slots_h_;
            qa.eps = c.eps;
            qa.n = T;
            qa.out = q_.as<float>();
            qa.ldo = hq;
            qa.rope_cos = rope_cos_.as<float>();
            qa.rope_sin = rope_sin_.as<float>();
            qa.pos0 = pos_dev;
            qa.heads = heads;
            qa.kv_heads = kvh;
            qa.hd = hd;
            MMArgs oa;
            oa.W = L0->o;
            oa.frags = af_.as<uint8_t>();
            oa.frag_stride = fb_q_;
            oa.n = T;
            oa.out = x;
            oa.ldo = h;
            oa.ofrags = xf;
            oa.ofrag_stride = fb_h_;
            oa.oss = ss;
            oa.oss_slots = slots_h_;
            MMArgs ga;
            ga.W = L0->gu;
            ga.frags = xf;
            ga.frag_stride = fb_h_;
            ga.ss = ss;
            ga.ss_slots = slots_h_;
            ga.eps = c.eps;
            ga.n = T;
            ga.ofrags = actf_.as<uint8_t>();
            ga.ofrag_stride = fb_in_;
            MMArgs da;
            da.W = L0->down;
            da.frags = actf_.as<uint8_t>();
            da.frag_stride = fb_in_;
            da.n = T;
            da.out = x;
            da.ldo = h;
            da.ofrags = xf;
            da.ofrag_stride = fb_h_;
            da.oss = ss;
            da.oss_slots = slots_h_;
            prof_begin();
            if (use_pass) {
                const PassArea area = pass_area_bind(pass_shape_, pass_area_.as<uint8_t>(), pass_flags_.as<int>());
                layer_pass(layer_ptrs_.as<LayerPtrs>(), int(c.layers), size_t(cur_) * max_ctx_ * kv, qa, pq, oa, po, ga, pg, da, pd, area,
                           ctl_.as<int>(), epoch_.as<int>(), pass_tl_.p ? pass_tl_.as<uint64_t>() : nullptr, s);
            } else {
                layer_stack(layer_ptrs_.as<LayerPtrs>(), int(c.layers), size_t(cur_) * max_ctx_ * kv, qa, pq, attn_scratch_.as<float>(),
                            attn_cnt_.as<int>(), af_.as<uint8_t>(), oa, po, ga, pg, da, pd, scr, ctl_.as<int>(), s,
                            stack_tl_.p ? stack_tl_.as<unsigned long long>() : nullptr);
            }
            for (size_t l = 0; l < c.layers; l++) {
                const DevLayer& L = prov_->layer(l);
                prof_end(L.qkv, T, l == 0);
                prof_end(L.o, T, false, 2.0 * kv * 4 * double(pos_ + T));  // + the K/V rows attention reads
                prof_end(L.gu, T, false);
                prof_end(L.down, T, false);
                prov_->release_layer(l);
            }
            stacked = true;
        }
    }
    // The dominant launch of a stacked pass is the stack itself.
    prof_skip_ = stacked && prof_ == 2;
    for (size_t l = 0; !stacked && l < c.layers; l++) {
        const DevLayer& L = prov_->layer(l);
        // This layer's caches: every sequence's for a batch, else the selected one's.
        const size_t cache_off = (l * size_t(n_seq_) + (bv ? 0 : size_t(cur_))) * max_ctx_ * kv;
        float* kc = kcache_.as<float>() + cache_off;
        float* vc = vcache_.as<float>() + cache_off;
        if (!res) x_frags(x, T, h, L.in_norm, xf, ss, s);
        MMArgs qa;
        {
            MMArgs& a = qa;
            a.W = L.qkv;
            a.frags = xf;
            a.frag_stride = fb_h_;
            a.ss = ss;
            a.ss_slots = slots_h_;
            a.eps = c.eps;
            a.n = T;
            a.bias = L.b_qkv;
            a.out = q_.as<float>();
            a.ldo = hq;
            a.kcache = kc;
            a.vcache = vc;
            a.rope_cos = rope_cos_.as<float>();
            a.rope_sin = rope_sin_.as<float>();
            a.pos0 = pos_dev;
            if (bv) {
                a.row_pos = bv->pos;
                a.row_seq = bv->seq;
                a.seq_stride = max_ctx_;
            }
            a.heads = heads;
            a.kv_heads = kvh;
            a.hd = hd;
        }
        const bool mt = T > int(FTOK);  // several token tiles: the multi-tile strips (same bits)
        const MMPlan pq = mm_plan(L.qkv, 1, kw_qkv_, T, mt ? mqs_ : qs_, wide_);
        {
            MMArgs a;
            a.W = L.o;
            a.frags = af_.as<uint8_t>();
            a.frag_stride = fb_q_;
            a.n = T;
            a.out = x;
            a.ldo = h;
            a.ofrags = xf;
            a.ofrag_stride = fb_h_;
            a.onorm = L.post_norm;
            a.oss = ss;
            a.oss_slots = slots_h_;
            const MMPlan po = mm_plan(L.o, 1, kw_o_, T, mt ? mos_ : os_, wide_);
            // One launch for attention and o when the o workgroups can fetch their weights while
            // attention runs (one token tile, every workgroup resident at once); q|k|v joins it
            // when it runs as one workgroup per strip, and attention then fetches the cached
            // keys and values while q|k|v runs.
            const bool fuse_ao = fuse_on_ && !bv && po.tiles == 1 && po.nsplit == 1 && po.wide == 1 && 64 * po.rg * po.kw <= 512 &&
                                 attention_o_workgroups(heads, po) <= device_cu_count();
            const bool fuse_qao = fuse_ao && fuse_qkv_ && pq.s == 1 && pq.rg == 1 && pq.nsplit == 1 && pq.wide == 1 && 64 * pq.kw <= 512 &&
                                  heads <= FLOW_ATTN_O && qkv_attention_o_workgroups(heads, pq, po) <= device_cu_count();
            if (pf_on_) {
                // While waiting for attention, the o workgroups read this layer's gate|up and
                // down weights once, so that their launch finds them in the memory-side cache.
                const uint8_t* end = L.down.scales ? reinterpret_cast<const uint8_t*>(L.down.scales) + tile_scale_bytes(L.down)
                                                   : L.down.data + tile_data_bytes(L.down);
                a.pf = L.gu.data;
                a.pf_bytes = size_t(end - L.gu.data);
            }
            if (fuse_qao) {
                prof_begin();
                qkv_attention_o(qa, pq, attn_scratch_.as<float>(), attn_cnt_.as<int>(), af_.as<uint8_t>(), a, po, scr, ctl_.as<int>(), s);
                prof_end(L.qkv, T);
                prof_end(L.o, T, false, 2.0 * kv * 4 * double(pos_ + T));  // + the K/V rows attention reads
            } else if (fuse_ao) {
                prof_begin();
                mm_qkv(qa, pq, scr, s);
                prof_end(L.qkv, T);
                prof_begin();
                attention_o(q_.as<float>(), hq, T, heads, kvh, hd, pos_dev, kc, vc, attn_scratch_.as<float>(), attn_cnt_.as<int>(),
                            af_.as<uint8_t>(), a, po, scr, ctl_.as<int>(), s);
                prof_end(L.o, T, true, 2.0 * kv * 4 * double(pos_ + T));  // + the K/V rows attention reads
            } else {
                prof_begin();
                mm_qkv(qa, pq, scr, s);
                prof_end(L.qkv, T);
                attention(q_.as<float>(), hq, T, heads, kvh, hd, pos_dev, bv ? bv->attn : AttnRows{}, kc, vc, attn_scratch_.as<float>(),
                          attn_cnt_.as<int>(), af_.as<uint8_t>(), s);
                prof_begin();
                mm_residual(a, po, scr, s);
                prof_end(L.o, T);
            }
        }
        {
            MMArgs g;
            g.W = L.gu;
            g.frags = xf;
            g.frag_stride = fb_h_;
            g.ss = ss;
            g.ss_slots = slots_h_;
            g.eps = c.eps;
            g.n = T;
            g.ofrags = actf_.as<uint8_t>();
            g.ofrag_stride = fb_in_;
            const bool last = l + 1 == c.layers;
            MMArgs d;
            d.W = L.down;
            d.frags = actf_.as<uint8_t>();
            d.frag_stride = fb_in_;
            d.n = T;
            d.out = x;
            d.ldo = h;
            if (last || res) {
                d.ofrags = xf;
                d.ofrag_stride = fb_h_;
                d.onorm = last ? fnorm_.as<float>() : prov_->layer(l + 1).in_norm;
                d.oss = ss;
                d.oss_slots = slots_h_;
            }
            if (pf_on_ && res && !last) {
                // While waiting for gate|up, the down workgroups read the next layer's q|k|v and
                // o weights once (resident layers: already in place).
                const DevLayer& N = prov_->layer(l + 1);
                const uint8_t* end = N.o.scales ? reinterpret_cast<const uint8_t*>(N.o.scales) + tile_scale_bytes(N.o)
                                                : N.o.data + tile_data_bytes(N.o);
                d.pf = N.qkv.data;
                d.pf_bytes = size_t(end - N.qkv.data);
            }
            const MMPlan pg = gu_plan(L.gu, kw_gu_, T, wide_), pd = mm_plan(L.down, 1, kw_down_, T, mt ? mds_ : ds_, wide_);
            // Fused only when both roles fit on the device at one workgroup per CU (their
            // wavefronts fill a CU's register file): a down workgroup that started after a
            // gate|up one had finished would fetch its weights late. Either path gives the same
            // bits (same plans).
            if (fuse_on_ && pg.tiles == 1 && pg.nsplit == 1 && pg.wide == 1 && pg.nrb + pd.nrb * pd.nsplit <= device_cu_count()) {
                // One launch: the down workgroups fetch their weights while gate|up runs.
                prof_begin();
                mm_gate_up_down(g, pg, d, pd, scr, ctl_.as<int>(), s);
                prof_end(L.gu, T);
                prof_end(L.down, T, false);
            } else {
                // gate|up with more strip pairs than CUs: the pipelined launch (same bits).
                prof_begin();
                if (pipe_on_ && mm_gate_up_pipe_fits(g, pg) && pg.nrb * GU_STRIPS > device_cu_count()) mm_gate_up_pipe(g, pg, s);
                else mm_gate_up(g, pg, scr, s);
                prof_end(L.gu, T);
                prof_begin();
                mm_residual(d, pd, scr, s);
                prof_end(L.down, T);
            }
        }
        prov_->release_layer(l);
    }
    if (n_logits > 0) {
        // Head (src/model.rs:190-216) over the token tiles holding the last n rows: the tied table
        // (one chunk when resident), per-block argmax partials, then the argmax. The final norm
        // was applied by the last layer's epilogue (fragments of x * w, 1 / rms here).
        const int t0 = (T - int(n_logits)) / FTOK, nh = T - FTOK * t0;
        head_off_ = size_t(T) - n_logits - size_t(FTOK) * t0;
        int blocks = 0;  // argmax partials written by this pass
        bool fused_final = false;
        for (size_t ci = 0; ci < prov_->n_head_chunks(); ci++) {
            HeadChunk hc = prov_->head_chunk(ci);
            MMArgs a;
            a.W = hc.mat;
            a.frags = xf + size_t(t0) * fb_h_;
            a.frag_stride = fb_h_;
            a.ss = ss + size_t(t0) * slots_h_ * FTOK;
            a.ss_slots = slots_h_;
            a.eps = c.eps;
            a.n = nh;
            a.out = want_logits ? logits_.as<float>() : nullptr;
            a.ldo = int(vpad_);
            a.arg_val = hpv_.as<float>();
            a.arg_idx = hpi_.as<int>();
            a.arg_stride = head_blocks_;
            a.arg_off = blocks;
            a.row_base = int(hc.first);
            a.row0 = hc.first == 0 ? row0_.as<float>() : nullptr;
            const MMPlan plan = mm_plan(hc.mat, 1, kw_head_, nh, 4);
            if (a.arg_off + plan.nrb > head_blocks_) fail("head blocks exceed the argmax buffer", LS_E_STATE);
            if (fin_host_ && accept_block && prov_->n_head_chunks() == 1) {
                // A verify block: the head's last workgroup finishes the argmax and the acceptance.
                a.fin_cnt = ctl_.as<int>() + FLOW_FIN;
                a.fin_ctl = ctl_.as<int>();
                a.fin_block = accept_block;
                a.fin_amax = amax_.as<uint32_t>();
                a.fin_host = fin_host_;
                fused_final = true;
            }
            prof_begin();
            blocks += mm_head(a, plan, scr, s);
            prof_end(hc.mat, nh);
            prov_->release_head_chunk(ci);
        }
        if (!fused_final)
            head_argmax_final(hpv_.as<float>(), hpi_.as<int>(), head_blocks_, blocks, row0_.as<float>(), nh, amax_.as<uint32_t>(),
                              accept_block, reinterpret_cast<uint32_t*>(ctl_.as<int>() + FLOW_ACC), s);

    }
    prof_skip_ = false;
    prov_->end_forward();
    if (!bv) pos_ += t;
}

void Model::forward(const uint32_t* tok, size_t n, float* logits, uint32_t* argmax) {
    HIPC(hipSetDevice(device_));
    check_request(tok, n);
    const size_t p0 = pos_;
    arm_failure();
    const uint32_t* dtok = stage_tokens(tok, n);
    const size_t n_chunks = (n + PREFILL_CHUNK - 1) / PREFILL_CHUNK;
    for (size_t ci = 0; ci < n_chunks; ci++) {
        const size_t a = ci * PREFILL_CHUNK, len = std::min(PREFILL_CHUNK, n - a);
        chunk_index_ = ci;
        forward_chunk(tok + a, dtok + a, len, ci + 1 == n_chunks ? 1 : 0, logits != nullptr);
    }
    chunk_index_ = 0;
    if (logits)
        HIPC(hipMemcpyAsync(logits, logits_.as<float>() + head_off_ * vpad_, cfg_.vocab * 4, hipMemcpyDeviceToHost, stream_));
    if (argmax) HIPC(hipMemcpyAsync(h_out_.p, amax_.as<uint32_t>() + head_off_, 4, hipMemcpyDeviceToHost, stream_));
    HIPC(hipMemcpyAsync(h_ctl_.p, ctl_.p, 4, hipMemcpyDeviceToHost, stream_));
    HIPC(hipStreamSynchronize(stream_));
    harvest();
    if (h_ctl_.as<int>()[FLOW_ERR]) pos_ = p0;  // a failed pass caches nothing
    check_flow(h_ctl_.as<int>());
    if (argmax) *argmax = h_out_.as<uint32_t>()[0];
}

void Model::forward_multi(const uint32_t* tok, size_t n, size_t n_logits, float* logits, uint32_t* argmax) {
    HIPC(hipSetDevice(device_));
    check_request(tok, n);
    if (n_logits == 0 || n_logits > n)
        fail("asked for logits at " + std::to_string(n_logits) + " positions of " + std::to_string(n) + " tokens");
    if (n > PREFILL_CHUNK) fail("forward_multi takes at most 128 tokens at a time");
    chunk_index_ = 0;
    const size_t p0 = pos_;
    arm_failure();
    forward_chunk(tok, stage_tokens(tok, n), n, n_logits, logits != nullptr);
    if (logits)
        HIPC(hipMemcpy2DAsync(logits, cfg_.vocab * 4, logits_.as<float>() + head_off_ * vpad_, vpad_ * 4, cfg_.vocab * 4,
                              n_logits, hipMemcpyDeviceToHost, stream_));
    if (argmax)
        HIPC(hipMemcpyAsync(h_out_.p, amax_.as<uint32_t>() + head_off_, n_logits * 4, hipMemcpyDeviceToHost, stream_));
    HIPC(hipMemcpyAsync(h_ctl_.p, ctl_.p, 4, hipMemcpyDeviceToHost, stream_));
    HIPC(hipStreamSynchronize(stream_));
    harvest();
    if (h_ctl_.as<int>()[FLOW_ERR]) pos_ = p0;  // a failed pass caches nothing
    check_flow(h_ctl_.as<int>());
    if (argmax) std::memcpy(argmax, h_out_.p, n_logits * 4);
}

void Model::verify_body(const uint32_t* block, size_t n) {
    // Over resident weights the embedding kernel reads the staged words from pinned host memory
    // (and mirrors them to the device for the later kernels) and the head writes the result back
    // there itself: no copy either way.
    const bool direct = direct_on_ && prov_->resident();
    struct Reset {
        Model* m;
        ~Reset() {
            m->mirror_ = StageMirror{};
            m->fin_host_ = nullptr;
        }
    } reset{this};
    if (direct) {
        mirror_ = StageMirror{h_stage_.as<int>(), stage_.as<int>(), int(n + 1), 1};
        fin_host_ = h_ctl_.as<uint32_t>();
    } else {
        HIPC(hipMemcpyAsync(stage_.p, h_stage_.p, (n + 1) * 4, hipMemcpyHostToDevice, stream_));
    }
    stage_pos_ = stage_.as<int>();
    const uint32_t* dtok = reinterpret_cast<const uint32_t*>(stage_.as<int>() + 1);
    forward_chunk(block, dtok, n, n, false, dtok);
    if (!direct) HIPC(hipMemcpyAsync(h_ctl_.p, ctl_.p, CTL_BACK * 4, hipMemcpyDeviceToHost, stream_));
}

size_t Model::debug_timeline(uint64_t* out, size_t cap) {
    const DevBuf& t = pass_tl_.p ? pass_tl_ : stack_tl_;
    if (!t.p) return 0;
    HIPC(hipStreamSynchronize(stream_));
    const size_t words = t.n / 8;
    if (out && cap) HIPC(hipMemcpy(out, t.p, std::min(cap, words) * 8, hipMemcpyDeviceToHost));
    return words;
}

size_t Model::debug_read(const char* name, void* out, size_t cap) {
    const std::string n(name ? name : "");
    const DevBuf* b = n == "x" ? &x_ : n == "xf" ? &xf_ : n == "ss" ? &ss_ : n == "q" ? &q_ : n == "af" ? &af_ : n == "actf" ? &actf_
                    : n == "kcache" ? &kcache_ : n == "vcache" ? &vcache_ : n == "pass_area" ? &pass_area_ : nullptr;
    if (!b) fail("no device buffer named '" + n + "'");
    HIPC(hipStreamSynchronize(stream_));
    if (out && cap && b->p) HIPC(hipMemcpy(out, b->p, std::min(cap, b->n), hipMemcpyDeviceToHost));
    return b->n;
}

void Model::arm_failure() {
    if (!fail_next_) return;
    fail_next_ = false;
    HIPC(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(ctl_.as<int>() + FLOW_ERR), 1, 1, stream_));
}

// A fused launch whose wait gave up (it never does unless a producer workgroup could not run)
// leaves garbage behind: report it and clear the control block for the next call.
void Model::check_flow(const int* ctl) {
    if (ctl[FLOW_ERR] == 0) return;
    // Every counter a failed launch may have left off zero: flows, split-K, attention merges.
    HIPC(hipMemsetAsync(ctl_.p, 0, ctl_.n, stream_));
    if (cnt_.p) HIPC(hipMemsetAsync(cnt_.p, 0, cnt_.n, stream_));
    if (attn_cnt_.p) HIPC(hipMemsetAsync(attn_cnt_.p, 0, attn_cnt_.n, stream_));
    HIPC(hipStreamSynchronize(stream_));
    fail("a fused launch timed out waiting for its producers; the results of this call are invalid", LS_E_DEVICE);
}

void Model::verify_greedy(const uint32_t* block, size_t n, uint32_t* m, uint32_t* next) {
    HIPC(hipSetDevice(device_));
    check_request(block, n);
    if (n > PREFILL_CHUNK) fail("a verify block takes at most 128 tokens");
    const size_t p = pos_;
    const std::pair<int, size_t> key(cur_, n);
    chunk_index_ = 0;
    // Host staging ([position][tokens], one chunk); the previous call has drained, so the
    // pinned buffer is free.
    h_stage_.as<int>()[0] = int(p);
    std::memcpy(h_stage_.as<int>() + 1, block, n * 4);
    arm_failure();
    const auto host0 = std::chrono::steady_clock::now();
    if (step_events_) HIPC(hipEventRecord(ev0_, stream_));
    if (graphs_on_ && !prof_ && prov_->resident()) {
        auto it = graphs_.find(key);
        if (it == graphs_.end()) {
            hipGraph_t g = nullptr;
            hipGraphExec_t ge = nullptr;
            HIPC(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
            try {
                verify_body(block, n);
            } catch (...) {
                (void)hipStreamEndCapture(stream_, &g);
                if (g) (void)hipGraphDestroy(g);
                pos_ = p;
                throw;
            }
            HIPC(hipStreamEndCapture(stream_, &g));
            const hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            HIPC(e);
            it = graphs_.emplace(key, ge).first;
        }
        HIPC(hipGraphLaunch(it->second, stream_));
    } else {
        verify_body(block, n);
    }
    if (step_events_) HIPC(hipEventRecord(ev1_, stream_));
    HIPC(hipStreamSynchronize(stream_));
    harvest();
    float ms = 0;
    if (step_events_) HIPC(hipEventElapsedTime(&ms, ev0_, ev1_));
    else ms = std::chrono::duration<float, std::milli>(std::chrono::steady_clock::now() - host0).count();
    last_step_ms_ = ms;
    const int* ctl = h_ctl_.as<int>();
    pos_ = p;
    check_flow(ctl);
    const uint32_t* o = reinterpret_cast<const uint32_t*>(ctl + FLOW_ACC);
    *m = o[0];
    *next = o[1];
    pos_ = p + o[0] + 1;  // truncate(p + m + 1), src/spec.rs:137-139
}

// A draft chain: k one-token verify passes (a block of one token accepts nothing and gives the
// argmax as `next`), each followed by chain_step, which makes that token the next pass's input
// one position further on. The staged words start as (position, first) and live on the device.
void Model::chain_body(size_t k) {
    HIPC(hipMemcpyAsync(stage_.p, h_stage_.p, 2 * 4, hipMemcpyHostToDevice, stream_));
    stage_pos_ = stage_.as<int>();
    const uint32_t* dtok = reinterpret_cast<const uint32_t*>(stage_.as<int>() + 1);
    for (size_t i = 0; i < k; i++) {
        forward_chunk(nullptr, dtok, 1, 1, false, dtok);
        chain_step(ctl_.as<int>(), stage_.as<int>(), chain_out_.as<uint32_t>(), int(i), int(k), stream_);
    }
    HIPC(hipMemcpyAsync(h_out_.p, chain_out_.p, (k + 1) * 4, hipMemcpyDeviceToHost, stream_));
}

void Model::draft_chain(uint32_t first, size_t k, uint32_t* out) {
    HIPC(hipSetDevice(device_));
    if (k == 0) return;
    if (k > MAX_CHAIN) fail("a draft chain takes at most " + std::to_string(MAX_CHAIN) + " passes");
    if (!prov_->resident()) fail("a draft chain runs over resident weights", LS_E_STATE);
    check_request(&first, 1);
    if (pos_ + k > max_ctx_) fail("the draft chain would pass the context limit");
    const size_t p = pos_;
    const std::pair<int, size_t> key(cur_, k);
    chunk_index_ = 0;
    h_stage_.as<int>()[0] = int(p);
    h_stage_.as<uint32_t>()[1] = first;
    arm_failure();
    if (graphs_on_ && !prof_) {
        auto it = chain_graphs_.find(key);
        if (it == chain_graphs_.end()) {
            hipGraph_t g = nullptr;
            hipGraphExec_t ge = nullptr;
            HIPC(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
            try {
                chain_body(k);
            } catch (...) {
                (void)hipStreamEndCapture(stream_, &g);
                if (g) (void)hipGraphDestroy(g);
                pos_ = p;
                throw;
            }
            HIPC(hipStreamEndCapture(stream_, &g));
            const hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            HIPC(e);
            it = chain_graphs_.emplace(key, ge).first;
        }
        HIPC(hipGraphLaunch(it->second, stream_));
    } else {
        chain_body(k);
    }
    HIPC(hipStreamSynchronize(stream_));
    harvest();
    const uint32_t* o = h_out_.as<uint32_t>();
    pos_ = p;
    if (o[k]) {
        // the same recovery as any pass whose in-launch wait gave up
        int ctl[CTL_BACK] = {};
        ctl[FLOW_ERR] = int(o[k]);
        check_flow(ctl);
    }
    for (size_t i = 0; i < k; i++) out[i] = o[i];
    pos_ = p + k;
}

// Batched verify: one pass over every sequence's block, rows in sequence order. Staging
// (ints): [attention segments 4 x n_segs][row positions R][row sequences R][block firsts n_seq]
// [block lengths n_seq][tokens R], moved by one copy.
void Model::batch_body(const uint32_t* blocks, size_t rows, size_t words, int n_segs) {
    HIPC(hipMemcpyAsync(stage_.p, h_stage_.p, words * 4, hipMemcpyHostToDevice, stream_));
    const int* d = stage_.as<int>();
    BatchView bv;
    bv.pos = d + 4 * size_t(n_segs);
    bv.seq = bv.pos + rows;
    const int* first = bv.seq + rows;
    const int* len = first + n_seq_;
    const uint32_t* dtok = reinterpret_cast<const uint32_t*>(len + n_seq_);
    bv.attn.segs = reinterpret_cast<const int4*>(d);
    bv.attn.n_segs = n_segs;
    bv.attn.pos = bv.pos;
    bv.attn.seq_stride = max_ctx_ * cfg_.kv_dim();
    stage_pos_ = d;
    chunk_index_ = 0;
    forward_chunk(blocks, dtok, rows, rows, false, nullptr, &bv);
    accept_greedy_batch(amax_.as<uint32_t>(), dtok, first, len, n_seq_, ctl_.as<int>(), bacc_.as<uint32_t>(), stream_);
    HIPC(hipMemcpyAsync(h_bacc_.p, bacc_.p, (1 + 2 * size_t(n_seq_)) * 4, hipMemcpyDeviceToHost, stream_));
}

void Model::verify_greedy_batch(const uint32_t* blocks, const size_t* lens, uint32_t* m, uint32_t* next) {
    HIPC(hipSetDevice(device_));
    if (!blocks || !lens || !m || !next) fail("no blocks, lengths or outputs");
    seq_pos_[size_t(cur_)] = pos_;
    size_t rows = 0;
    for (int q = 0; q < n_seq_; q++) {
        const std::string who = "sequence " + std::to_string(q);
        if (lens[q] == 0) fail(who + " has an empty block");
        if (lens[q] > MAX_BLOCK) fail(who + ": a batched verify block takes at most " + std::to_string(MAX_BLOCK) + " tokens");
        if (seq_pos_[size_t(q)] + lens[q] > max_ctx_)
            fail("context is full: " + who + " has " + std::to_string(seq_pos_[size_t(q)]) + " cached + " + std::to_string(lens[q]) +
                 " new tokens, above the limit of " + std::to_string(max_ctx_));
        rows += lens[q];
    }
    for (size_t i = 0; i < rows; i++)
        if (blocks[i] >= cfg_.vocab) fail("token id " + std::to_string(blocks[i]) + " is outside the vocabulary");
    // Attention segments: each sequence's rows in pieces of at most 16 from its first row (one
    // piece for a verify block of up to 16 rows, wherever it sits in the tiles).
    std::vector<int> segs;
    for (int q = 0, r = 0; q < n_seq_; q++) {
        const int end = r + int(lens[q]);
        while (r < end) {
            const int e = std::min(end, r + int(FTOK));
            segs.insert(segs.end(), {r, e - r, q, 0});
            r = e;
        }
    }
    const int n_segs = int(segs.size() / 4);
    int* hp = h_stage_.as<int>();
    std::memcpy(hp, segs.data(), segs.size() * 4);
    int* hpos = hp + segs.size();
    int* hseq = hpos + rows;
    int* hfirst = hseq + rows;
    int* hlen = hfirst + n_seq_;
    for (int q = 0, r = 0; q < n_seq_; q++) {
        hfirst[q] = r;
        hlen[q] = int(lens[q]);
        for (size_t i = 0; i < lens[q]; i++, r++) {
            hpos[r] = int(seq_pos_[size_t(q)] + i);
            hseq[r] = q;
        }
    }
    std::memcpy(hlen + n_seq_, blocks, rows * 4);
    const size_t words = segs.size() + 3 * rows + 2 * size_t(n_seq_);
    arm_failure();
    const auto host0 = std::chrono::steady_clock::now();
    if (step_events_) HIPC(hipEventRecord(ev0_, stream_));
    if (graphs_on_ && !prof_ && prov_->resident()) {
        const std::vector<size_t> key(lens, lens + n_seq_);
        auto it = batch_graphs_.find(key);
        if (it == batch_graphs_.end()) {
            hipGraph_t g = nullptr;
            hipGraphExec_t ge = nullptr;
            HIPC(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
            try {
                batch_body(blocks, rows, words, n_segs);
            } catch (...) {
                (void)hipStreamEndCapture(stream_, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            HIPC(hipStreamEndCapture(stream_, &g));
            const hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            HIPC(e);
            it = batch_graphs_.emplace(key, ge).first;
        }
        HIPC(hipGraphLaunch(it->second, stream_));
    } else {
        batch_body(blocks, rows, words, n_segs);
    }
    if (step_events_) HIPC(hipEventRecord(ev1_, stream_));
    HIPC(hipStreamSynchronize(stream_));
    harvest();
    float ms = 0;
    if (step_events_) HIPC(hipEventElapsedTime(&ms, ev0_, ev1_));
    else ms = std::chrono::duration<float, std::milli>(std::chrono::steady_clock::now() - host0).count();
    last_step_ms_ = ms;
    const uint32_t* o = h_bacc_.as<uint32_t>();
    check_flow(reinterpret_cast<const int*>(o));  // word 0 is the control block's error word
    for (int q = 0; q < n_seq_; q++) {
        m[q] = o[1 + 2 * q];
        next[q] = o[2 + 2 * q];
        seq_pos_[size_t(q)] += m[q] + 1;  // truncate(p + m + 1) per sequence, src/spec.rs:137-139
    }
    pos_ = seq_pos_[size_t(cur_)];
}

}  // namespace ls
