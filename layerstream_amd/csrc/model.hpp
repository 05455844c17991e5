// The device-side Model (src/model.rs:16-140) and its weight providers (src/provider.rs).
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <vector>

#include "common.hpp"
#include "fused.hpp"
#include "kernels.hpp"
#include "pass.hpp"
#include "source.hpp"

namespace ls {

void hip_check(hipError_t e, const char* what);
#define HIPC(x) ::ls::hip_check((x), #x)

// Device allocation owned by one object.
struct DevBuf {
    void* p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    explicit DevBuf(size_t bytes);
    ~DevBuf();
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
    DevBuf& operator=(DevBuf&& o) noexcept;
    template <class T> T* as() const { return static_cast<T*>(p); }
};

// Pinned host allocation (hipHostMalloc).
struct PinnedBuf {
    void* p = nullptr;
    size_t n = 0;
    PinnedBuf() = default;
    explicit PinnedBuf(size_t bytes);
    ~PinnedBuf();
    PinnedBuf(const PinnedBuf&) = delete;
    PinnedBuf& operator=(const PinnedBuf&) = delete;
    PinnedBuf(PinnedBuf&& o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
    PinnedBuf& operator=(PinnedBuf&& o) noexcept;
    template <class T> T* as() const { return static_cast<T*>(p); }
};

// One transformer layer on the device, tile layout: q|k|v fused (rows h, kv, kv; q and k rows
// with RoPE pairs adjacent), gate|up fused with 16 GU_STRIPS-row blocks interleaved (gate block
// a, up block a, ...), o and down; f32 bias and norms.
struct DevLayer {
    TMat qkv, o, gu, down;
    const float* b_qkv = nullptr;
    const float* in_norm = nullptr;
    const float* post_norm = nullptr;
};

// Byte offsets of one layer inside a device arena.
struct LayerArena {
    TMat qkv, o, gu, down;  // shapes
    size_t qkv_d, qkv_s, o_d, o_s, gu_d, gu_s, down_d, down_s, b_qkv, in_norm, post_norm, total;
};
LayerArena layer_arena(const Config& c);
DevLayer bind_layer(const LayerArena& a, uint8_t* base);
void clear_layer(const LayerArena& a, uint8_t* base, hipStream_t s);
// Rearrange a raw layer block (reference layout, already on the device) into the arena.
void build_layer_device(const Config& c, const LayerLayout& L, const uint8_t* raw_dev, const LayerArena& a, uint8_t* base,
                        hipStream_t s);

struct HeadChunk {
    size_t first = 0, rows = 0;
    TMat mat;
};

constexpr size_t HEAD_ROWS = 4096;  // src/provider.rs:21
// Streamed table pieces: four of the reference's chunks per copy (about a layer block at int4), so
// the table crosses PCIe in 10 copies instead of 38. Every logit depends on its own row only, so
// the piece size changes no value.
constexpr size_t STREAM_HEAD_ROWS = 4 * HEAD_ROWS;

class DeviceProvider {
public:
    virtual ~DeviceProvider() = default;
    virtual const char* name() const = 0;
    virtual void begin_forward(bool with_head) = 0;
    virtual const DevLayer& layer(size_t l) = 0;  // ordered before later work on the compute stream
    virtual void release_layer(size_t l) = 0;     // the compute stream has every kernel of layer l
    virtual size_t n_head_chunks() const = 0;
    virtual HeadChunk head_chunk(size_t c) = 0;
    virtual void release_head_chunk(size_t c) = 0;
    virtual void end_forward() = 0;
    // True when every layer stays on the device (layer(l) may be asked for out of order).
    virtual bool resident() const = 0;
    // x[t][h] = embedding rows of host tokens (device tokens copy for the resident table); with
    // frags also the fragments of x * w and the sum-of-squares partials.
    // With a mirror (resident tables only) the tokens are read from its pinned host words, which the
    // kernel also copies to the device (the call's staging copy).
    virtual void embed(const uint32_t* host_tokens, const uint32_t* dev_tokens, int t, float* x, const float* w,
                       uint8_t* frags, float* ss, const StageMirror& mirror) = 0;
    virtual ls_report report() const = 0;
};

std::unique_ptr<DeviceProvider> make_resident(const Source& src, hipStream_t compute);
std::unique_ptr<DeviceProvider> make_stream(const Source& src, int slots, size_t max_rows, hipStream_t compute);

// Device rows of a pass over several sequences (set up by verify_greedy_batch).
struct BatchView {
    const int* pos = nullptr;  // per launch row: position in its sequence
    const int* seq = nullptr;  // per launch row: sequence
    AttnRows attn;
};

// One model on one device. It holds n_seq independent sequences (K/V caches and positions)
// over one copy of the weights; forward, forward_multi, verify_greedy, truncate, reset and pos
// act on the selected sequence (0 unless select() says otherwise), verify_greedy_batch on all.
class Model {
public:
    Model(const Source& src, int mode, int slots, size_t max_ctx, int device, int n_seq = 1);
    ~Model();
    const Config& cfg() const { return cfg_; }
    size_t pos() const { return pos_; }
    size_t max_ctx() const { return max_ctx_; }
    void reset() { pos_ = 0; }
    void truncate(size_t pos);
    int n_seq() const { return n_seq_; }
    int selected() const { return cur_; }
    void select(int seq);
    // One verify pass over a block per sequence (blocks concatenated, lens[s] tokens for
    // sequence s): the greedy acceptance of each, as verify_greedy would give it alone.
    void verify_greedy_batch(const uint32_t* blocks, const size_t* lens, uint32_t* m, uint32_t* next);
    // Model::forward: logits/argmax of the last token (each may be null).
    void forward(const uint32_t* tok, size_t n, float* logits, uint32_t* argmax);
    void forward_multi(const uint32_t* tok, size_t n, size_t n_logits, float* logits, uint32_t* argmax);
    void verify_greedy(const uint32_t* block, size_t n, uint32_t* m, uint32_t* next);
    // k greedy one-token passes chained on the device (a draft model's proposals, src/spec.rs:100-107):
    // out[i] is the argmax after consuming first, out[0] .. out[i - 1]; the model advances by k.
    // The same tokens as k calls of forward + argmax, with one host wait for all of them.
    void draft_chain(uint32_t first, size_t k, uint32_t* out);
    bool chains_on_device() const { return prov_->resident(); }
    ls_report report() const { return prov_->report(); }
    double last_step_ms() const { return last_step_ms_; }
    int device() const { return device_; }
    // mode 0: off; 1: every matrix launch; 2: each pass's dominant launch (the layer stack when a
    // pass runs as one, else every matrix launch).
    void set_profiling(int mode);
    void set_graphs(bool on);
    ls_kernel_stat read_profile();
    // Test hook: the next device pass starts with the control block's error word set.
    void debug_fail_next() { fail_next_ = true; }
    // Per-unit stamps of the last persistent pass (LS_PASS_TIMELINE=1), copied to out (cap
    // words); returns the words available (0 without a timeline).
    size_t debug_timeline(uint64_t* out, size_t cap);
    // A copy of an internal device buffer (debugging): returns its size in bytes, copies up to cap.
    size_t debug_read(const char* name, void* out, size_t cap);

private:
    void check_request(const uint32_t* tok, size_t n) const;
    // Pushes t tokens through every layer; with n_logits > 0 also the head for the last rows,
    // logits stored when want_logits.
    // With accept_block (device tokens of a verify block) the argmax kernel also writes the
    // greedy acceptance (m, next) to acc_.
    // With bv the rows belong to several sequences (positions and caches from bv, no position
    // update).
    void forward_chunk(const uint32_t* tok, const uint32_t* dtok, size_t t, size_t n_logits, bool want_logits,
                       const uint32_t* accept_block = nullptr, const BatchView* bv = nullptr);
    const uint32_t* stage_tokens(const uint32_t* tok, size_t n);
    // The device part of a verify step (token and position copies from the pinned staging
    // buffers, forward pass, acceptance, result copy): what a graph captures.
    void verify_body(const uint32_t* block, size_t n);
    // The device part of a draft chain of k passes (what a graph captures).
    void chain_body(size_t k);
    // The device part of a batched verify step; words: staged ints, n_segs: attention segments.
    void batch_body(const uint32_t* blocks, size_t rows, size_t words, int n_segs);
    void plan_kw_from_env();
    void harvest();
    void prof_begin();
    void prof_end(const TMat& W, int nt, bool launch = true, double extra_bytes = 0);
    void check_flow(const int* ctl);
    // Sets the error word on the stream when debug_fail_next() asked for it (outside any graph).
    void arm_failure();

    Config cfg_;
    int device_;
    size_t max_ctx_, pos_ = 0, chunk_index_ = 0;
    int n_seq_ = 1, cur_ = 0;
    std::vector<size_t> seq_pos_;  // positions of the sequences not selected
    size_t rows_cap_ = 0;          // launch rows the buffers hold (a prefill chunk or a batch)
    hipStream_t stream_ = nullptr;
    std::unique_ptr<DeviceProvider> prov_;
    DevBuf kcache_, vcache_, rope_cos_, rope_sin_, fnorm_, stage_;
    // x_: residual rows; xf_/ss_: fragments and sum-of-squares partials of the next normalised
    // input; af_: attention output fragments; actf_: SiLU(g) * u fragments; part_/cnt_: split-K
    // scratch; hpv_/hpi_: head-block argmax partials; row0_: logits of row 0.
    DevBuf x_, q_, xf_, ss_, af_, actf_, part_, cnt_, attn_scratch_, attn_cnt_, logits_, hpv_, hpi_, row0_, amax_, ctl_, bacc_;
    // Resident models: every layer's pointers for the layer-stack launch (LayerPtrs per layer).
    DevBuf layer_ptrs_;
    DevBuf stack_tl_;  // layer-stack timeline (LS_STACK_TIMELINE=1): [workgroup][4] stamps
    // The persistent pass (one-tile passes over resident layers; LS_PASS=0: the layer stack): its
    // exchange area, flag lines and epoch word (bumped by the embedding kernel before each pass),
    // and per-unit timeline stamps when LS_PASS_TIMELINE=1.
    bool pass_on_ = false;
    DevBuf pass_area_, pass_flags_, epoch_, pass_tl_;
    PassArea pass_shape_;
    PinnedBuf h_stage_, h_out_, h_ctl_, h_bacc_;
    // Control block: FLOW_WORDS words of fused-launch counters, then the acceptance (m, next).
    static constexpr int CTL_BACK = FLOW_ACC + 2;  // control words copied back after a pass: error, acceptance
    bool fuse_on_ = true;
    bool fuse_qkv_ = true;  // q|k|v joins the attention + o launch
    bool pf_on_ = true;     // fused consumers prefetch the next launch's weights
    bool pipe_on_ = true;   // large single-tile gate|up as a pipelined launch (LS_PIPE=0: k_mm)
    bool stack_on_ = true;  // one-tile passes over resident layers run as one layer-stack launch (LS_STACK=0: per layer)
    const int* stage_pos_ = nullptr;  // device positions of the staged chunks
    size_t vpad_ = 0, fb_h_ = 0, fb_q_ = 0, fb_in_ = 0;
    int head_blocks_ = 0, slots_h_ = 0;
    size_t head_off_ = 0;  // launch row of the first requested head row
    // wavefronts along K per row group: q|k|v, o, gate|up, down, head
    int kw_qkv_ = 7, kw_o_ = 7, kw_gu_ = 7, kw_down_ = 8, kw_head_ = 7;
    int wide_ = 1;  // K share of a wavefront in 128-column units (MMPlan::wide) for every layer matrix
    int qs_ = 1, os_ = 1, ds_ = DOWN_STRIPS;  // strips per wavefront of q|k|v, o and down
    int mqs_ = 1, mos_ = 1, mds_ = DOWN_STRIPS;  // the same in launches over several token tiles
    hipEvent_t ev0_ = nullptr, ev1_ = nullptr;
    double last_step_ms_ = 0;
    int prof_ = 0;  // profiling mode (set_profiling)
    // Verify steps over resident weights read their staged words from pinned host memory and the
    // head writes the result there (LS_DIRECT=0: a copy each way instead).
    bool direct_on_ = true;
    // Verify steps time themselves on the host clock, from the launch until the result is back
    // (LS_STEP_EVENTS=1: device events around the launch instead; their markers cost ~4 us a step).
    bool step_events_ = false;
    StageMirror mirror_;
    uint32_t* fin_host_ = nullptr;
    bool prof_skip_ = false;  // launches of this pass outside the profiled set
    bool graphs_on_ = true;
    bool fail_next_ = false;
    std::map<std::pair<int, size_t>, hipGraphExec_t> graphs_;  // verify step per (sequence, block length)
    std::map<std::vector<size_t>, hipGraphExec_t> batch_graphs_;  // batched verify step per block lengths
    std::map<std::pair<int, size_t>, hipGraphExec_t> chain_graphs_;  // draft chain per (sequence, length)
    DevBuf chain_out_;  // a draft chain's tokens, then its error word
    std::vector<hipEvent_t> prof_ev_;
    size_t prof_used_ = 0;
    ls_kernel_stat prof_acc_{};
};

}  // namespace ls
