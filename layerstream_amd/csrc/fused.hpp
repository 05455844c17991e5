// Fused MFMA kernels of the verify step (gfx950).
//
// Weights use the "tile" layout: rows in strips of 16 (the MFMA M dimension), columns padded to a
// multiple of 128 and cut into chunks of 16 bytes per lane ([strip][chunk][64 lanes][16 B]), so
// that a wavefront load of one chunk of one strip is 1 KiB of contiguous memory and each lane
// receives exactly the A operand of v_mfma_f32_16x16x32_bf16 for its row and k-block. A chunk
// covers 32 columns for bf16, 64 for int8 and 128 for int4. Scales are [strip][group][16 rows]
// bf16.
//
// Activations reach the MFMA B operand as "fragments": three bf16 terms whose sum is the f32
// value exactly, stored per tile of 16 tokens as [k-step][term][64 lanes][16 B] (lane l holds
// token l % 16, columns 32 k-step + 8 (l / 16) + [0, 8)). Every matrix input is written in this
// form by the kernel that produces it (embedding, attention, the residual and SiLU epilogues), so
// the matrix kernels start streaming weights at once. Inputs that the reference RMS-normalises
// are stored as x * w; the per-token 1 / rms is applied to the matrix output in the epilogue,
// from sum-of-squares partials (one per 16 columns, [tile][slot][16 tokens]) that the producer
// writes beside the fragments.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ls {

struct TMat {
    const uint8_t* data = nullptr;
    const uint16_t* scales = nullptr;
    int bits = 16, group = 0;
    int rows = 0, cols = 0;
    int n_strips = 0;   // padded to a multiple of 4 (64 rows) or more
    int n_chunks = 0;   // chunks per strip
    int n_groups = 0;   // groups per row, padding columns included
};

constexpr int FTOK = 16;  // tokens per tile (the MFMA N dimension)

__host__ __device__ inline int tile_chunk_cols(int bits) { return bits == 16 ? 32 : (bits == 8 ? 64 : 128); }
__host__ __device__ inline int tile_kpad(int cols) { return (cols + 127) / 128 * 128; }
// Rows are padded to a multiple of row_align.
TMat tile_shape(int bits, int group, int rows, int cols, int row_align = 64);
size_t tile_data_bytes(const TMat& m);
size_t tile_scale_bytes(const TMat& m);
TMat tile_bind(const TMat& shape, uint8_t* data, uint16_t* scales);
// Rearrange `rows` reference rows (raw, on the device) into the tile layout. Source row r goes
// to destination row row_off + (r / block) * stride + r % block (block = rows: contiguous); with
// pair_hd > 0 the rows of each pair_hd-row head are first reordered so that RoPE pairs are
// adjacent (row j -> 2j, row j + pair_hd / 2 -> 2j + 1).
void tile_repack(const uint8_t* raw, int rows, const TMat& dst, int row_off, int block, int stride, hipStream_t s,
                 int pair_hd = 0);
// Initialise padding: zero-weight bytes and zero scales over the whole matrix.
void tile_clear(const TMat& m, hipStream_t s);

// Bytes of one token tile of fragments for `cols` input columns.
__host__ __device__ inline size_t frag_tile_bytes(int cols) { return size_t(tile_kpad(cols)) / 32 * 3 * 1024; }
// Sum-of-squares slots (16 columns each) of a row of `cols` values.
__host__ __device__ inline int ss_slots(int cols) { return (cols + 15) / 16; }
// gate|up rows are interleaved in blocks of 16 * GU_STRIPS (gate block, up block, ...). A
// workgroup row group holds a gate block and its up block. One wavefront streams both (4 strips),
// so the input fragments it loads serve both, and a workgroup of 7 wavefronts along K fits the
// layer stack's 512 threads. Groups of 16 need the registers for their extra MFMAs, so they use
// two wavefronts of one block each.
constexpr int GU_STRIPS = 2;
__host__ __device__ constexpr int gu_wave_strips(int bits, int group) { return (bits == 16 || group != 16) ? 2 * GU_STRIPS : GU_STRIPS; }
// Strips per wavefront of the down projection: its K (the FFN width) is long and its rows few,
// so two strips halve the input-fragment reads per weight byte.
constexpr int DOWN_STRIPS = 2;

// A call's staged words (positions, then tokens) read by the first kernel of a pass straight from
// pinned host memory and mirrored into device memory for the later kernels, in place of a copy.
struct StageMirror {
    const int* host = nullptr;  // pinned host words (device-accessible)
    int* dev = nullptr;         // their device copy
    int words = 0;
    int tok_off = 0;  // first token word
    // When set, the embedding kernel adds one to this device word (the persistent pass's epoch).
    int* epoch = nullptr;
};
// Embedding rows of tokens from a tile-layout table (src/kernels.rs:95-121 dequantization) into
// x [n][cols], plus fragments of x * w and sum-of-squares partials. With a mirror the tokens are
// read from its host words (tok_off on) and all its words are copied to the device.
void tile_embed(const TMat& E, const uint32_t* tokens, int n, float* x, const float* w, uint8_t* frags, float* ss,
                hipStream_t s, const StageMirror& mirror = StageMirror{});
// Fragments (of x * w, or of x when w is null) and sum-of-squares partials (when ss is not null)
// of rows [0, n) of x [n][cols].
void x_frags(const float* x, int n, int cols, const float* w, uint8_t* frags, float* ss, hipStream_t s);

struct MMArgs {
    TMat W;
    // Layer-stack timeline words of this workgroup (profiling; null: none): 3 its inputs loaded
    // (wavefront 0), 4 products issued (wavefront 0), 5 row-group sums done, 6 epilogue stores
    // issued.
    unsigned long long* tlw = nullptr;
    // input: fragments, tile stride frag_stride; optional RMSNorm (1 / rms from ss partials)
    const uint8_t* frags = nullptr;
    size_t frag_stride = 0;
    const float* ss = nullptr;
    int ss_slots = 0;
    float eps = 0;
    int n = 0;  // tokens of the launch (tiles of 16)
    // epilogue
    const float* bias = nullptr;
    float* out = nullptr;  // q rows / residual rows / logits
    int ldo = 0;
    float* kcache = nullptr;
    float* vcache = nullptr;
    const float* rope_cos = nullptr;
    const float* rope_sin = nullptr;
    const int* pos0 = nullptr;  // device scalar: position of token 0 of the launch
    // Rows of several sequences (device, per launch row; null for one sequence): row i sits at
    // position row_pos[i] of sequence row_seq[i], whose K/V rows start seq_stride rows into the
    // caches.
    const int* row_pos = nullptr;
    const int* row_seq = nullptr;
    size_t seq_stride = 0;
    int heads = 0, kv_heads = 0, hd = 0;
    // output fragments and sum-of-squares partials (residual: of x * onorm; SiLU: of act)
    uint8_t* ofrags = nullptr;
    size_t ofrag_stride = 0;
    const float* onorm = nullptr;
    float* oss = nullptr;
    int oss_slots = 0;
    // head: per-block argmax partials [tile][arg_stride][16], block index arg_off + block
    float* arg_val = nullptr;
    int* arg_idx = nullptr;
    int arg_stride = 0, arg_off = 0;
    int row_base = 0;       // added to argmax row indices
    float* row0 = nullptr;  // logits of row 0 per token ([tile * 16 + token]), when set
    // Consumers of a fused launch: bytes to read (into LDS, discarded) while waiting for the
    // input, so that a later launch finds them in the memory-side cache.
    const uint8_t* pf = nullptr;
    size_t pf_bytes = 0;
    // Head only: the last workgroup to finish (fin_cnt, zero between launches, counts them)
    // reduces every workgroup's argmax partials (row0 holds logits[.][0]) into fin_amax, applies
    // greedy acceptance to the verify block fin_block (n tokens; src/spec.rs:119-127) and writes
    // [ctl[FLOW_ERR], m, next] to fin_host (pinned host memory) and m, next to ctl + FLOW_ACC.
    int* fin_cnt = nullptr;
    int* fin_ctl = nullptr;
    const uint32_t* fin_block = nullptr;
    uint32_t* fin_amax = nullptr;
    uint32_t* fin_host = nullptr;
};

// Work split of one launch: each wavefront streams s strips (16 s rows); a workgroup owns rg
// such row groups and one of nsplit K ranges, cut among kw wavefronts per row group. With
// nsplit > 1 the pieces meet in `part` and the last workgroup of a row block to finish adds them
// in split order (counters in `cnt` start at zero and are left at zero). A wavefront's share of K
// is 128 columns, or 256 when wide is 2 (hidden sizes of 2048 and more: 8 wavefronts then cover
// the row without a split, so every role of such a layer fits a 512-thread workgroup). The share
// decides the summation order, so every launch of a model uses the same wide.
struct MMPlan {
    int s = 1, rg = 1, kw = 1, nsplit = 1, nrb = 1, tiles = 1, wide = 1;
};
// Wavefronts a matrix workgroup may hold: 16 (1024 threads, at most 128 registers each), but 8
// for four bf16 or groups-of-16 strips per wavefront, whose wider chunks or extra MFMAs need more
// registers.
__host__ __device__ constexpr int mm_max_waves(int bits, int group, int strips) {
    return (strips == 4 && (bits == 16 || group == 16)) ? 8 : 16;
}
MMPlan mm_plan(const TMat& W, int rg, int kw, int n_tokens, int strips, int wide = 1);
// The gate|up plan: gu_wave_strips strips per wavefront, row groups making one gate and up block.
MMPlan gu_plan(const TMat& W, int kw, int n_tokens, int wide = 1);
size_t mm_part_floats(const MMPlan& p);
size_t mm_counters(const MMPlan& p);

// Compute units of the current device (cached after the first call).
int device_cu_count();
// Time the next matrix launch of this thread: the dispatch itself records `start` when the
// kernel begins and `stop` when it ends (hipExtLaunchKernel), so no marker sits in between.
void mm_time_next_launch(hipEvent_t start, hipEvent_t stop);

struct MMScratch {
    float* part = nullptr;
    int* cnt = nullptr;
};

// In-launch dataflow between the two workgroup roles of a fused launch. Producer workgroup r
// adds 1 to counter r / per once its output is stored; the consumers of counter j wait until it
// reaches the number of producers that feed it, count themselves in the counter's second word,
// and the last of `consumers` puts both words back to zero. Counters sit FLOW_CNT_STRIDE words
// apart (their own cache lines). A wait that gives up sets the error word and goes on.
//
// A counter with many consumers is mirrored: each producer adds 1 to `mirrors` copies on
// separate lines and consumer w polls copy w % mirrors, so that no line is polled by more than
// a few workgroups (atomics on one line are served one after another). Counter j, copy m is
// slot base + j mirrors + m; the consumer count sits beside copy 0. Every copy must have a
// consumer (mirrors <= consumers, consumers numbered 0, 1, ...), so that every copy is complete
// before the last consumer resets them.
struct Flow {
    int* ctl = nullptr;  // control block, FLOW_WORDS ints, zero between launches
    int producers = 0;
    int per = 1;        // producers per counter
    int consumers = 0;  // consumer workgroups per counter
    int base = 0;       // first counter slot of this launch
    int want = 0;       // when set: the count every counter waits for (producers may feed several)
    int mirrors = 1;    // copies of each counter
    // Counter slots this producer puts back to zero just before it signals (two ranges of slots:
    // first, count), for flows whose consumers (consumers == 0: they do not count themselves)
    // have all finished waiting by then.
    int zero0 = 0, nzero0 = 0, zero1 = 0, nzero1 = 0;
    // When set, the wait stores the s_memrealtime count (100 MHz) at which its input was there.
    unsigned long long* stamp = nullptr;
};
// Control block words: error flag, greedy acceptance (m, next), the head's finished-workgroup
// count (its own 128-byte line), then the counter slots (gate|up
// -> down from slot 0, FLOW_GU_MIRRORS per down K split; q|k|v -> attention one per head from
// slot 0; attention -> o at FLOW_ATTN_O, FLOW_AO_MIRRORS copies).
enum { FLOW_ERR = 0, FLOW_ACC = 1, FLOW_FIN = 32, FLOW_CNT0 = 64, FLOW_CNT_STRIDE = 64, FLOW_COUNTERS = 48, FLOW_ATTN_O = 40 };
constexpr int FLOW_GU_MIRRORS = 2, FLOW_AO_MIRRORS = 8;
constexpr int FLOW_WORDS = FLOW_CNT0 + FLOW_CNT_STRIDE * FLOW_COUNTERS;

// QKV projection + 1/rms + bias + RoPE + K/V append (plan strips 1). Rows: q heads and k heads
// with each head's RoPE pairs adjacent (tile row 2j: dimension j, 2j + 1: dimension j + hd / 2),
// then v heads.
void mm_qkv(const MMArgs& a, const MMPlan& p, const MMScratch& sc, hipStream_t s);
// x[row] += W x; then fragments of x * onorm and sum-of-squares partials of the new rows (plan
// strips 1, 2 or 4).
void mm_residual(const MMArgs& a, const MMPlan& p, const MMScratch& sc, hipStream_t s);
// gate|up projection (row blocks of 16 GU_STRIPS interleaved gate, up; plan from gu_plan) +
// 1/rms + SiLU(g) * u -> act fragments.
void mm_gate_up(const MMArgs& a, const MMPlan& p, const MMScratch& sc, hipStream_t s);
// The same gate|up over one token tile as a pipelined launch (one workgroup per CU walking a range
// of gate and up strip pairs, its input fragments held in registers, the next pairs' weights in
// flight while one pair's epilogue runs); the same bits as mm_gate_up under the same plan. Fits a
// plan of one tile, one row group, 16 wavefronts along K, no K split, scale groups inside a chunk.
bool mm_gate_up_pipe_fits(const MMArgs& a, const MMPlan& p);
void mm_gate_up_pipe(const MMArgs& a, const MMPlan& p, hipStream_t s);
// gate|up then down (plan strips DOWN_STRIPS) in one launch for one token tile: each down K
// split waits only for the gate|up row blocks that produce its columns. ctl is the control
// block (FLOW_WORDS ints).
void mm_gate_up_down(const MMArgs& gu, const MMPlan& pgu, const MMArgs& dn, const MMPlan& pdn, const MMScratch& sc,
                     int* ctl, hipStream_t s);
// Attention (one token tile of one sequence, see attention() in kernels.hpp) and the o
// projection (mm_residual, plan strips 1 without a K split) in one launch: the o workgroups
// load their weights while attention runs. ctl is the control block.
void attention_o(const float* q, int ldq, int t, int heads, int kv_heads, int hd, const int* pos0, const float* kc, const float* vc,
                 float* scratch, int* cnt, uint8_t* frags, const MMArgs& o, const MMPlan& po, const MMScratch& sc, int* ctl,
                 hipStream_t s);
// Workgroups of an attention_o launch (its grid, one workgroup per CU at most).
int attention_o_workgroups(int heads, const MMPlan& po);
// q|k|v (mm_qkv, plan strips 1 without a K split: one workgroup per 16-row strip), attention and
// o in one launch for one token tile: q|k|v rows are stored through the coherent path and each
// strip counts itself done for the heads that read it (a q strip for its head, a k or v strip for
// every head of its group); the attention workgroups load the keys and values cached before this
// pass while q|k|v runs, wait for their head, then read q and the new rows coherently; o as in
// attention_o. q, the caches and the position come from qa.
void qkv_attention_o(const MMArgs& qa, const MMPlan& pq, float* scratch, int* cnt, uint8_t* frags, const MMArgs& o, const MMPlan& po,
                     const MMScratch& sc, int* ctl, hipStream_t s);
// Workgroups of a qkv_attention_o launch.
int qkv_attention_o_workgroups(int heads, const MMPlan& pq, const MMPlan& po);

// Weights, vectors and caches of one resident layer, for the layer-stack launch (a device array,
// one entry per layer).
struct LayerPtrs {
    TMat qkv, o, gu, down;
    const float* b_qkv = nullptr;
    const float* post_norm = nullptr;
    const float* next_norm = nullptr;  // the next layer's input norm; the final norm after the last layer
    float* kc = nullptr;               // this layer's K/V cache rows of sequence 0
    float* vc = nullptr;
};
// Counter slots of the layer-stack launch: FLOW_LAYER_STRIDE per layer after the FLOW_COUNTERS of
// the per-layer launches. Inside a layer's block: q|k|v -> attention from FL_Q (one per head),
// attention -> o at FL_A, o -> gate|up at FL_O, down -> the next layer's q|k|v at FL_D (each
// FL_MIRRORS copies), gate|up -> down from FL_G (FLOW_GU_MIRRORS copies per down K split).
enum { FLOW_LAYER_STRIDE = 160, FL_Q = 0, FL_A = 32, FL_O = 48, FL_D = 64, FL_G = 80, FL_MIRRORS = 16 };
// Words of a control block that serves launches over `layers` layers.
inline size_t flow_words(int layers) {
    return FLOW_CNT0 + size_t(FLOW_CNT_STRIDE) * (FLOW_COUNTERS + size_t(FLOW_LAYER_STRIDE) * size_t(layers));
}
struct LayerFlows {
    int* ctl = nullptr;
    int layers = 0;
    int gu_per = 1;                      // gate|up row blocks per down K split
    int m_a = 1, m_o = 1, m_d = 1, m_g = 1;  // copies of the attention -> o, o -> gate|up, down -> q|k|v, gate|up -> down counters
    // Per-workgroup timeline (LS_STACK_TIMELINE=1), [workgroup][8] s_memrealtime counts: 0 entry,
    // 1 input there (after the wait), 2 done, 3-6 matrix roles' phases (MMArgs::tlw); word 7 is
    // layer << 8 | role (0 q|k|v, 1 attention, 2 o, 3 gate|up, 4 down).
    unsigned long long* tl = nullptr;
};
// Workgroups of one layer in the layer-stack launch.
int layer_stack_workgroups(int heads, const MMPlan& pq, const MMPlan& po, const MMPlan& pg, const MMPlan& pd);
// Why plans of a pass over t tokens cannot run as a layer stack, or null when they can.
const char* layer_stack_unfit(int t, int heads, int kv_heads, int hd, const MMPlan& pq, const MMPlan& po, const MMPlan& pg,
                              const MMPlan& pd);
// Every layer of a one-tile pass in one launch: per layer q|k|v (+ RoPE, K/V append), attention,
// o (+ residual), gate|up (+ SiLU) and down (+ residual), the same plans and so the same bits as
// the per-layer launches. qa/oa/ga/da carry everything but the per-layer pointers, which come
// from lp (caches offset by seq_off floats). The fragments and partials of x * next_norm after
// the last layer are left for the head. ctl holds flow_words(layers) words, zero between launches.
void layer_stack(const LayerPtrs* lp, int layers, size_t seq_off, const MMArgs& qa, const MMPlan& pq, float* attn_scratch, int* attn_cnt,
                 uint8_t* af, const MMArgs& oa, const MMPlan& po, const MMArgs& ga, const MMPlan& pg, const MMArgs& da,
                 const MMPlan& pd, const MMScratch& sc, int* ctl, hipStream_t s, unsigned long long* timeline = nullptr);

// Output head (plan strips 4, rg 1): logits (1/rms applied), optional logits store, argmax
// partials at [tile][arg_off + b][16] for b below the returned count. With a.fin_cnt (one head
// launch, arg_off 0) it also does what head_argmax_final does for a verify block.
int mm_head(const MMArgs& a, const MMPlan& p, const MMScratch& sc, hipStream_t s);
// Final argmax over head-block partials (src/spec.rs:41-49 rule) for n tokens; row0 holds
// logits[.][0]. With a verify block (device tokens, n of them) it also writes the greedy
// acceptance acc[0] = m, acc[1] = next (src/spec.rs:119-127).
void head_argmax_final(const float* pv, const int* pi, int arg_stride, int nblocks, const float* row0, int n, uint32_t* amax,
                       const uint32_t* block, uint32_t* acc, hipStream_t s);

// Greedy acceptance of several verify blocks from the argmax of every launch row: block s
// holds rows [first[s], first[s] + len[s]) with tokens tok (src/spec.rs:119-127 per block).
// out = [ctl[FLOW_ERR], m_0, next_0, m_1, next_1, ...].
void accept_greedy_batch(const uint32_t* amax, const uint32_t* tok, const int* first, const int* len, int n_seq, const int* ctl,
                         uint32_t* out, hipStream_t s);
// One link of a draft chain, after a one-token verify pass: the pass's greedy token
// (ctl[FLOW_ACC + 1]) becomes out[i] and the next pass's input (stage[1]), whose position is one
// more (stage[0] += 1); out[n] keeps the error word.
void chain_step(const int* ctl, int* stage, uint32_t* out, int i, int n, hipStream_t s);

}  // namespace ls
