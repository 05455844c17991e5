// The persistent layer pass (pass.hip): every layer of a one-tile pass in one launch of one
// workgroup per CU, with tagged exchanges between the stages instead of counters.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fused.hpp"

namespace ls {

// Stages of one layer. Units of QKV (one q|k|v strip), ATT (one of ATTN_SPLIT key-block sets of
// a head; set 0 also merges the head: MRG), O (one o strip), GU (one gate|up row block) and DN
// (one down row block and K split; split 0 also adds the splits: FIX) publish their outputs in
// the exchange area, each with a flag line.
enum { PS_QKV = 0, PS_ATT = 1, PS_MRG = 2, PS_O = 3, PS_GU = 4, PS_DNP = 5, PS_FIX = 6, PS_STAGES = 7 };
constexpr int PASS_MAXU = 256;  // flag lines per stage

// Tagged units: 16 bytes {w0, w1, w2, tag}, written with one store, tag = (epoch << 6) | layer.
// A consumer that reads a unit whose tag differs reads it again, so a producer raises its flag
// right after issuing its stores, without waiting for them.
struct PassArea {
    uint8_t* base = nullptr;  // two sets of buffers, even and odd layers
    size_t set_bytes = 0;
    // offsets inside a set:
    size_t qkvx = 0;  // q|k|v rows: [token][octet of 8 reference dims][3 units]
    size_t atts = 0;  // attention states of sets 1..: [head][set][token][state units]
    size_t af = 0;    // attention output fragments: [k-step][column group][token][4 units]
    size_t xar = 0;   // residual rows after o: [strip][token][6 units] (16 rows, then the sum of squares)
    size_t xaf = 0;   // fragments of those rows * post_norm
    size_t actf = 0;  // SiLU(gate) * up fragments
    size_t dnp = 0;   // down pieces of splits 1..: [row block][split][token][pieces units]
    size_t xr = 0;    // residual rows after down: [strip][token][6 units]
    size_t xf = 0;    // fragments of those rows * the next layer's input norm
    size_t xass = 0;  // sums of squares of the rows after o: [strip][token] 8-byte units {ss, tag}
    size_t xss = 0;   // the same after down
    // Buffers that many units read whole (fragments, sums of squares) are written in `repl`
    // copies, copy r at offset + r * stride; consumer unit u reads copy u % repl, which spreads
    // the simultaneous reads over more memory channels.
    int repl = 1;
    size_t af_r = 0, xaf_r = 0, actf_r = 0, xf_r = 0, ss_r = 0;
    int* flags = nullptr;  // [2 sets][PS_STAGES][PASS_MAXU] lines of 16 ints
    size_t flag_bytes = 0;
};
constexpr int PASS_MAX_REPL = 16;
// Byte sizes of the area for a model shape (the buffers of one set, repl copies of the broadcast
// ones) and the flag lines.
PassArea pass_area_shape(int hidden, int heads, int kv_heads, int hd, int inter, const MMPlan& pd, int repl);
PassArea pass_area_bind(const PassArea& shape, uint8_t* base, int* flags);

// Why a one-tile pass with these plans cannot run as a persistent pass, or null when it can.
const char* layer_pass_unfit(int t, int heads, int kv_heads, int hd, const MMPlan& pq, const MMPlan& po, const MMPlan& pg,
                             const MMPlan& pd);
// Every layer of a one-tile pass, with the plans and so the bits of the per-layer launches (the
// same arguments as layer_stack). epoch: a device word that increases by one before each pass
// (the embedding kernel's). timeline: null, or pass_timeline_words() u64 for per-unit stamps.
void layer_pass(const LayerPtrs* lp, int layers, size_t seq_off, const MMArgs& qa, const MMPlan& pq, const MMArgs& oa,
                const MMPlan& po, const MMArgs& ga, const MMPlan& pg, const MMArgs& da, const MMPlan& pd, const PassArea& area,
                int* ctl, const int* epoch, uint64_t* timeline, hipStream_t s);
size_t pass_timeline_words(int layers);

}  // namespace ls
