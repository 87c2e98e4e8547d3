// Device data structures and kernel launchers shared by the host code.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace ribn {

constexpr int kPageTokens = 16;   // KV page size (crates/qwen/src/gguf.rs:16)
constexpr int kMaxSplits = 128;   // split-K limit of decode attention
constexpr int kMaxSplitTokens = 512;   // positions one attention workgroup covers

// A quantized matrix after load-time re-tiling: `rows` output rows of `k`
// inputs, GGML row n = input-contiguous. Each GGML block is split into
// 16-byte-aligned planes so every wavefront load is a coalesced 128-bit load:
//   Q4_K: a = qs   [rows][nb][128]   b = scales [rows][nb][16]   c = d|dmin [rows][nb][4]
//         (the twelve packed 6-bit scale/min bytes unpacked to one byte each,
//          dword p = sc(2p), sc(2p+1), m(2p), m(2p+1): the pair lane p reads)
//   Q6_K: a = ql   [rows][nb][128]   b = qh [rows][nb][64]
//         c = sc   [rows][nb][16] reordered: byte 2c+slot holds sub-block scale
//                  s = 8(c/4) + c%4 + 4 slot (the two scales unit c needs)
//         d = d    [rows][nb] (f16)
//   Q8_0: a = qs   [rows][nb][32]    b = d  [rows][nb] (f16)
// The planes hold exactly the GGUF values (no requantization). Q6_K and Q8_0
// keep their block size (210 / 34 bytes); Q4_K grows from 144 to 148 bytes
// per block because its 6-bit scales are stored unpacked.
struct QMat {
    uint32_t type;
    uint32_t rows;
    uint32_t k;
    uint32_t nb;   // blocks per row
    const uint8_t* a;
    const uint8_t* b;
    const uint8_t* c;
    const uint8_t* d;
};

// Per-sequence device state. `pos` is the position of the token the next step
// consumes (tokens[pos]); the step that samples writes tokens[pos + 1].
struct SeqState {
    int32_t pos;
    uint32_t last_token;
    int32_t max_pages;
    int32_t max_ctx;
    int32_t* pages;      // logical page -> physical page
    uint32_t* tokens;    // [max_ctx + 1]
};

// The graphs read the active sequence through this indirection, so one
// captured graph serves every sequence: the host swaps `seq` with a tiny copy.
// The embedding kernel (first of every step) also copies the active
// sequence's position and page-table pointer here, so later kernels of the
// step reach them in one dependent load instead of two.
struct StepCtl {
    SeqState* seq;
    int32_t pos;
    int32_t pad;
    const int32_t* pages;
};

enum MvMode : int32_t {
    MV_STORE = 0,   // out[row] = y (+ bias)
    MV_ADD = 1,     // out[row] += y   (residual epilogue)
    MV_SILU = 2,    // pair (gate, up): out[j] = silu(gate_j) * up_j
    MV_HEAD = 3,    // vocab logits + greedy argmax (token written to the sequence)
};

struct MvSeg {
    QMat w;
    QMat w2;             // MV_SILU: the up matrix (same type/shape as w)
    float* out;
    const float* bias;   // optional per-row bias
    int32_t wg_begin;    // first workgroup of this segment
    int32_t pad;
};

struct HeadEpi {
    uint64_t* partial;      // [n_wg] packed (key, ~index)
    uint32_t* counter;      // arrival counter (left at 0)
};

// One launch of the fused dequant-matvec. Segments 0 and 1 share the value
// type `type_a`; segment 2 may use `type_b` (QKV: attn_v is Q6_K in Q4_K_M).
struct MvArgs {
    const float* x;          // input vector [k]
    const float* norm_w;     // optional RMSNorm weight: x := rms_norm(x) * w
    float eps;
    int32_t k;
    int32_t mode;
    int32_t nseg;
    int32_t items_per_wave;  // item = 2 weight rows (or one gate/up pair)
    uint32_t type_a, type_b;
    MvSeg seg[3];
    HeadEpi head;
    const StepCtl* ctl;
};

// Per-step rotary table: cos/sin of theta_p = pos * base^(-2p/rot) for the
// active sequence's position, written by the embedding kernel.
struct EmbedArgs {
    QMat w;
    int32_t hidden;
    float* h;
    const StepCtl* ctl;
    const float* inv_freq;   // [rot/2] base^(-2p/rot), f32 (powf on the host)
    float* rope;             // [rot]: cos[0..rot/2), sin[rot/2..rot)
    int32_t half_rot;
};

struct AttnArgs {
    const float* raw;        // QKV projection output [hq*hd | hkv*hd | hkv*hd]
    const float* q_norm;     // optional per-head RMSNorm weights [hd]
    const float* k_norm;
    const float* rope;       // EmbedArgs::rope
    uint16_t* kcache;        // [pages][hkv][16][hd] (bf16 or f16)
    uint16_t* vcache;
    float* part;             // split partials [hkv][n_splits][G*hd + 2*G]
    uint32_t* counters;      // [hkv] (left at 0)
    float* out;              // [hq][hd]
    const StepCtl* ctl;
    int32_t hq, hkv, hd, rot, n_splits, kv_f16;
    float eps;
    float scale_log2;        // log2(e) / sqrt(hd)
};

// Launchers (kernels.hip). All enqueue on `stream` and return hipSuccess or the launch error.
hipError_t launch_matvec(const MvArgs& a, int n_wg, hipStream_t stream);
int matvec_rows_per_wg(const MvArgs& a);
size_t matvec_lds_bytes(int k);
hipError_t launch_attention(const AttnArgs& a, hipStream_t stream);
hipError_t launch_embed(const EmbedArgs& a, hipStream_t stream);
hipError_t launch_advance(const StepCtl* ctl, hipStream_t stream);
hipError_t launch_dequant(const QMat& w, float* out, hipStream_t stream);
hipError_t launch_argmax(const float* logits, uint32_t n, uint64_t* partial, uint32_t* counter,
                         uint32_t* out, hipStream_t stream);

}  // namespace ribn
