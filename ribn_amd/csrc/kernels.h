// Device data structures and kernel launchers shared by the host code.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace ribn {

constexpr int kPageTokens = 16;   // KV page size (crates/qwen/src/gguf.rs:16)
constexpr int kMaxSplits = 512;   // split-K limit of decode attention

// A quantized matrix after load-time re-tiling: `rows` output rows of `k`
// inputs, GGML row n = input-contiguous. Each GGML block is split into
// 16-byte-aligned planes so every wavefront load is a coalesced 128-bit load:
//   Q4_K: a = qs   [rows][nb][128]   b = head [rows][nb][16] (d, dmin, 12 scale bytes)
//   Q6_K: a = ql   [rows][nb][128]   b = qh [rows][nb][64]
//         c = sc   [rows][nb][16]    d = d  [rows][nb] (f16)
//   Q8_0: a = qs   [rows][nb][32]    b = d  [rows][nb] (f16)
// The planes hold exactly the GGUF bytes (no requantization): bytes per block
// are unchanged (144 / 210 / 34).
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
struct StepCtl {
    SeqState* seq;
};

enum MvMode : int32_t {
    MV_STORE = 0,   // out[row] = y (+ bias)
    MV_ADD = 1,     // out[row] += y   (residual epilogue)
    MV_SILU = 2,    // pair (gate, up): out[j] = silu(gate_j) * up_j
    MV_QKV = 3,     // q/k/v projection with head epilogue (norm, rope, KV append)
    MV_HEAD = 4,    // vocab logits + greedy argmax
};

struct MvSeg {
    QMat w;
    QMat w2;             // MV_SILU: the up matrix (same type/shape as w)
    float* out;
    const float* bias;   // optional per-row bias
    int32_t wg_begin;    // first workgroup of this segment
    int32_t kind;        // MV_QKV: 0 = q, 1 = k, 2 = v
};

struct QkvEpi {
    float* raw;             // [q_dim + 2*kv_dim] projection outputs (+bias)
    float* q_out;           // [hq][hd] after norm + rope
    uint16_t* kcache;       // layer K cache [pages][hkv][16][hd] (bf16 or f16)
    uint16_t* vcache;
    const float* q_norm;    // optional [hd]
    const float* k_norm;
    uint32_t* counters;     // [hq + hkv] per-head arrival counters (left at 0)
    int32_t hq, hkv, hd, rot;
    float rope_base, eps;
    int32_t kv_f16;         // cache element: 0 = bf16, 1 = binary16
};

struct HeadEpi {
    uint64_t* partial;      // [n_wg] packed (key, ~index)
    uint32_t* counter;      // arrival counter (left at 0)
};

struct MvArgs {
    const float* x;          // input vector [k]
    const float* norm_w;     // optional RMSNorm weight: x := rms_norm(x) * w
    float eps;
    int32_t k;
    int32_t mode;
    int32_t nseg;
    int32_t items_per_wave;  // item = 2 weight rows (or one gate/up pair)
    MvSeg seg[3];
    QkvEpi qkv;
    HeadEpi head;
    const StepCtl* ctl;
};

struct AttnArgs {
    const float* q;          // [hq][hd] (normed, roped)
    const uint16_t* kcache;  // [pages][hkv][16][hd] bf16
    const uint16_t* vcache;
    float* part;             // [hq][n_splits][hd + 2]
    uint32_t* counters;      // [hkv] (left at 0)
    float* out;              // [hq][hd]
    const StepCtl* ctl;
    int32_t hq, hkv, hd, n_splits;
    float scale_log2;        // log2(e) / sqrt(hd)
    int32_t kv_f16;          // cache element: 0 = bf16, 1 = binary16
};

// Launchers (kernels.hip). All enqueue on `stream` and return hipSuccess or the launch error.
hipError_t launch_matvec(const MvArgs& a, int n_wg, hipStream_t stream);
int matvec_rows_per_wg(const MvArgs& a);
size_t matvec_lds_bytes(int k);
hipError_t launch_attention(const AttnArgs& a, hipStream_t stream);
hipError_t launch_embed(const QMat& w, int hidden, float* h, const StepCtl* ctl, hipStream_t stream);
hipError_t launch_advance(const StepCtl* ctl, hipStream_t stream);
hipError_t launch_dequant(const QMat& w, float* out, hipStream_t stream);
hipError_t launch_argmax(const float* logits, uint32_t n, uint64_t* partial, uint32_t* counter,
                         uint32_t* out, hipStream_t stream);

}  // namespace ribn
