// Device data structures and kernel launchers shared by the host code.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace ribn {

constexpr int kPageTokens = 16;   // KV page size (crates/qwen/src/gguf.rs:16)
constexpr int kMaxSplits = 128;   // split-K limit of decode attention
constexpr int kMaxSplitTokens = 2048;   // positions one attention workgroup covers

// Decode-attention splits for a context of `ctx` positions, a power of two
// (measured on MI355X for head_dim 64 and 128, 1 to 8 query heads per KV head):
// one workgroup up to 128 positions; at least 4 and about 128 positions each up
// to 2048; about 256 each up to 8192 and beyond that at least 32 splits of at
// most about 1024 positions, at most kMaxSplits
// (a split then covers at most kMaxSplitTokens positions for contexts up to
// kMaxSplits * kMaxSplitTokens).
__host__ __device__ inline int splits_for_ctx(int ctx) {
    if (ctx <= 128) return 1;
    const int per = ctx <= 2048 ? 128 : ctx <= 8192 ? 256 : 1024;
    const int want = (ctx + per - 1) / per;
    // beyond 8192 positions at least 32 splits (16K: 18.8 us against 25.6 us at
    // 16 splits for the 32B shape with the separate merge launch)
    int s = ctx <= 8192 ? 4 : 32;
    while (s < want && s < kMaxSplits) s <<= 1;
    return s;
}

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
    // Q4_K / Q6_K, optional: the GEMM-ordered copy read by the dequantizing GEMM
    // (one block of kGemmBlkQ4 / kGemmBlkQ6 bytes per 16-row group and 128-wide
    // K tile, each lane's fragment bytes contiguous; layout in gemm_pack, model.hip)
    const uint8_t* g;
};
constexpr size_t kGemmBlkQ4 = 1216, kGemmBlkQ6 = 1696;

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
    float* rec;          // hybrid models: the active sequence's recurrent state (else null)
};

enum MvMode : int32_t {
    MV_STORE = 0,   // out[row] = y (+ bias)
    MV_ADD = 1,     // out[row] += y   (residual epilogue)
    MV_SILU = 2,    // pair (gate, up): out[j] = silu(gate_j) * up_j
    MV_HEAD = 3,    // vocab logits + greedy argmax (token written to the sequence)
    MV_ADD_MERGED = 4,   // kernel variant of MV_ADD chosen for MvArgs::parts (not a host mode)
};

struct MvSeg {
    QMat w;
    QMat w2;             // MV_SILU: the up matrix (same type/shape as w)
    float* out;
    const float* res;    // MV_ADD: residual input, out[row] = res[row] + y (res == out: in place)
    const float* bias;   // optional per-row bias
    int32_t wg_begin;    // first workgroup of this segment
    int32_t ipw;         // items per wave in this segment
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
    int32_t items_per_wave;  // default items per wave (item = 2 weight rows, or one gate/up pair)
    int32_t waves;           // waves per workgroup of a standalone launch: 4 (0 means 4) or 8
    uint32_t type_a, type_b;
    MvSeg seg[3];
    HeadEpi head;
    const StepCtl* ctl;
    // MV_ADD only, optional: x is the merge of decode attention's split partials
    // (AttnArgs::defer), records [hkv][parts_splits][parts_g * parts_hd + 2 parts_g]
    const float* parts;
    int32_t parts_splits, parts_g, parts_hd;
    // rows > 1 (up to kMvMaxRows; MV_STORE, MV_ADD, MV_SILU): that many input rows
    // ldx floats apart, outputs and residuals ldo floats apart, each weight
    // loaded once for all rows; 0 or 1: one row
    int32_t rows, ldx, ldo;
};
constexpr int kMvMaxRows = 4;

// Largest split count whose partials the attention-output projection merges
// itself (AttnArgs::defer); beyond it the attention launch merges them.
constexpr int kDeferMaxSplits = 8;
// Largest split count the separate merge launch takes (one split per lane).
constexpr int kMergeMaxSplits = 64;

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
    int32_t defer;           // 1 (1 < n_splits <= kDeferMaxSplits): leave the split partials in `part`, the
                             // output in binary16, for the next matvec (MvArgs::parts) to merge;
                             // 2 (kDeferMaxSplits < n_splits <= kMergeMaxSplits): leave them (fp32) for
                             // attention_merge_kernel; 0: the attention launch merges them itself
    float eps;
    float scale_log2;        // log2(e) / sqrt(hd)
};

// Persistent decode step: one launch runs a whole token step (embedding, every
// layer, head) with grid-wide barriers between dependent stages. Every stage
// writes a buffer of its own in a per-step arena, so no buffer is written after
// any workgroup has read it within a launch.
struct LayerDev {
    MvArgs qkv, o, gu, down;   // laid out for the persistent grid
    AttnArgs attn;             // n_splits is chosen in the kernel from the context
};

// Bytes of the persistent step's barrier state: 18 words spaced 64 words
// (256 bytes) apart, rounded up (layout in step.h).
constexpr int kStepBarWords = 64 * 18;
constexpr size_t kStepBarBytes = 8192;
static_assert(kStepBarWords * 4 <= (int)kStepBarBytes, "barrier state larger than its allocation");

struct StepArgs {
    const LayerDev* layers;
    int32_t n_layers;
    int32_t head;              // 1: final norm + head + argmax; 0: advance the position only
    EmbedArgs embed;           // embed.h = arena h0
    MvArgs head_mv;
    uint32_t* bar;             // grid barrier state: kStepBarBytes, zeroed at load (layout in step.h)
    uint64_t timeout_ticks;    // barrier wait limit in wall-clock ticks
    const StepCtl* ctl;
    uint64_t* stamps;          // optional: workgroup 0's wall clock at start and after each stage
};

// Chunked prefill (prefill.hip). One GEMM launch over up to three weight
// matrices (segments) sharing the input: Y[M][col0 + n] (row stride ldy) =
// X[M][k] deq(W)^T (+ bias[n]) for the w.rows rows of each segment; X is
// binary16. Segments 0 and 1 share a value type; tile0 = the segment's first
// 128-row tile (0, then cumulative).
struct PrefillSeg {
    QMat w;
    int col0, tile0;
    const float* bias;   // optional [w.rows]
};
struct PrefillGemm {
    const uint16_t* x;   // [m][k] binary16
    int m, k;
    float* y;
    int ldy;
    const float* res;    // MV_ADD: y = res + x w^T (res may be y)
    int mode;            // MV_STORE or MV_ADD
    int nseg;
    PrefillSeg seg[3];
    // split-K: ksplit > 1 splits the K tiles over blockIdx.z; split z writes its
    // partial sums (split 0 with the bias) to part + z m ldy, and a fixed-order
    // reduction then writes y = (res) + sum of the partials
    int ksplit;
    float* part;
    // optional step fused after the result (into the split-K reduction when
    // there is one, else a separate launch), per output row r:
    //   GEMM_POST_RMS_F16:  post_out[r][i] = f16(rms_norm(y[r]) * post_w[i]), y written too
    //   GEMM_POST_SILU_F16: y[r] = gate | up halves of ldy / 2 columns;
    //                       post_out[r][j] = f16(silu(gate) * up), y not written when split
    int post;
    const float* post_w;
    float post_eps;
    uint16_t* post_out;
};
constexpr int GEMM_POST_NONE = 0, GEMM_POST_RMS_F16 = 1, GEMM_POST_SILU_F16 = 2;

// Rows of one prefill chunk at positions pos0 .. pos0 + m - 1.
struct PrefillRows {
    const float* qkv;    // [m][ld_qkv]: q | k | v projections
    int ld_qkv;
    float* qout;         // [m][hq * hd] q after norm and rope
    uint16_t* attn16;    // [m][hq * hd] attention output, binary16
    int m, pos0;
    int hq, hkv, hd, rot, kv_f16;
    const float* q_norm;
    const float* k_norm;
    const float* inv_freq;
    float eps;
    const int32_t* pages;
    uint16_t* kcache;
    uint16_t* vcache;
};

constexpr int kGemmTileN = 128;   // weight rows per prefill-GEMM workgroup
inline int gemm_tiles(int rows) { return (rows + kGemmTileN - 1) / kGemmTileN; }
size_t prefill_gemm_lds_bytes();
// split count launch_prefill_gemm would use for this GEMM (partials need ksplit * m * ldy floats)
int prefill_gemm_splits(int m, int k, int n_tiles);
hipError_t launch_prefill_gemm(const PrefillGemm& g, hipStream_t stream);
hipError_t launch_rows_rms_f16(const float* x, int m, int k, const float* w, float eps, bool norm, uint16_t* out,
                               int ldo, hipStream_t stream);
hipError_t launch_embed_rows(const QMat& w, const uint32_t* tokens, int m, int hidden, float* h, hipStream_t stream);
hipError_t launch_qk_rope_append(const PrefillRows& p, hipStream_t stream);
hipError_t launch_prefill_attention(const PrefillRows& p, hipStream_t stream);
hipError_t launch_silu_mul_f16(const float* gu, int f, int m, uint16_t* act, hipStream_t stream);
hipError_t launch_set_pos(SeqState* s, int pos, hipStream_t stream);

// Gated-DeltaNet block of a qwen35 hybrid layer (hybrid.hip), between the
// segmented input matvec (mixed | z | beta_raw, alpha_raw) and ssm_out. Channel
// layout of `mixed` / `act`: q heads [hk][d], k heads [hk][d], v heads [hv][d].
// Recurrent state of the active sequence at ctl->rec: this layer's delta-rule
// matrices at state_off ([hv][d rows = key][d cols = value]) and its
// convolution history at conv_off ([channels][conv_k - 1], oldest first).
struct GdnArgs {
    const float* mixed;
    const float* z;          // [hv][d]
    const float* ba;         // [hv] beta_raw, then [hv] alpha_raw
    const float* dt_bias;    // [hv]
    const float* ssm_a;      // [hv], already -exp(A_log)
    const float* conv_w;     // [channels][conv_k]
    const float* ssm_norm;   // [d]
    float* act;              // [channels]: conv + SiLU, q/k heads l2-normalized
    float* gated;            // [hv][d] gated-norm output, ssm_out's input
    const StepCtl* ctl;
    size_t state_off, conv_off;
    int hk, hv, d, conv_k;
    float eps;
};
hipError_t launch_gdn(const GdnArgs& a, hipStream_t stream);
// x[i] *= sigmoid(gate[i]) (the gated full-attention output gate)
hipError_t launch_gate_mul(float* x, const float* gate, int n, hipStream_t stream);

// Launchers (kernels.hip). All enqueue on `stream` and return hipSuccess or the launch error.
hipError_t launch_matvec(const MvArgs& a, int n_wg, hipStream_t stream);
// launch_matvec's rows > 1 case (matvec_rows.hip), after its checks
hipError_t launch_matvec_rows(const MvArgs& a, int n_wg, hipStream_t stream);
int matvec_rows_per_wg(const MvArgs& a);
size_t matvec_lds_bytes(int k, int rows = 1);
// Most input rows one matvec launch takes for inputs of k values (staged rows
// must fit the 160 KB of LDS), at most kMvMaxRows.
int matvec_max_rows(int k);
hipError_t launch_attention(const AttnArgs& a, hipStream_t stream);
hipError_t launch_attention_merge(const AttnArgs& a, hipStream_t stream);
// Timing variant of a gate/up (MV_SILU) matvec launch: also folds the launch's
// first workgroup start and last workgroup end (wall-clock ticks) into clk[0]
// (atomic min; start it at UINT64_MAX) and clk[1] (atomic max; start it at 0).
hipError_t launch_matvec_clocked(const MvArgs& a, int n_wg, unsigned long long* clk, hipStream_t stream);

// Batched decode: one decode row per sequence, all in one step. Row r consumes
// the token at position pos[r] of the sequence in slot slot[r]; its page table
// is pages + slot[r] * max_pages.
struct DecodeRows {
    int rows;
    const int32_t* slot;
    const int32_t* pos;
    const int32_t* pages;      // [slots][max_pages]
    int max_pages;
    const float* raw;          // [rows][ld_raw] q | k | v projections
    int ld_raw;
    float* out;                // [rows][ld_out] attention output
    int ld_out;
    float* rope;               // [rows][rot] cos | sin of each row's position
    float* part;               // [rows][part_stride] split partials
    size_t part_stride;
    uint32_t* counters;        // [rows][hkv] (left at 0)
    int split_tokens;          // positions per split: a row splits its context into
                               // rows_splits(ctx, split_tokens) parts
};
// power of two >= ctx / split_tokens, at most kMaxSplits
__host__ __device__ inline int rows_splits(int ctx, int split_tokens) {
    int s = 1;
    while (s * split_tokens < ctx && s < kMaxSplits) s <<= 1;
    return s;
}
// decode attention (split-K over each row's own cache; base carries the layer's
// weights, caches and n_splits); grid splits x hkv x rows
hipError_t launch_attention_rows(const AttnArgs& base, const DecodeRows& r, hipStream_t stream);
// rope[r] = cos | sin of pos[r] * inv_freq
hipError_t launch_rope_rows(const float* inv_freq, int rot, const DecodeRows& r, hipStream_t stream);
// token of each row: tokens[slot[r] * ld + pos[r]]
hipError_t launch_gather_row_tokens(const uint32_t* tokens, int ld, const DecodeRows& r, uint32_t* out,
                                    hipStream_t stream);
// greedy argmax of each row of logits [rows][V] (first maximum, NaN skipped), written as the
// next token of the row's sequence: tokens[pos + 1], last_token, and pos advanced by one
// (part: [rows][64] scratch keys)
hipError_t launch_rows_argmax_commit(const float* logits, int V, const DecodeRows& r, SeqState* slots,
                                     uint64_t* part, hipStream_t stream);
hipError_t launch_embed(const EmbedArgs& a, hipStream_t stream);
hipError_t launch_advance(const StepCtl* ctl, hipStream_t stream);
hipError_t launch_dequant(const QMat& w, float* out, hipStream_t stream);
hipError_t launch_dequant_f16(const QMat& w, uint16_t* out, hipStream_t stream);

// Plain binary16 GEMM on hipBLASLt for resident dequantized weights:
// y[m][ldy] (+)= x[m][k] w16[n][k]^T (+ bias[n]), FP32 output and accumulation.
struct BlasGemm;
hipError_t blas_create(BlasGemm** out, hipStream_t stream);
void blas_destroy(BlasGemm* b);
hipError_t blas_gemm(BlasGemm* b, const uint16_t* x, int m, int k, const uint16_t* w16, int n, float* y, int ldy,
                     bool add, const float* bias, hipStream_t stream);
// A compiled configuration of the persistent step kernel: matrix value types
// (q/k, v, attn_output, gate/up, down, head), head dimension, query heads per
// KV head, KV element type.
struct StepKey {
    int qa, qb, o, gu, dn, ht, hd, g, kv_f16;
};
// Workgroups of the step kernel for `key` that fit on the device at once (0:
// no compiled kernel for this configuration); *lds receives its LDS bytes.
int step_grid(const StepKey& key, int max_k, int device, size_t* lds);
hipError_t launch_step(const StepArgs& a, const StepKey& key, int n_wg, size_t lds, hipStream_t stream);
hipError_t launch_argmax(const float* logits, uint32_t n, uint64_t* partial, uint32_t* counter,
                         uint32_t* out, hipStream_t stream);

// ---------------------------------------------------------------------------
// Integer-dot projections (the reference's GemvMode::IntegerDot): inputs packed
// as Q8_1 (per 32 values: word half(d) | half(sum) << 16, then 32 signed bytes
// q = round(x / d), d = max|x| / 127), weights read once for up to
// kIdMaxMembers packed inputs.
constexpr int kIdMaxMembers = 8;
struct IdArgs {
    const uint32_t* xq;     // [members][k/32 * 9] Q8_1 words
    int32_t k;
    int32_t members;        // 1 .. kIdMaxMembers
    int32_t ld;             // output / residual row stride (floats) between members
    int32_t mode;           // MV_STORE (+ bias), MV_ADD or MV_SILU
    int32_t nseg;
    int32_t items_per_wave;
    uint32_t type_a, type_b;   // segments 0, 1: type_a; segment 2: type_b
    MvSeg seg[3];           // out / res / bias of member m at + m * ld
};
// Grid size of the launch after laying the segments out over n_cu compute units.
int intdot_layout(IdArgs& a, int n_cu);
hipError_t launch_intdot(const IdArgs& a, int n_wg, hipStream_t stream);
// Q8_1 words of `rows` rows of k values (k % 32 == 0): x row r at x + r * ldx,
// words of row r at out + r * (k / 32) * 9. With norm_w, each row is first
// RMS-normalized: x * (1 / sqrt(mean(x^2) + eps)) * w.
hipError_t launch_q8_1_rows(const float* x, int ldx, int rows, int k, const float* norm_w, float eps, uint32_t* out,
                            hipStream_t stream);
// Q8_1 words of n values (n % 32 == 0) as one flat vector.
hipError_t launch_quantize_q8_1(const float* x, size_t n, uint32_t* out, hipStream_t stream);

}  // namespace ribn
