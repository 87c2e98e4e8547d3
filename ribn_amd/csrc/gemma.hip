// Gemma 4 text decoder on gfx950 behind the reference's GemmaDecode seam
// (crates/gemma4/src/executor/backend.rs:10-33: advance_prefill, prefill,
// decode, position, close), loading a BF16 SafeTensors package the way
// Gemma4Source::open does (crates/gemma4/src/source.rs:56-160) and computing
// the reference's eager BF16 policy (crates/gemma4/src/cpu/): every operation
// in FP32, one BF16 rounding of its result.
//
// The reference CPU decoder is the parity anchor, so the kernels keep its
// arithmetic order instead of reassociating:
//  * projections: one thread per output; its FP32 sum runs over k in ascending
//    order with separately rounded multiplies and adds. Weights are transposed
//    at load ([in][out]) so a wave's loads of one k are contiguous;
//  * norms and softmax totals: sequential sums in one thread;
//  * exp, tanh and pow are evaluated in double and rounded to FP32 once;
//  * rotary factors (cos/sin) are computed on the host with the C library, as
//    the reference does, and uploaded per step.
// The model is small (configs[0]: 41.6 M parameters), so this favours exact
// parity over speed; a step is a few dozen short launches on one stream.
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/ribn_rocm.h"
#include "json.h"

namespace ribn {
namespace {

constexpr int kMaxLayers = 64;
enum { kSliding = 0, kFull = 1 };

struct GemmaConfig {
    int vocab = 0, hidden = 0, intermediate = 0, heads = 0, kv_heads = 0;
    int ple = 0, ple_vocab = 0, context = 0, window = 0, layers = 0;
    float eps = 0.f, softcap = 0.f;
    int kind[kMaxLayers] = {}, head_dim[kMaxLayers] = {}, kv_owner[kMaxLayers] = {}, proportional[kMaxLayers] = {};
    float theta[kMaxLayers] = {};
};

// ---------------------------------------------------------------- device math

__device__ __forceinline__ float ld_bf(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t to_bf(float v) {
    const uint32_t bits = __float_as_uint(v);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float exp_f(float x) { return (float)exp((double)x); }
__device__ __forceinline__ float tanh_f(float x) { return (float)tanh((double)x); }

// Y[r][n] = bf16(sum_k X[r][k] * W[n][k]) with WT = W transposed ([K][N]); one
// thread per output, k ascending (cpu/linear.rs:23-66). X rows are staged in LDS.
__global__ __launch_bounds__(256) void project_kernel(const uint16_t* x, int ldx, const uint16_t* wt, int K, int N,
                                                      uint16_t* y, int ldy) {
    extern __shared__ uint16_t xs[];
    const int r = blockIdx.y, n = blockIdx.x * 256 + threadIdx.x;
    for (int k = threadIdx.x; k < K; k += 256) xs[k] = x[(size_t)r * ldx + k];
    __syncthreads();
    if (n >= N) return;
    float sum = 0.f;
    const uint16_t* w = wt + n;
    int k = 0;
    for (; k + 8 <= K; k += 8) {
        uint16_t wv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) wv[i] = w[(size_t)(k + i) * N];
#pragma unroll
        for (int i = 0; i < 8; i++) sum = __fadd_rn(sum, __fmul_rn(ld_bf(xs[k + i]), ld_bf(wv[i])));
    }
    for (; k < K; k++) sum = __fadd_rn(sum, __fmul_rn(ld_bf(xs[k]), ld_bf(w[(size_t)k * N])));
    y[(size_t)r * ldy + n] = to_bf(sum);
}

typedef unsigned u4v __attribute__((ext_vector_type(4)));

// The same projection for one to four rows, built for latency: workgroup b
// owns output columns [b C, b C + C) of every row. Its 256 threads first copy
// the K x C weight slab and the input rows into LDS as FP32 (exact: BF16 is a
// truncated FP32), every global load in flight at once. The slab is stored
// transposed, K + 1 words per column, so lane c's reads fall on distinct banks.
// Thread (row, c) then forms bf16(sum_k x[row][k] w[k][c]), k ascending with
// separately rounded multiplies and adds: the same sum as project_kernel, bit
// for bit, at two VALU instructions per k. C is a power of two in [8, 64] with
// K C <= 32768 (128 KB of slab); N and K are multiples of 8.
__global__ __launch_bounds__(256) void project_cols_kernel(const uint16_t* x, int ldx, int rows, const uint16_t* wt,
                                                           int K, int N, int C, uint16_t* y, int ldy) {
    extern __shared__ __attribute__((aligned(16))) float ldsf[];
    const int KW = K + 1;                                          // words per column
    float* ws = ldsf;                                              // [C][KW]
    float* xs = ldsf + ((size_t)C * KW + 3) / 4 * 4;               // [rows][K], 16-byte aligned
    const int n0 = blockIdx.x * C, tid = threadIdx.x;
    const int cols = min(C, N - n0);
    const int cpr = C / 8;                    // 16-byte chunks per slab row of the global layout
    const int total = (K / 2) * cpr;          // <= 2048 (K C <= 32768): at most 8 per thread
    u4v v0[8], v1[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const int j = q * 256 + tid;
        const int kp = j / cpr, cc = (j % cpr) * 8;
        v0[q] = v1[q] = u4v{0u, 0u, 0u, 0u};
        if (j < total && cc < cols) {
            v0[q] = *reinterpret_cast<const u4v*>(wt + (size_t)(2 * kp) * N + n0 + cc);
            v1[q] = *reinterpret_cast<const u4v*>(wt + (size_t)(2 * kp + 1) * N + n0 + cc);
        }
    }
    // the input rows: 16-byte chunks of 8 values, at most 8 per thread
    const int xch = rows * (K / 8);
    u4v xv[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const int j = q * 256 + tid;
        xv[q] = j < xch ? *reinterpret_cast<const u4v*>(x + (size_t)(j / (K / 8)) * ldx + (j % (K / 8)) * 8)
                        : u4v{0u, 0u, 0u, 0u};
    }
    auto lo = [](uint32_t w) { return __uint_as_float(w << 16); };
    auto hi = [](uint32_t w) { return __uint_as_float(w & 0xffff0000u); };
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const int j = q * 256 + tid;
        if (j >= total) break;
        const int kp = j / cpr, cc = (j % cpr) * 8;
        const uint32_t a[4] = {v0[q].x, v0[q].y, v0[q].z, v0[q].w}, b[4] = {v1[q].x, v1[q].y, v1[q].z, v1[q].w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float* col = ws + (size_t)(cc + i) * KW + 2 * kp;
            col[0] = (i & 1) ? hi(a[i >> 1]) : lo(a[i >> 1]);
            col[1] = (i & 1) ? hi(b[i >> 1]) : lo(b[i >> 1]);
        }
    }
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const int j = q * 256 + tid;
        if (j < xch) {
            const uint32_t a[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
            float4* dst = reinterpret_cast<float4*>(xs + (size_t)j * 8);
            dst[0] = float4{lo(a[0]), hi(a[0]), lo(a[1]), hi(a[1])};
            dst[1] = float4{lo(a[2]), hi(a[2]), lo(a[3]), hi(a[3])};
        }
    }
    __syncthreads();
    const int r = tid / C, c = tid % C;
    if (r >= rows || c >= cols) return;
    const float4* xr = reinterpret_cast<const float4*>(xs + (size_t)r * K);
    const float* wr = ws + (size_t)c * KW;
    float sum = 0.f;
    for (int k4 = 0; k4 < K / 4; k4++) {
        const float4 xq = xr[k4];
        const float w0 = wr[4 * k4], w1 = wr[4 * k4 + 1], w2 = wr[4 * k4 + 2], w3 = wr[4 * k4 + 3];
        sum = __fadd_rn(sum, __fmul_rn(xq.x, w0));
        sum = __fadd_rn(sum, __fmul_rn(xq.y, w1));
        sum = __fadd_rn(sum, __fmul_rn(xq.z, w2));
        sum = __fadd_rn(sum, __fmul_rn(xq.w, w3));
    }
    y[(size_t)r * ldy + n0 + c] = to_bf(sum);
}

// rms_norm / rms_norm_scale_free (cpu/norm.rs:41-82): one workgroup per row.
// The squares are formed by all threads into LDS (each rounded as the
// reference rounds it); one thread then adds them in index order, reading LDS
// eight at a time, so the energy is the reference's sequential sum.
__global__ __launch_bounds__(256) void rms_kernel(const uint16_t* x, int ldx, int width, float eps,
                                                  const uint16_t* scale, uint16_t* y, int ldy, const int* dpos,
                                                  size_t ypos) {
    extern __shared__ float sq[];
    if (dpos) y += (size_t)*dpos * ypos;   // graph replays: the output row follows the device position   // [width] squares, then the inverse at [width]
    const uint16_t* row = x + (size_t)blockIdx.x * ldx;
    for (int i = threadIdx.x; i < width; i += 256) {
        const float v = ld_bf(row[i]);
        sq[i] = __fmul_rn(v, v);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float e = 0.f;
        int i = 0;
        for (; i + 8 <= width; i += 8) {
            float t[8];
#pragma unroll
            for (int j = 0; j < 8; j++) t[j] = sq[i + j];
#pragma unroll
            for (int j = 0; j < 8; j++) e = __fadd_rn(e, t[j]);
        }
        for (; i < width; i++) e = __fadd_rn(e, sq[i]);
        const float mean = __fdiv_rn(e, (float)width);
        sq[width] = (float)pow((double)__fadd_rn(mean, eps), -0.5);
    }
    __syncthreads();
    const float inv = sq[width];
    for (int i = threadIdx.x; i < width; i += 256) {
        float v = __fmul_rn(ld_bf(row[i]), inv);
        if (scale) v = __fmul_rn(v, ld_bf(scale[i]));
        y[(size_t)blockIdx.x * ldy + i] = to_bf(v);
    }
}

enum EwOp { EW_ADD = 0, EW_MUL = 1, EW_SCALE = 2, EW_GELU = 3, EW_SOFTCAP = 4 };

// elementwise ops with the reference's rounding points (cpu/elementwise.rs)
__global__ __launch_bounds__(256) void elementwise_kernel(int op, const uint16_t* a, const uint16_t* b, size_t n,
                                                          float f, uint16_t* out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float x = ld_bf(a[i]);
    float v;
    if (op == EW_ADD) v = __fadd_rn(x, ld_bf(b[i]));
    else if (op == EW_MUL) v = __fmul_rn(x, ld_bf(b[i]));
    else if (op == EW_SCALE) v = __fmul_rn(x, f);
    else if (op == EW_GELU) {
        const float alpha = 0.7978846f, cubic = 0.044715f;
        const float inner = __fmul_rn(__fmul_rn(alpha, x), __fadd_rn(1.0f, __fmul_rn(__fmul_rn(cubic, x), x)));
        v = __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanh_f(inner)));
    } else {   // soft cap: divide, tanh, multiply, rounded after each
        const float d = ld_bf(to_bf(__fdiv_rn(x, f)));
        const float t = ld_bf(to_bf(tanh_f(d)));
        v = __fmul_rn(t, f);
    }
    out[i] = to_bf(v);
}

// per-layer input: (rms(context) + token identity) / sqrt(2), each step rounded
// (ple_combine, cpu/elementwise.rs:101-107); identity rows have stride ldi
__global__ __launch_bounds__(256) void ple_input_kernel(const uint16_t* ctx, const uint16_t* identity, int ldi, int n,
                                                        int width, uint16_t* out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n * width) return;
    const int r = i / width, j = i % width;
    const float s = ld_bf(to_bf(__fadd_rn(ld_bf(ctx[i]), ld_bf(identity[(size_t)r * ldi + j]))));
    out[i] = to_bf(__fmul_rn(s, 0.70710677f));
}

// token rows of an embedding table times a scale (decoder.rs:348-359)
__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* table, int width, const uint32_t* tokens,
                                                    float scale, uint16_t* out) {
    const uint32_t t = tokens[blockIdx.y];
    for (int i = blockIdx.x * 256 + threadIdx.x; i < width; i += gridDim.x * 256)
        out[(size_t)blockIdx.y * width + i] = to_bf(__fmul_rn(ld_bf(table[(size_t)t * width + i]), scale));
}

// split-half rotary with BF16-rounded products (cpu/rotary.rs:88-134)
__global__ __launch_bounds__(256) void rotary_kernel(const uint16_t* x, int rows, int heads, int width,
                                                     const uint16_t* cs, const uint16_t* sn, uint16_t* y,
                                                     const int* dpos, size_t ypos) {
    if (dpos) y += (size_t)*dpos * ypos;
    const int half = width / 2;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)rows * heads * half) return;
    const int j = (int)(i % half);
    const size_t rh = i / half;
    const int r = (int)(rh / heads);
    const size_t base = rh * width;
    const size_t f = (size_t)r * width + j;
    const float a = ld_bf(x[base + j]), b = ld_bf(x[base + j + half]);
    auto rp = [](float p, float q) { return ld_bf(to_bf(__fmul_rn(p, q))); };
    const float first = __fadd_rn(rp(a, ld_bf(cs[f])), rp(-b, ld_bf(sn[f])));
    const float second = __fadd_rn(rp(b, ld_bf(cs[f + half])), rp(a, ld_bf(sn[f + half])));
    y[base + j] = to_bf(first);
    y[base + j + half] = to_bf(second);
}

// causal / sliding GQA attention (cpu/attention.rs:211-276): one workgroup per
// (query row, head). Scores: per key, columns summed in order, rounded to BF16;
// softmax total summed in key order by one thread; output columns summed in key order.
__global__ __launch_bounds__(256) void attention_kernel(const uint16_t* q, int seq, const uint16_t* keys,
                                                        const uint16_t* values, int kv_seq, int heads, int kv_heads,
                                                        int width, int window, int q_start, uint16_t* out,
                                                        const int* dpos) {
    extern __shared__ float sc[];   // [kv_seq] scores, then weights
    if (dpos) {   // graph replays: the chunk starts at the device position
        q_start = *dpos;
        kv_seq = q_start + seq;
    }
    __shared__ float stat[2];
    const int pos = blockIdx.x, h = blockIdx.y;
    const int kvh = h / (heads / kv_heads);
    const int head_step = heads * width, kv_step = kv_heads * width;
    const int absolute = q_start + pos;
    int last = absolute < kv_seq - 1 ? absolute : kv_seq - 1;
    int first = 0;
    if (window > 0) {
        int a = absolute - (window - 1);
        if (a < 0) a = 0;
        first = a < last ? a : last;
    }
    const uint16_t* qr = q + (size_t)pos * head_step + (size_t)h * width;
    for (int t = first + threadIdx.x; t <= last; t += 256) {
        const uint16_t* kr = keys + (size_t)t * kv_step + (size_t)kvh * width;
        float s = 0.f;
#pragma unroll 8
        for (int i = 0; i < width; i++) s = __fadd_rn(s, __fmul_rn(ld_bf(qr[i]), ld_bf(kr[i])));
        sc[t] = ld_bf(to_bf(s));
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = -INFINITY;
        for (int t = first; t <= last; t++) m = fmaxf(m, sc[t]);
        stat[0] = m;
    }
    __syncthreads();
    for (int t = first + threadIdx.x; t <= last; t += 256) sc[t] = exp_f(__fsub_rn(sc[t], stat[0]));
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.f;
        for (int t = first; t <= last; t++) total = __fadd_rn(total, sc[t]);
        stat[1] = total;
    }
    __syncthreads();
    for (int t = first + threadIdx.x; t <= last; t += 256) sc[t] = ld_bf(to_bf(__fdiv_rn(sc[t], stat[1])));
    __syncthreads();
    for (int i = threadIdx.x; i < width; i += 256) {
        float acc = 0.f;
#pragma unroll 8
        for (int t = first; t <= last; t++)
            acc = __fadd_rn(acc, __fmul_rn(sc[t], ld_bf(values[(size_t)t * kv_step + (size_t)kvh * width + i])));
        out[(size_t)pos * head_step + (size_t)h * width + i] = to_bf(acc);
    }
}

// ---------------------------------------------------------------- host side

uint16_t bf16_host(float v) {
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}
float load_host(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

struct Mat {             // device BF16 matrix; `t` is the transposed copy used by projections
    uint16_t* rows = nullptr;   // [n][k] (embedding gathers) or nullptr
    uint16_t* t = nullptr;      // [k][n]
    int n = 0, k = 0;
};

struct LayerW {
    Mat q, k, v, o, gate, up, down, ple_gate, ple_proj;
    uint16_t *q_norm = nullptr, *k_norm = nullptr, *input_norm = nullptr, *post_attn_norm = nullptr;
    uint16_t *pre_ffn_norm = nullptr, *post_ffn_norm = nullptr, *post_ple_norm = nullptr;
    float layer_scalar = 1.f;
};

}  // namespace
}  // namespace ribn

struct ribn_rocm_gemma {
    ribn::GemmaConfig c;
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<void*> allocs;
    ribn::Mat embed;        // rows = token table, t = output head ([hidden][vocab])
    uint16_t* ple_embed = nullptr;   // [ple_vocab][layers * ple]
    ribn::Mat ple_proj;     // [layers * ple][hidden]
    uint16_t *ple_norm = nullptr, *final_norm = nullptr;
    ribn::LayerW layer[ribn::kMaxLayers];
    uint16_t* keys[ribn::kMaxLayers] = {};
    uint16_t* values[ribn::kMaxLayers] = {};
    int max_rows = 0, position = 0;
    // activations for up to max_rows rows
    uint16_t *hidden, *identity, *projection, *per_layer, *normed, *q, *qn, *attended, *proj, *gate, *up, *down,
        *kbuf, *knbuf, *vbuf, *cosine, *sine, *pg, *logits;
    uint32_t* tokens;
    int maxhd = 0;
    std::vector<uint16_t> host_cs, host_sn;   // [layers][rows][maxhd] rotary factors of the current chunk
    float embed_scale = 0.f, ple_embed_scale = 0.f, ple_projection_scale = 0.f;
    bool faulted = false;
    std::vector<float> inv_freq[ribn::kMaxLayers];
    // graph-replayed decode rows: device position and rotary factors of the row,
    // their pinned host sources, and the captured step
    int* d_pos = nullptr;
    uint16_t* d_rot = nullptr;       // [2][layers][maxhd]: cos, then sin
    uint32_t* h_step = nullptr;      // pinned: token, position
    uint16_t* h_rot = nullptr;       // pinned: as d_rot
    hipGraphExec_t decode_graph = nullptr;
};

namespace ribn {
namespace {

int gfail(char* err, size_t len, const std::string& m, int code) {
    if (err && len) std::snprintf(err, len, "%s", m.c_str());
    return code;
}

#define GCHK(x)                                                                                  \
    do {                                                                                         \
        hipError_t e_ = (x);                                                                     \
        if (e_ != hipSuccess) {                                                                  \
            if (G) G->faulted = true;                                                            \
            return gfail(err, err_len, std::string("HIP error: ") + hipGetErrorString(e_) + " at " #x, \
                         RIBN_ERR_DEVICE);                                                       \
        }                                                                                        \
    } while (0)

hipError_t galloc(ribn_rocm_gemma* G, void** p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 16);
    if (e == hipSuccess) G->allocs.push_back(*p);
    return e;
}
template <typename T>
hipError_t galloc(ribn_rocm_gemma* G, T** p, size_t bytes) {
    return galloc(G, reinterpret_cast<void**>(p), bytes);
}

bool read_file(const std::string& path, std::string& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::ostringstream ss;
    ss << f.rdbuf();
    out = ss.str();
    return true;
}

// ---- config (crates/gemma4/src/config.rs:59-124, 255-380)
bool num(const json::Value* o, const char* k, double& v) {
    const json::Value* x = o ? o->get(k) : nullptr;
    if (!x || !x->is_number()) return false;
    v = x->num;
    return true;
}
bool pos_int(const json::Value* o, const char* k, int& v, std::string& err) {
    double d;
    if (!num(o, k, d) || d < 1 || d != std::floor(d) || d > 1e9) {
        err = std::string(k) + ": expected a positive integer";
        return false;
    }
    v = (int)d;
    return true;
}
bool str_is(const json::Value* o, const char* k, const char* want) {
    const json::Value* x = o ? o->get(k) : nullptr;
    return x && x->kind == json::Value::String && x->str == want;
}
bool bool_is(const json::Value* o, const char* k, bool want) {
    const json::Value* x = o ? o->get(k) : nullptr;
    return x && x->kind == json::Value::Bool && x->b == want;
}

bool parse_config(const json::Value& root, GemmaConfig& c, std::string& err) {
    if (!str_is(&root, "model_type", "gemma4")) { err = "model_type: expected gemma4"; return false; }
    if (!bool_is(&root, "tie_word_embeddings", true)) { err = "tie_word_embeddings: expected true"; return false; }
    if (!str_is(&root, "dtype", "bfloat16")) { err = "dtype: expected bfloat16"; return false; }
    const json::Value* t = root.get("text_config");
    if (!t || t->kind != json::Value::Object) { err = "text_config: missing"; return false; }
    if (!str_is(t, "model_type", "gemma4_text")) { err = "text_config.model_type: expected gemma4_text"; return false; }
    if (!str_is(t, "hidden_activation", "gelu_pytorch_tanh")) { err = "hidden_activation: expected gelu_pytorch_tanh"; return false; }
    for (const char* k : {"attention_bias", "attention_k_eq_v", "enable_moe_block", "use_double_wide_mlp"})
        if (!bool_is(t, k, false)) { err = std::string(k) + ": expected false"; return false; }
    int shared_raw = 0, local_dim = 0, global_dim = 0;
    if (!pos_int(t, "vocab_size", c.vocab, err) || !pos_int(t, "hidden_size", c.hidden, err) ||
        !pos_int(t, "intermediate_size", c.intermediate, err) || !pos_int(t, "num_attention_heads", c.heads, err) ||
        !pos_int(t, "num_key_value_heads", c.kv_heads, err) || !pos_int(t, "hidden_size_per_layer_input", c.ple, err) ||
        !pos_int(t, "vocab_size_per_layer_input", c.ple_vocab, err) ||
        !pos_int(t, "max_position_embeddings", c.context, err) || !pos_int(t, "sliding_window", c.window, err) ||
        !pos_int(t, "num_hidden_layers", c.layers, err) || !pos_int(t, "head_dim", local_dim, err) ||
        !pos_int(t, "global_head_dim", global_dim, err))
        return false;
    double d;
    if (!num(t, "num_kv_shared_layers", d) || d < 0 || d != std::floor(d)) { err = "num_kv_shared_layers: expected an unsigned integer"; return false; }
    shared_raw = (int)d;
    if (!num(t, "rms_norm_eps", d) || !(d > 0)) { err = "rms_norm_eps: must be positive"; return false; }
    c.eps = (float)d;
    if (!num(t, "final_logit_softcapping", d) || !(d > 0)) { err = "final_logit_softcapping: must be positive"; return false; }
    c.softcap = (float)d;
    if (c.layers > kMaxLayers) { err = "num_hidden_layers: more than 64 layers"; return false; }
    if (shared_raw >= c.layers) { err = "num_kv_shared_layers: sharing needs a nonempty owner prefix"; return false; }
    if (local_dim % 2 || global_dim % 8) { err = "head dimensions: local must be even, global divisible by eight"; return false; }
    if (c.heads % c.kv_heads) { err = "num_key_value_heads: must divide query head count"; return false; }
    if (c.context > 16384) { err = "max_position_embeddings: more than 16384 positions"; return false; }
    if (c.ple_vocab < c.vocab) { err = "vocab_size_per_layer_input: must cover every text token ID"; return false; }
    const json::Value* lt = t->get("layer_types");
    if (!lt || lt->kind != json::Value::Array || (int)lt->arr.size() != c.layers) { err = "layer_types: one explicit attention type per layer is required"; return false; }
    for (int i = 0; i < c.layers; i++) {
        const json::Value& v = lt->arr[i];
        if (v.kind == json::Value::String && v.str == "sliding_attention") c.kind[i] = kSliding;
        else if (v.kind == json::Value::String && v.str == "full_attention") c.kind[i] = kFull;
        else { err = "layer_types: unsupported attention"; return false; }
    }
    if (c.kind[c.layers - 1] != kFull) { err = "layer_types: last layer must explicitly be full attention"; return false; }
    const json::Value* rope = t->get("rope_parameters");
    const json::Value* rs = rope ? rope->get("sliding_attention") : nullptr;
    const json::Value* rf = rope ? rope->get("full_attention") : nullptr;
    double th_s, th_f, prf;
    if (!rs || !rf || !str_is(rs, "rope_type", "default") || !str_is(rf, "rope_type", "proportional") ||
        !num(rs, "rope_theta", th_s) || !num(rf, "rope_theta", th_f) || !num(rf, "partial_rotary_factor", prf) ||
        prf != 0.25 || !(th_s > 0) || !(th_f > 0)) {
        err = "rope_parameters: expected default sliding and quarter-proportional full RoPE";
        return false;
    }
    const int owners = c.layers - shared_raw;
    for (int i = 0; i < c.layers; i++) {
        c.head_dim[i] = c.kind[i] == kFull ? global_dim : local_dim;
        c.proportional[i] = c.kind[i] == kFull;
        c.theta[i] = (float)(c.kind[i] == kFull ? th_f : th_s);
        if (i < owners) c.kv_owner[i] = i;
        else {
            int o = -1;
            for (int j = owners - 1; j >= 0; j--)
                if (c.kind[j] == c.kind[i]) { o = j; break; }
            if (o < 0) { err = "KV sharing: tail attention kind has no owner in the prefix"; return false; }
            c.kv_owner[i] = o;
        }
    }
    return true;
}

// ---- SafeTensors package (model.safetensors)
struct TensorRef {
    std::vector<int64_t> shape;
    size_t begin = 0, end = 0;
};

bool parse_safetensors(const std::string& blob, std::map<std::string, TensorRef>& out, size_t& data0, std::string& err) {
    if (blob.size() < 8) { err = "model.safetensors: truncated header"; return false; }
    uint64_t hn = 0;
    std::memcpy(&hn, blob.data(), 8);
    if (hn > blob.size() - 8) { err = "model.safetensors: header length exceeds the file"; return false; }
    json::Value h;
    if (!json::parse(blob.substr(8, hn), h, err)) return false;
    if (h.kind != json::Value::Object) { err = "model.safetensors: header is not an object"; return false; }
    data0 = 8 + hn;
    for (auto& kv : h.obj) {
        if (kv.first == "__metadata__") continue;
        const json::Value& e = kv.second;
        const json::Value* dt = e.get("dtype");
        const json::Value* sh = e.get("shape");
        const json::Value* of = e.get("data_offsets");
        if (!dt || !sh || !of || sh->kind != json::Value::Array || of->kind != json::Value::Array || of->arr.size() != 2) {
            err = kv.first + ": malformed tensor entry";
            return false;
        }
        if (dt->str != "BF16") { err = kv.first + ": expected BF16"; return false; }
        TensorRef r;
        for (auto& s : sh->arr) r.shape.push_back((int64_t)s.num);
        r.begin = (size_t)of->arr[0].num;
        r.end = (size_t)of->arr[1].num;
        if (r.end < r.begin || data0 + r.end > blob.size()) { err = kv.first + ": data outside the file"; return false; }
        out[kv.first] = r;
    }
    return true;
}

std::vector<float> inverse_frequencies(const GemmaConfig& c, int l) {
    // rotary_inverse_frequency (config.rs:217-247), host FP32 powf as the reference
    const int pairs = c.head_dim[l] / 2, active = c.proportional[l] ? pairs / 4 : pairs;
    std::vector<float> f(pairs, 0.f);
    for (int p = 0; p < active; p++) {
        const float e = (float)(p * 2) / (float)c.head_dim[l];
        f[p] = 1.0f / powf(c.theta[l], e);
    }
    return f;
}

}  // namespace
}  // namespace ribn

using namespace ribn;

extern "C" void ribn_rocm_gemma_close(ribn_rocm_gemma* G) {
    if (!G) return;
    hipSetDevice(G->device);
    if (G->stream) hipStreamSynchronize(G->stream);
    if (G->decode_graph) hipGraphExecDestroy(G->decode_graph);
    if (G->h_step) hipHostFree(G->h_step);
    if (G->h_rot) hipHostFree(G->h_rot);
    for (void* p : G->allocs) hipFree(p);
    if (G->stream) hipStreamDestroy(G->stream);
    delete G;
}

extern "C" int ribn_rocm_gemma_open(const char* package_dir, int32_t device, ribn_rocm_gemma** out, char* err,
                                    size_t err_len) {
    ribn_rocm_gemma* G = nullptr;
    if (!package_dir || !out) return gfail(err, err_len, "null argument", RIBN_ERR_INVALID);
    *out = nullptr;
    const std::string dir(package_dir);
    std::string text, blob, msg;
    if (!read_file(dir + "/config.json", text)) return gfail(err, err_len, "cannot read " + dir + "/config.json", RIBN_ERR_IO);
    json::Value root;
    if (!json::parse(text, root, msg)) return gfail(err, err_len, "config.json: " + msg, RIBN_ERR_FORMAT);
    GemmaConfig c;
    if (!parse_config(root, c, msg)) return gfail(err, err_len, "config.json: " + msg, RIBN_ERR_FORMAT);
    if (!read_file(dir + "/model.safetensors", blob))
        return gfail(err, err_len, "cannot read " + dir + "/model.safetensors", RIBN_ERR_IO);
    std::map<std::string, TensorRef> inv;
    size_t data0 = 0;
    if (!parse_safetensors(blob, inv, data0, msg)) return gfail(err, err_len, msg, RIBN_ERR_FORMAT);
    {   // every parameter present with its config shape (parameters.rs:106-160), before any device work
        const int H = c.hidden, P = c.ple, packed = c.layers * c.ple;
        std::vector<std::pair<std::string, std::vector<int64_t>>> specs = {
            {"embed_tokens.weight", {c.vocab, H}}, {"embed_tokens_per_layer.weight", {c.ple_vocab, packed}},
            {"per_layer_model_projection.weight", {packed, H}}, {"per_layer_projection_norm.weight", {P}},
            {"norm.weight", {H}}};
        for (int l = 0; l < c.layers; l++) {
            const std::string lp = "layers." + std::to_string(l) + ".";
            const int hd = c.head_dim[l];
            specs.push_back({lp + "self_attn.q_proj.weight", {c.heads * hd, H}});
            if (c.kv_owner[l] == l) {
                specs.push_back({lp + "self_attn.k_proj.weight", {c.kv_heads * hd, H}});
                specs.push_back({lp + "self_attn.v_proj.weight", {c.kv_heads * hd, H}});
                specs.push_back({lp + "self_attn.k_norm.weight", {hd}});
            }
            specs.push_back({lp + "self_attn.o_proj.weight", {H, c.heads * hd}});
            specs.push_back({lp + "self_attn.q_norm.weight", {hd}});
            for (const char* nm : {"input_layernorm.weight", "post_attention_layernorm.weight",
                                   "pre_feedforward_layernorm.weight", "post_feedforward_layernorm.weight",
                                   "post_per_layer_input_norm.weight"})
                specs.push_back({lp + nm, {H}});
            specs.push_back({lp + "mlp.gate_proj.weight", {c.intermediate, H}});
            specs.push_back({lp + "mlp.up_proj.weight", {c.intermediate, H}});
            specs.push_back({lp + "mlp.down_proj.weight", {H, c.intermediate}});
            specs.push_back({lp + "per_layer_input_gate.weight", {P, H}});
            specs.push_back({lp + "per_layer_projection.weight", {H, P}});
            specs.push_back({lp + "layer_scalar", {1}});
        }
        for (auto& sp : specs) {
            auto it = inv.find("model.language_model." + sp.first);
            if (it == inv.end()) return gfail(err, err_len, "missing model.language_model." + sp.first, RIBN_ERR_FORMAT);
            if (it->second.shape != sp.second)
                return gfail(err, err_len, "model.language_model." + sp.first + ": shape disagrees with the config",
                             RIBN_ERR_FORMAT);
            size_t count = 1;
            for (auto d : sp.second) count *= (size_t)d;
            if (it->second.end - it->second.begin != 2 * count)
                return gfail(err, err_len, "model.language_model." + sp.first + ": byte length disagrees with its shape",
                             RIBN_ERR_FORMAT);
        }
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
        return gfail(err, err_len, "no such HIP device", RIBN_ERR_DEVICE);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess || std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
        return gfail(err, err_len, "device is not gfx950", RIBN_ERR_DEVICE);
    G = new ribn_rocm_gemma();
    G->c = c;
    G->device = device;
    auto bail = [&](int code) {
        ribn_rocm_gemma_close(G);
        return code;
    };
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&G->stream, hipStreamNonBlocking) != hipSuccess)
        return bail(gfail(err, err_len, "cannot create a HIP stream", RIBN_ERR_DEVICE));

    const std::string pre = "model.language_model.";
    // find + shape-check one parameter (parameters.rs:106-160)
    auto find = [&](const std::string& name, std::vector<int64_t> shape, const uint16_t** host) -> bool {
        auto it = inv.find(pre + name);
        if (it == inv.end()) { msg = "missing " + pre + name; return false; }
        if (it->second.shape != shape) { msg = pre + name + ": shape disagrees with the config"; return false; }
        size_t count = 1;
        for (auto s : shape) count *= (size_t)s;
        if (it->second.end - it->second.begin != 2 * count) { msg = pre + name + ": byte length disagrees with its shape"; return false; }
        *host = reinterpret_cast<const uint16_t*>(blob.data() + data0 + it->second.begin);
        return true;
    };
    auto upload = [&](const uint16_t* h, size_t count, uint16_t** d) -> hipError_t {
        hipError_t e = galloc(G, d, 2 * count);
        if (e != hipSuccess) return e;
        return hipMemcpy(*d, h, 2 * count, hipMemcpyHostToDevice);
    };
    // matrix [n][k]: transposed copy for projections, optional row copy
    auto matrix = [&](const std::string& name, int n, int k, bool keep_rows, Mat* m) -> int {
        const uint16_t* h;
        if (!find(name, {n, k}, &h)) return RIBN_ERR_FORMAT;
        std::vector<uint16_t> tr((size_t)n * k);
        for (int i = 0; i < n; i++)
            for (int j = 0; j < k; j++) tr[(size_t)j * n + i] = h[(size_t)i * k + j];
        m->n = n;
        m->k = k;
        if (upload(tr.data(), tr.size(), &m->t) != hipSuccess) return RIBN_ERR_DEVICE;
        if (keep_rows && upload(h, (size_t)n * k, &m->rows) != hipSuccess) return RIBN_ERR_DEVICE;
        return RIBN_OK;
    };
    auto vec = [&](const std::string& name, int n, uint16_t** d) -> int {
        const uint16_t* h;
        if (!find(name, {n}, &h)) return RIBN_ERR_FORMAT;
        return upload(h, (size_t)n, d) == hipSuccess ? RIBN_OK : RIBN_ERR_DEVICE;
    };
    const int H = c.hidden, P = c.ple, packed = c.layers * c.ple;
    int rc = matrix("embed_tokens.weight", c.vocab, H, true, &G->embed);
    if (rc == RIBN_OK) {
        const uint16_t* h;
        rc = find("embed_tokens_per_layer.weight", {c.ple_vocab, packed}, &h) ? RIBN_OK : RIBN_ERR_FORMAT;
        if (rc == RIBN_OK && upload(h, (size_t)c.ple_vocab * packed, &G->ple_embed) != hipSuccess) rc = RIBN_ERR_DEVICE;
    }
    if (rc == RIBN_OK) rc = matrix("per_layer_model_projection.weight", packed, H, false, &G->ple_proj);
    if (rc == RIBN_OK) rc = vec("per_layer_projection_norm.weight", P, &G->ple_norm);
    if (rc == RIBN_OK) rc = vec("norm.weight", H, &G->final_norm);
    for (int l = 0; l < c.layers && rc == RIBN_OK; l++) {
        const std::string lp = "layers." + std::to_string(l) + ".";
        const int hd = c.head_dim[l];
        LayerW& w = G->layer[l];
        rc = matrix(lp + "self_attn.q_proj.weight", c.heads * hd, H, false, &w.q);
        if (rc == RIBN_OK && c.kv_owner[l] == l) {
            rc = matrix(lp + "self_attn.k_proj.weight", c.kv_heads * hd, H, false, &w.k);
            if (rc == RIBN_OK) rc = matrix(lp + "self_attn.v_proj.weight", c.kv_heads * hd, H, false, &w.v);
            if (rc == RIBN_OK) rc = vec(lp + "self_attn.k_norm.weight", hd, &w.k_norm);
        }
        if (rc == RIBN_OK) rc = matrix(lp + "self_attn.o_proj.weight", H, c.heads * hd, false, &w.o);
        if (rc == RIBN_OK) rc = vec(lp + "self_attn.q_norm.weight", hd, &w.q_norm);
        if (rc == RIBN_OK) rc = vec(lp + "input_layernorm.weight", H, &w.input_norm);
        if (rc == RIBN_OK) rc = vec(lp + "post_attention_layernorm.weight", H, &w.post_attn_norm);
        if (rc == RIBN_OK) rc = vec(lp + "pre_feedforward_layernorm.weight", H, &w.pre_ffn_norm);
        if (rc == RIBN_OK) rc = vec(lp + "post_feedforward_layernorm.weight", H, &w.post_ffn_norm);
        if (rc == RIBN_OK) rc = matrix(lp + "mlp.gate_proj.weight", c.intermediate, H, false, &w.gate);
        if (rc == RIBN_OK) rc = matrix(lp + "mlp.up_proj.weight", c.intermediate, H, false, &w.up);
        if (rc == RIBN_OK) rc = matrix(lp + "mlp.down_proj.weight", H, c.intermediate, false, &w.down);
        if (rc == RIBN_OK) rc = matrix(lp + "per_layer_input_gate.weight", P, H, false, &w.ple_gate);
        if (rc == RIBN_OK) rc = matrix(lp + "per_layer_projection.weight", H, P, false, &w.ple_proj);
        if (rc == RIBN_OK) rc = vec(lp + "post_per_layer_input_norm.weight", H, &w.post_ple_norm);
        if (rc == RIBN_OK) {
            const uint16_t* h;
            if (!find(lp + "layer_scalar", {1}, &h)) rc = RIBN_ERR_FORMAT;
            else w.layer_scalar = load_host(h[0]);
        }
        G->inv_freq[l] = inverse_frequencies(c, l);
    }
    if (rc != RIBN_OK) return bail(gfail(err, err_len, rc == RIBN_ERR_FORMAT ? msg : "device allocation failed", rc));

    // caches and activations
    G->max_rows = c.context < 512 ? c.context : 512;
    const size_t R = (size_t)G->max_rows;
    int maxhd = 0;
    for (int l = 0; l < c.layers; l++) maxhd = c.head_dim[l] > maxhd ? c.head_dim[l] : maxhd;
    bool ok = true;
    for (int l = 0; l < c.layers && ok; l++)
        if (c.kv_owner[l] == l) {
            const size_t n = (size_t)c.context * c.kv_heads * c.head_dim[l];
            ok = galloc(G, &G->keys[l], 2 * n) == hipSuccess && galloc(G, &G->values[l], 2 * n) == hipSuccess;
        }
    const size_t qw = (size_t)c.heads * maxhd, kw = (size_t)c.kv_heads * maxhd;
    ok = ok && galloc(G, &G->hidden, 2 * R * H) == hipSuccess && galloc(G, &G->identity, 2 * R * packed) == hipSuccess &&
         galloc(G, &G->projection, 2 * R * packed) == hipSuccess &&
         galloc(G, &G->per_layer, 2 * R * packed) == hipSuccess && galloc(G, &G->normed, 2 * R * H) == hipSuccess &&
         galloc(G, &G->q, 2 * R * qw) == hipSuccess && galloc(G, &G->qn, 2 * R * qw) == hipSuccess &&
         galloc(G, &G->attended, 2 * R * qw) == hipSuccess && galloc(G, &G->proj, 2 * R * H) == hipSuccess &&
         galloc(G, &G->gate, 2 * R * c.intermediate) == hipSuccess &&
         galloc(G, &G->up, 2 * R * c.intermediate) == hipSuccess && galloc(G, &G->down, 2 * R * H) == hipSuccess &&
         galloc(G, &G->kbuf, 2 * R * kw) == hipSuccess && galloc(G, &G->knbuf, 2 * R * kw) == hipSuccess &&
         galloc(G, &G->vbuf, 2 * R * kw) == hipSuccess &&
         galloc(G, &G->cosine, 2 * (size_t)c.layers * R * maxhd) == hipSuccess &&
         galloc(G, &G->sine, 2 * (size_t)c.layers * R * maxhd) == hipSuccess && galloc(G, &G->pg, 2 * R * P) == hipSuccess &&
         galloc(G, &G->logits, 2 * (size_t)c.vocab) == hipSuccess && galloc(G, &G->tokens, 4 * R) == hipSuccess;
    if (!ok) return bail(gfail(err, err_len, "device allocation failed", RIBN_ERR_DEVICE));
    G->maxhd = maxhd;
    // decode rows replay a graph when every score of a row fits the attention kernel's LDS
    if (4 * (size_t)c.context <= 60 * 1024) {
        ok = galloc(G, &G->d_pos, 4) == hipSuccess && galloc(G, &G->d_rot, 2 * 2 * (size_t)c.layers * maxhd) == hipSuccess &&
             hipHostMalloc((void**)&G->h_step, 8, 0) == hipSuccess &&
             hipHostMalloc((void**)&G->h_rot, 2 * 2 * (size_t)c.layers * maxhd, 0) == hipSuccess;
        if (!ok) return bail(gfail(err, err_len, "device allocation failed", RIBN_ERR_DEVICE));
    }
    G->host_cs.assign((size_t)c.layers * R * maxhd, 0);
    G->host_sn.assign((size_t)c.layers * R * maxhd, 0);
    // decoder scales (decoder.rs:78-95)
    G->embed_scale = load_host(bf16_host(std::sqrt((float)H)));
    G->ple_embed_scale = load_host(bf16_host(std::sqrt((float)P)));
    G->ple_projection_scale = 1.0f / std::sqrt((float)H);
    *out = G;
    return RIBN_OK;
}

namespace ribn {
namespace {

hipError_t project(ribn_rocm_gemma* G, const uint16_t* x, int rows, int ldx, const Mat& w, uint16_t* y, int ldy) {
    if (rows <= 4 && w.n % 8 == 0 && w.k % 8 == 0 && w.k <= 4096 && ldx % 8 == 0) {
        int C = 64;
        while (C > 8 && (size_t)w.k * C > 32768) C >>= 1;
        if (rows * C <= 256 && rows * (w.k / 8) <= 2048 && (size_t)w.k * C <= 32768) {
            const size_t lds = ((size_t)C * (w.k + 1) + 3) / 4 * 16 + (size_t)rows * w.k * 4;
            if (lds > 65536) {   // the slab and rows can exceed 64 KB of LDS (per device: every launch)
                const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&project_cols_kernel),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
                if (e != hipSuccess) return e;
            }
            project_cols_kernel<<<(w.n + C - 1) / C, 256, lds, G->stream>>>(x, ldx, rows, w.t, w.k, w.n, C, y, ldy);
            return hipGetLastError();
        }
    }
    const dim3 grid((w.n + 255) / 256, rows);
    project_kernel<<<grid, 256, 2 * (size_t)w.k, G->stream>>>(x, ldx, w.t, w.k, w.n, y, ldy);
    return hipGetLastError();
}
hipError_t rms(ribn_rocm_gemma* G, const uint16_t* x, int rows, int width, int ldx, const uint16_t* scale, uint16_t* y,
               int ldy, const int* dpos = nullptr, size_t ypos = 0) {
    if (width > 16000) return hipErrorInvalidValue;   // squares staged in LDS
    rms_kernel<<<rows, 256, 4 * ((size_t)width + 1), G->stream>>>(x, ldx, width, G->c.eps, scale, y, ldy, dpos, ypos);
    return hipGetLastError();
}
hipError_t ew(ribn_rocm_gemma* G, int op, const uint16_t* a, const uint16_t* b, size_t n, float f, uint16_t* out) {
    elementwise_kernel<<<(unsigned)((n + 255) / 256), 256, 0, G->stream>>>(op, a, b, n, f, out);
    return hipGetLastError();
}

// rotary factors of every layer for positions p0 .. p0 + n - 1, on the host with
// the C library's cosf/sinf as the reference (cpu/rotary.rs:33-81): row r of
// layer l at cs / sn + l * fstride + r * head_dim
void fill_rotary(const ribn_rocm_gemma* G, int p0, int n, uint16_t* cs_all, uint16_t* sn_all, size_t fstride) {
    const GemmaConfig& c = G->c;
    for (int l = 0; l < c.layers; l++) {
        const int hd = c.head_dim[l], half = hd / 2;
        uint16_t* cs = cs_all + (size_t)l * fstride;
        uint16_t* sn = sn_all + (size_t)l * fstride;
        for (int r = 0; r < n; r++) {
            const float position = (float)(p0 + r);
            for (int p = 0; p < half; p++) {
                const float phase = position * G->inv_freq[l][p];
                const uint16_t cb = bf16_host(cosf(phase)), sb = bf16_host(sinf(phase));
                cs[(size_t)r * hd + p] = cs[(size_t)r * hd + p + half] = cb;
                sn[(size_t)r * hd + p] = sn[(size_t)r * hd + p + half] = sb;
            }
        }
    }
}

// The launches of one chunk of n rows (decoder.rs:334-409, 447-626), tokens in
// G->tokens and rotary factors at cos_base / sin_base (layer l at + l * fstride).
// dpos == nullptr: the chunk starts at the host position G->position. Otherwise
// the chunk is one decode row at the position in device memory *dpos (graph
// replays: every launch argument is then the same at every position).
hipError_t chunk_body(ribn_rocm_gemma* G, int n, bool last_logits, const int* dpos, const uint16_t* cos_base,
                      const uint16_t* sin_base, size_t fstride) {
    const GemmaConfig& c = G->c;
    const int H = c.hidden, P = c.ple, packed = c.layers * P, F = c.intermediate;
    const int p0 = dpos ? 0 : G->position;
    hipError_t e;
#define GE(x) do { if ((e = (x)) != hipSuccess) return e; } while (0)
    embed_kernel<<<dim3((H + 255) / 256, n), 256, 0, G->stream>>>(G->embed.rows, H, G->tokens, G->embed_scale, G->hidden);
    GE(hipGetLastError());
    embed_kernel<<<dim3((packed + 255) / 256, n), 256, 0, G->stream>>>(G->ple_embed, packed, G->tokens,
                                                                      G->ple_embed_scale, G->identity);
    GE(hipGetLastError());
    GE(project(G, G->hidden, n, H, G->ple_proj, G->projection, packed));
    GE(ew(G, EW_SCALE, G->projection, nullptr, (size_t)n * packed, G->ple_projection_scale, G->projection));
    // per-layer inputs: rms over each layer's slice, then (context + token) / sqrt(2)
    for (int l = 0; l < c.layers; l++) {
        uint16_t* dst = G->per_layer + (size_t)l * n * P;
        GE(rms(G, G->projection + (size_t)l * P, n, P, packed, G->ple_norm, G->pg, P));
        ple_input_kernel<<<(n * P + 255) / 256, 256, 0, G->stream>>>(G->pg, G->identity + (size_t)l * P, packed, n, P,
                                                                      dst);
        GE(hipGetLastError());
    }
    for (int l = 0; l < c.layers; l++) {
        const LayerW& w = G->layer[l];
        const int hd = c.head_dim[l], half = hd / 2, qw = c.heads * hd, kw = c.kv_heads * hd;
        const uint16_t* cosine = cos_base + (size_t)l * fstride;
        const uint16_t* sine = sin_base + (size_t)l * fstride;
        // attention block (decoder.rs:487-577)
        GE(rms(G, G->hidden, n, H, H, w.input_norm, G->normed, H));
        GE(project(G, G->normed, n, H, w.q, G->q, qw));
        GE(rms(G, G->q, n * c.heads, hd, hd, w.q_norm, G->qn, hd));
        const unsigned rq = (unsigned)(((size_t)n * c.heads * half + 255) / 256);
        rotary_kernel<<<rq, 256, 0, G->stream>>>(G->qn, n, c.heads, hd, cosine, sine, G->q, nullptr, 0);
        GE(hipGetLastError());
        if (c.kv_owner[l] == l) {
            GE(project(G, G->normed, n, H, w.k, G->kbuf, kw));
            GE(rms(G, G->kbuf, n * c.kv_heads, hd, hd, w.k_norm, G->knbuf, hd));
            const unsigned rk = (unsigned)(((size_t)n * c.kv_heads * half + 255) / 256);
            rotary_kernel<<<rk, 256, 0, G->stream>>>(G->knbuf, n, c.kv_heads, hd, cosine, sine,
                                                    G->keys[l] + (size_t)p0 * kw, dpos, (size_t)kw);
            GE(hipGetLastError());
            GE(project(G, G->normed, n, H, w.v, G->vbuf, kw));
            GE(rms(G, G->vbuf, n * c.kv_heads, hd, hd, nullptr, G->values[l] + (size_t)p0 * kw, hd, dpos, (size_t)kw));
        }
        const int owner = c.kv_owner[l];
        // LDS for every score: the chunk's own length, or the whole context for a replayed row
        const int kv_seq = p0 + n, kv_lds = dpos ? c.context : kv_seq;
        attention_kernel<<<dim3(n, c.heads), 256, 4 * (size_t)kv_lds, G->stream>>>(
            G->q, n, G->keys[owner], G->values[owner], kv_seq, c.heads, c.kv_heads, hd,
            c.kind[l] == kSliding ? c.window : 0, p0, G->attended, dpos);
        GE(hipGetLastError());
        GE(project(G, G->attended, n, qw, w.o, G->proj, H));
        GE(rms(G, G->proj, n, H, H, w.post_attn_norm, G->normed, H));
        GE(ew(G, EW_ADD, G->hidden, G->normed, (size_t)n * H, 0.f, G->hidden));
        // feed-forward block and per-layer input gate (decoder.rs:579-626)
        GE(rms(G, G->hidden, n, H, H, w.pre_ffn_norm, G->normed, H));
        GE(project(G, G->normed, n, H, w.gate, G->gate, F));
        GE(project(G, G->normed, n, H, w.up, G->up, F));
        GE(ew(G, EW_GELU, G->gate, nullptr, (size_t)n * F, 0.f, G->gate));
        GE(ew(G, EW_MUL, G->gate, G->up, (size_t)n * F, 0.f, G->gate));
        GE(project(G, G->gate, n, F, w.down, G->down, H));
        GE(rms(G, G->down, n, H, H, w.post_ffn_norm, G->normed, H));
        GE(ew(G, EW_ADD, G->hidden, G->normed, (size_t)n * H, 0.f, G->hidden));
        GE(project(G, G->hidden, n, H, w.ple_gate, G->pg, P));
        GE(ew(G, EW_GELU, G->pg, nullptr, (size_t)n * P, 0.f, G->pg));
        GE(ew(G, EW_MUL, G->pg, G->per_layer + (size_t)l * n * P, (size_t)n * P, 0.f, G->pg));
        GE(project(G, G->pg, n, P, w.ple_proj, G->down, H));
        GE(rms(G, G->down, n, H, H, w.post_ple_norm, G->normed, H));
        GE(ew(G, EW_ADD, G->hidden, G->normed, (size_t)n * H, 0.f, G->hidden));
        GE(ew(G, EW_SCALE, G->hidden, nullptr, (size_t)n * H, w.layer_scalar, G->hidden));
    }
    if (last_logits) {   // project_logits (decoder.rs:411-430): final norm, tied head, soft cap
        GE(rms(G, G->hidden + (size_t)(n - 1) * H, 1, H, H, G->final_norm, G->normed, H));
        GE(project(G, G->normed, 1, H, G->embed, G->logits, c.vocab));
        GE(ew(G, EW_SOFTCAP, G->logits, nullptr, (size_t)c.vocab, c.softcap, G->logits));
    }
#undef GE
    return hipSuccess;
}

// one chunk of at most max_rows rows at the decoder's position, launched directly
int gemma_chunk(ribn_rocm_gemma* G, const uint32_t* tokens, int n, bool last_logits, char* err, size_t err_len) {
    const size_t fstride = (size_t)G->max_rows * G->maxhd;
    GCHK(hipMemcpyAsync(G->tokens, tokens, 4 * (size_t)n, hipMemcpyHostToDevice, G->stream));
    fill_rotary(G, G->position, n, G->host_cs.data(), G->host_sn.data(), fstride);
    GCHK(hipMemcpyAsync(G->cosine, G->host_cs.data(), 2 * G->host_cs.size(), hipMemcpyHostToDevice, G->stream));
    GCHK(hipMemcpyAsync(G->sine, G->host_sn.data(), 2 * G->host_sn.size(), hipMemcpyHostToDevice, G->stream));
    GCHK(chunk_body(G, n, last_logits, nullptr, G->cosine, G->sine, fstride));
    G->position += n;
    return RIBN_OK;
}

bool gemma_eager() {
    static const bool eager = [] {
        const char* v = std::getenv("RIBN_ROCM_EAGER");
        return v && v[0] == '1';
    }();
    return eager;
}

// One decode row replayed from a HIP graph: the token, the position and the
// row's rotary factors go to device memory first (from pinned host memory),
// then the captured launches of chunk_body run with every argument fixed.
int gemma_decode_row(ribn_rocm_gemma* G, uint32_t token, char* err, size_t err_len) {
    const GemmaConfig& c = G->c;
    G->h_step[0] = token;
    G->h_step[1] = (uint32_t)G->position;
    fill_rotary(G, G->position, 1, G->h_rot, G->h_rot + (size_t)c.layers * G->maxhd, (size_t)G->maxhd);
    GCHK(hipMemcpyAsync(G->tokens, &G->h_step[0], 4, hipMemcpyHostToDevice, G->stream));
    GCHK(hipMemcpyAsync(G->d_pos, &G->h_step[1], 4, hipMemcpyHostToDevice, G->stream));
    GCHK(hipMemcpyAsync(G->d_rot, G->h_rot, 2 * 2 * (size_t)c.layers * G->maxhd, hipMemcpyHostToDevice, G->stream));
    if (!G->decode_graph) {
        hipGraph_t g = nullptr;
        GCHK(hipStreamBeginCapture(G->stream, hipStreamCaptureModeThreadLocal));
        const hipError_t e2 = chunk_body(G, 1, true, G->d_pos, G->d_rot, G->d_rot + (size_t)c.layers * G->maxhd,
                                         (size_t)G->maxhd);
        const hipError_t e = hipStreamEndCapture(G->stream, &g);
        if (e2 != hipSuccess) {
            if (g) hipGraphDestroy(g);
            GCHK(e2);
        }
        GCHK(e);
        const hipError_t e3 = hipGraphInstantiate(&G->decode_graph, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        GCHK(e3);
    }
    GCHK(hipGraphLaunch(G->decode_graph, G->stream));
    G->position += 1;
    return RIBN_OK;
}

int gemma_step(ribn_rocm_gemma* G, const uint32_t* tokens, uint32_t n, uint16_t* logits, char* err, size_t err_len) {
    if (!G) return gfail(err, err_len, "null handle", RIBN_ERR_INVALID);
    if (G->faulted) return gfail(err, err_len, "ROCm Gemma decoder is faulted", RIBN_ERR_FAULTED);
    const GemmaConfig& c = G->c;
    // step (decoder.rs:129-192): reject empty, overlong or out-of-range chunks without state change
    if (!tokens || n == 0 || (uint64_t)G->position + n > (uint64_t)c.context)
        return gfail(err, err_len, "empty, overlong or out-of-range token chunk", RIBN_ERR_INVALID);
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)c.vocab)
            return gfail(err, err_len, "empty, overlong or out-of-range token chunk", RIBN_ERR_INVALID);
    GCHK(hipSetDevice(G->device));
    if (n == 1 && logits && G->d_pos && !gemma_eager()) {
        int rc = gemma_decode_row(G, tokens[0], err, err_len);
        if (rc != RIBN_OK) return rc;
        GCHK(hipMemcpyAsync(logits, G->logits, 2 * (size_t)c.vocab, hipMemcpyDeviceToHost, G->stream));
        GCHK(hipStreamSynchronize(G->stream));
        return RIBN_OK;
    }
    // rows beyond max_rows run as consecutive sub-chunks (prefill equals serial)
    for (uint32_t done = 0; done < n;) {
        const int m = (int)std::min<uint32_t>(n - done, (uint32_t)G->max_rows);
        const bool last = done + m == n;
        int rc = gemma_chunk(G, tokens + done, m, last && logits != nullptr, err, err_len);
        if (rc != RIBN_OK) return rc;
        done += m;
    }
    if (logits) GCHK(hipMemcpyAsync(logits, G->logits, 2 * (size_t)c.vocab, hipMemcpyDeviceToHost, G->stream));
    GCHK(hipStreamSynchronize(G->stream));
    return RIBN_OK;
}

}  // namespace
}  // namespace ribn

extern "C" int ribn_rocm_gemma_info(const ribn_rocm_gemma* G, ribn_rocm_gemma_info_t* out) {
    if (!G || !out) return RIBN_ERR_INVALID;
    out->vocab = (uint32_t)G->c.vocab;
    out->hidden = (uint32_t)G->c.hidden;
    out->layers = (uint32_t)G->c.layers;
    out->context = (uint32_t)G->c.context;
    return RIBN_OK;
}

extern "C" int ribn_rocm_gemma_prefill(ribn_rocm_gemma* G, const uint32_t* tokens, uint32_t n, uint16_t* logits,
                                       char* err, size_t err_len) {
    if (!logits) return gfail(err, err_len, "null logits buffer", RIBN_ERR_INVALID);
    return gemma_step(G, tokens, n, logits, err, err_len);
}

extern "C" int ribn_rocm_gemma_advance_prefill(ribn_rocm_gemma* G, const uint32_t* tokens, uint32_t n, char* err,
                                               size_t err_len) {
    return gemma_step(G, tokens, n, nullptr, err, err_len);
}

extern "C" int ribn_rocm_gemma_decode(ribn_rocm_gemma* G, uint32_t token, uint16_t* logits, char* err,
                                      size_t err_len) {
    if (!logits) return gfail(err, err_len, "null logits buffer", RIBN_ERR_INVALID);
    return gemma_step(G, &token, 1, logits, err, err_len);
}

extern "C" uint32_t ribn_rocm_gemma_position(const ribn_rocm_gemma* G) { return G ? (uint32_t)G->position : 0u; }

extern "C" int ribn_rocm_gemma_reset(ribn_rocm_gemma* G) {
    if (!G) return RIBN_ERR_INVALID;
    G->position = 0;
    return RIBN_OK;
}
