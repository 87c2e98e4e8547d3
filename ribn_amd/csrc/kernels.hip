// Hand-written HIP kernels for gfx950 (CDNA4, wave64) on ribn's decode path.
//
// Decode at batch 1 streams every weight once per token, so the matvec is the
// hot path and it is HBM-bound. Design:
//  * weights stay in their GGUF block encoding, re-tiled at load into
//    16-byte-aligned planes (kernels.h, QMat) so each lane issues 128-bit
//    non-temporal loads and a wave reads 1 KiB of contiguous quants;
//  * the input vector is staged once per workgroup in LDS in 16-bit fixed point
//    (one fp32 scale per 64 values, two signed bytes per value), and the quants
//    meet it in v_dot4_i32_i8 with exact int32 accumulation; per-16 fp32 sums
//    of x carry the Q4_K minimum and the Q6_K offset terms;
//  * RMSNorm is a workgroup prologue; residual add, SwiGLU and the vocab argmax
//    are epilogues; q/k head norm, NeoX rope and the KV append live in the
//    attention prologue, so one layer is 5 launches.
// Reference semantics followed: gguf_gemv (nvidia/src/qwen_reference.rs:31-40),
// rms_norm_raw (:550-556), rope (:406-425), attention (:431-461), ffn (:529-539),
// argmax (nvidia/src/model_ops.rs:203-260), dequant (gguf/src/lib.rs:577-649).
#include <algorithm>

#include "matvec.h"

namespace ribn {
namespace {

__global__ __launch_bounds__(kThreads) void dequant_kernel(QMat w, float* out) {
    size_t idx = (size_t)blockIdx.x * kThreads + threadIdx.x;
    size_t total = (size_t)w.rows * w.k;
    if (idx >= total) return;
    out[idx] = deq_elem(w, (uint32_t)(idx / w.k), (uint32_t)(idx % w.k));
}

// Rows of w dequantized exactly and rounded to binary16 (RNE): out[r][e] for
// r < w.rows, row stride w.k (the resident-weight GEMM operands).
__global__ __launch_bounds__(kThreads) void dequant_f16_kernel(QMat w, uint16_t* out) {
    const size_t idx = (size_t)blockIdx.x * kThreads + threadIdx.x;
    const size_t total = (size_t)w.rows * w.k;
    if (idx >= total) return;
    const float v = deq_elem(w, (uint32_t)(idx / w.k), (uint32_t)(idx % w.k));
    out[idx] = __half_as_ushort(__float2half_rn(v));
}

// Token embedding: one row of token_embd dequantized exactly
// (q4_k_embedding, kernels/quantized/q4_k.cu:1; reference decode.rs:577-582),
// plus the step's rotary table: theta_p = pos * base^(-2p/rot) in f32 and its
// sin/cos (qwen_reference.rs:406-425), shared by every layer of the step.
__global__ __launch_bounds__(kThreads) void embed_kernel(EmbedArgs a) {
    const SeqState* s = a.ctl->seq;
    const int pos = s->pos;
    const uint32_t tok = s->tokens[pos];
    const int e = blockIdx.x * kThreads + threadIdx.x;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        StepCtl* c = const_cast<StepCtl*>(a.ctl);
        c->pos = pos;
        c->pages = s->pages;
    }
    if (e < a.hidden) a.h[e] = deq_elem(a.w, tok, (uint32_t)e);
    if (blockIdx.x == 0 && (int)threadIdx.x < a.half_rot) {
        const float theta = (float)pos * a.inv_freq[threadIdx.x];
        a.rope[threadIdx.x] = cosf(theta);
        a.rope[a.half_rot + threadIdx.x] = sinf(theta);
    }
}

__global__ void advance_kernel(const StepCtl* ctl) {
    if (threadIdx.x == 0) ctl->seq->pos += 1;
}



template <int HD, int G, bool F16>
__global__ __launch_bounds__(kThreads) void attention_kernel(AttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    attention_item<HD, G, F16, false>(a, blockIdx.x, blockIdx.y, a.ctl->pos, a.ctl->pages, lds, NoSync{});
}

// Standalone greedy argmax (model_ops.rs:203-260) used by tests.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* logits, uint32_t n, uint64_t* partial,
                                                          uint32_t* counter, uint32_t* out) {
    __shared__ uint64_t wbest[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t b = 0ull;
    for (uint32_t i = blockIdx.x * kThreads + tid; i < n; i += gridDim.x * kThreads) b = max(b, argmax_key(logits[i], i));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) b = max(b, (uint64_t)__shfl_xor(b, o));
    if (lane == 0) wbest[wave] = b;
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < kWaves; i++) wbest[0] = max(wbest[0], wbest[i]);
        st_agent(partial + blockIdx.x, wbest[0]);
    }
    if (!arrive_last(counter, gridDim.x)) return;
    b = 0ull;
    for (int i = tid; i < (int)gridDim.x; i += kThreads) b = max(b, ld_agent(partial + i));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) b = max(b, (uint64_t)__shfl_xor(b, o));
    __syncthreads();
    if (lane == 0) wbest[wave] = b;
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < kWaves; i++) wbest[0] = max(wbest[0], wbest[i]);
        *out = wbest[0] ? 0xffffffffu - (uint32_t)(wbest[0] & 0xffffffffu) : 0u;
    }
}

template <int HD, int G, bool F16>
__global__ __launch_bounds__(kThreads) void attention_rows_kernel(AttnArgs a, DecodeRows r) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int row = blockIdx.z;
    const int ns = rows_splits(r.pos[row] + 1, r.split_tokens);
    if ((int)blockIdx.x >= ns) return;   // a shorter row uses fewer splits
    AttnArgs ar = a;
    ar.n_splits = ns;
    ar.raw = r.raw + (size_t)row * r.ld_raw;
    ar.out = r.out + (size_t)row * r.ld_out;
    ar.rope = r.rope + (size_t)row * a.rot;
    ar.part = r.part + (size_t)row * r.part_stride;
    ar.counters = r.counters + (size_t)row * a.hkv;
    attention_item<HD, G, F16, false>(ar, blockIdx.x, blockIdx.y, r.pos[row], r.pages + (size_t)r.slot[row] * r.max_pages,
                                      lds, NoSync{});
}

__global__ __launch_bounds__(kThreads) void rope_rows_kernel(const float* inv_freq, int half, DecodeRows r) {
    const int row = blockIdx.x;
    const float pos = (float)r.pos[row];
    for (int p = threadIdx.x; p < half; p += kThreads) {
        const float theta = pos * inv_freq[p];
        r.rope[(size_t)row * 2 * half + p] = cosf(theta);
        r.rope[(size_t)row * 2 * half + half + p] = sinf(theta);
    }
}

__global__ void gather_row_tokens_kernel(const uint32_t* tokens, int ld, DecodeRows r, uint32_t* out) {
    const int row = blockIdx.x * 64 + threadIdx.x;
    if (row < r.rows) out[row] = tokens[(size_t)r.slot[row] * ld + r.pos[row]];
}

// Greedy argmax of each row of logits in two launches: workgroup (c, row) keeps
// the best key of chunk c of the row (kArgChunks chunks, all loads of a thread
// issued together), then one wave per row reduces the chunk keys and commits the
// token (first maximum, NaN skipped: the packed key orders by value, then by
// lowest index).
constexpr int kArgChunks = 64;
__global__ __launch_bounds__(256) void rows_argmax_part_kernel(const float* logits, int V, uint64_t* part) {
    __shared__ uint64_t wbest[4];
    const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* lg = logits + (size_t)row * V;
    const int per = (V + kArgChunks - 1) / kArgChunks;
    const int lo = c * per, hi = min(V, lo + per);
    uint64_t b = 0ull;
#pragma unroll 4
    for (int i = lo + tid; i < hi; i += 256) b = max(b, argmax_key(lg[i], (uint32_t)i));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) b = max(b, (uint64_t)__shfl_xor(b, o));
    if (lane == 0) wbest[wave] = b;
    __syncthreads();
    if (tid == 0) part[(size_t)row * kArgChunks + c] = max(max(wbest[0], wbest[1]), max(wbest[2], wbest[3]));
}

__global__ __launch_bounds__(64) void rows_argmax_commit_kernel(const uint64_t* part, DecodeRows r, SeqState* slots) {
    const int row = blockIdx.x, lane = threadIdx.x;
    uint64_t b = part[(size_t)row * kArgChunks + lane];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) b = max(b, (uint64_t)__shfl_xor(b, o));
    if (lane == 0) {
        const uint32_t tok = b ? 0xffffffffu - (uint32_t)(b & 0xffffffffu) : 0u;
        SeqState* s = &slots[r.slot[row]];
        const int pos = r.pos[row];
        if (pos + 1 <= s->max_ctx) s->tokens[pos + 1] = tok;
        s->last_token = tok;
        s->pos = pos + 1;
    }
}

template <int HD, int G, bool F16>
hipError_t attention_rows_launch(const AttnArgs& a, const DecodeRows& r, hipStream_t st) {
    constexpr size_t lds = sizeof(AttnLds<HD, G>);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_rows_kernel<HD, G, F16>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    attention_rows_kernel<HD, G, F16><<<dim3(a.n_splits, a.hkv, r.rows), kThreads, lds, st>>>(a, r);
    return hipGetLastError();
}

template <int HD, bool F16>
hipError_t attention_rows_dispatch(const AttnArgs& a, const DecodeRows& r, hipStream_t st) {
    switch (a.hq / a.hkv) {
    case 1: return attention_rows_launch<HD, 1, F16>(a, r, st);
    case 2: return attention_rows_launch<HD, 2, F16>(a, r, st);
    case 3: return attention_rows_launch<HD, 3, F16>(a, r, st);
    case 4: return attention_rows_launch<HD, 4, F16>(a, r, st);
    case 5: return attention_rows_launch<HD, 5, F16>(a, r, st);
    case 6: return attention_rows_launch<HD, 6, F16>(a, r, st);
    case 7: return attention_rows_launch<HD, 7, F16>(a, r, st);
    case 8: return attention_rows_launch<HD, 8, F16>(a, r, st);
    default: return hipErrorInvalidValue;
    }
}

template <int HD, int G, bool F16>
hipError_t attention_launch(const AttnArgs& a, hipStream_t st) {
    constexpr size_t lds = sizeof(AttnLds<HD, G>);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<HD, G, F16>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    attention_kernel<HD, G, F16><<<dim3(a.n_splits, a.hkv), kThreads, lds, st>>>(a);
    return hipGetLastError();
}

template <int HD, bool F16>
hipError_t attention_dispatch(const AttnArgs& a, hipStream_t st) {
    switch (a.hq / a.hkv) {
    case 1: return attention_launch<HD, 1, F16>(a, st);
    case 2: return attention_launch<HD, 2, F16>(a, st);
    case 3: return attention_launch<HD, 3, F16>(a, st);
    case 4: return attention_launch<HD, 4, F16>(a, st);
    case 5: return attention_launch<HD, 5, F16>(a, st);
    case 6: return attention_launch<HD, 6, F16>(a, st);
    case 7: return attention_launch<HD, 7, F16>(a, st);
    case 8: return attention_launch<HD, 8, F16>(a, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

size_t matvec_lds_bytes(int k, int rows) { return (size_t)std::max(rows, 1) * mv_red_offset(k) + 64 * 4; }

constexpr size_t kLdsBytes = 160 * 1024;

int matvec_max_rows(int k) {
    int r = kMvMaxRows;
    while (r > 1 && matvec_lds_bytes(k, r) > kLdsBytes) r--;
    return r;
}

int matvec_rows_per_wg(const MvArgs& a) { return a.items_per_wave * mv_waves(a) * (a.mode == MV_SILU ? 1 : 2); }

hipError_t launch_matvec(const MvArgs& a, int n_wg, hipStream_t st) {
    if (n_wg <= 0 || a.k <= 0 || a.k % 16) return hipErrorInvalidValue;
    if (a.waves != 0 && a.waves != 4 && a.waves != 8) return hipErrorInvalidValue;
    for (int i = 0; i < a.nseg; i++)   // per-row addends are held one per lane (mv_addend)
        if ((a.mode == MV_ADD || a.seg[i].bias) && a.seg[i].ipw > 32) return hipErrorInvalidValue;
    if (a.parts && (a.mode != MV_ADD || a.parts_splits < 2 || a.parts_splits > kDeferMaxSplits || a.parts_g < 1 ||
                    a.parts_hd < 16 || a.parts_hd % 16 || a.k % (a.parts_hd * a.parts_g)))
        return hipErrorInvalidValue;
    if (a.rows > 1) {
        if (a.rows > matvec_max_rows(a.k) || a.parts || a.ldx < a.k) return hipErrorInvalidValue;
        return launch_matvec_rows(a, n_wg, st);
    }
    switch (a.mode) {
    case MV_STORE: return matvec_dispatch<MV_STORE>(a, n_wg, st);
    case MV_ADD: return a.parts ? matvec_dispatch<MV_ADD_MERGED>(a, n_wg, st) : matvec_dispatch<MV_ADD>(a, n_wg, st);
    case MV_SILU: return matvec_dispatch<MV_SILU>(a, n_wg, st);
    case MV_HEAD: return matvec_dispatch<MV_HEAD>(a, n_wg, st);
    default: return hipErrorInvalidValue;
    }
}

// Merge of a long context's split partials (AttnArgs::defer == 2), one wave per
// query head: lane s holds split s's statistics (m_s, l_s), every lane DPL
// output dims. out[h][d] = sum_s w_s o_s[d] / sum_s w_s l_s with
// w_s = 2^(m_s - max m) (0 for an empty split): the log-sum-exp merge of the
// attention launch's own, with all of a head's partial loads in flight at once
// and the query heads spread over many waves instead of one workgroup per KV head.
template <int DPL, int MAXS>
__global__ __launch_bounds__(256) void attention_merge_kernel(const float* part, int ns, int G, int hkv, float* out) {
    constexpr int HD = 64 * DPL;
    const int wv = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (wv >= hkv * G) return;   // wave-uniform
    const int j = wv / G, gg = wv % G, rec = G * HD + 2 * G;
    const float* kv = part + (size_t)j * ns * rec;
    const int sl = min(lane, ns - 1);
    const float m = lane < ns ? kv[(size_t)sl * rec + G * HD + gg] : -INFINITY;
    const float l = lane < ns ? kv[(size_t)sl * rec + G * HD + G + gg] : 0.f;
    float o[MAXS][DPL];
#pragma unroll
    for (int s = 0; s < MAXS; s++) {
        const float* src = kv + (size_t)min(s, ns - 1) * rec + gg * HD + lane * DPL;
#pragma unroll
        for (int i = 0; i < DPL; i++) o[s][i] = src[i];
    }
    const float mx = wave_max(m);
    const float w = m == -INFINITY ? 0.f : exp2f(m - mx);
    const float den = wave_sum(w * l);
    float acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; i++) acc[i] = 0.f;
#pragma unroll
    for (int s = 0; s < MAXS; s++) {
        const float ws = __shfl(w, s);   // 0 for s >= ns
#pragma unroll
        for (int i = 0; i < DPL; i++) acc[i] = fmaf(ws, o[s][i], acc[i]);
    }
    const float inv = 1.0f / den;
#pragma unroll
    for (int i = 0; i < DPL; i++) out[(size_t)wv * HD + lane * DPL + i] = acc[i] * inv;
}

hipError_t launch_matvec_clocked(const MvArgs& a, int n_wg, unsigned long long* clk, hipStream_t st) {
    if (a.mode != MV_SILU || n_wg < 1 || !clk) return hipErrorInvalidValue;
    const size_t lds = matvec_lds_bytes(a.k, 1);
#define RIBN_MVC(A)                                                                                              \
    if (a.type_a == A) {                                                                                         \
        if (lds > 65536) {                                                                                       \
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&matvec_clocked_kernel<A, A, MV_SILU>), \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);           \
            if (e != hipSuccess) return e;                                                                       \
        }                                                                                                        \
        matvec_clocked_kernel<A, A, MV_SILU><<<n_wg, mv_waves(a) * 64, lds, st>>>(a, clk);                       \
        return hipGetLastError();                                                                                \
    }
    RIBN_MVC(12) RIBN_MVC(14) RIBN_MVC(8)
#undef RIBN_MVC
    return hipErrorInvalidValue;
}

hipError_t launch_attention_merge(const AttnArgs& a, hipStream_t st) {
    const int G = a.hq / a.hkv, ns = a.n_splits;
    if (ns <= kDeferMaxSplits || ns > kMergeMaxSplits || a.hkv < 1 || a.hq % a.hkv) return hipErrorInvalidValue;
    const dim3 grid((a.hq + 3) / 4);
#define RIBN_MERGE(D)                                                                                             \
    if (a.hd == 64 * D) {                                                                                         \
        if (ns <= 16) attention_merge_kernel<D, 16><<<grid, 256, 0, st>>>(a.part, ns, G, a.hkv, a.out);          \
        else if (ns <= 32) attention_merge_kernel<D, 32><<<grid, 256, 0, st>>>(a.part, ns, G, a.hkv, a.out);     \
        else attention_merge_kernel<D, 64><<<grid, 256, 0, st>>>(a.part, ns, G, a.hkv, a.out);                   \
        return hipGetLastError();                                                                                 \
    }
    RIBN_MERGE(1) RIBN_MERGE(2)
#undef RIBN_MERGE
    return hipErrorInvalidValue;
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
    if (a.n_splits < 1 || a.n_splits > kMaxSplits || a.hkv < 1 || a.hq % a.hkv || a.rot > a.hd || a.rot % 2)
        return hipErrorInvalidValue;
    if (a.defer == 1 && a.n_splits > kDeferMaxSplits) return hipErrorInvalidValue;
    if (a.defer == 2 && (a.n_splits <= kDeferMaxSplits || a.n_splits > kMergeMaxSplits || (a.hd != 64 && a.hd != 128)))
        return hipErrorInvalidValue;
    if (a.hd == 128) return a.kv_f16 ? attention_dispatch<128, true>(a, st) : attention_dispatch<128, false>(a, st);
    if (a.hd == 64) return a.kv_f16 ? attention_dispatch<64, true>(a, st) : attention_dispatch<64, false>(a, st);
    if (a.hd == 256) return a.kv_f16 ? attention_dispatch<256, true>(a, st) : attention_dispatch<256, false>(a, st);
    return hipErrorInvalidValue;
}

hipError_t launch_attention_rows(const AttnArgs& a, const DecodeRows& r, hipStream_t st) {
    if (r.rows < 1 || a.n_splits < 1 || a.n_splits > kMaxSplits || a.hkv < 1 || a.hq % a.hkv || a.rot > a.hd ||
        a.rot % 2)
        return hipErrorInvalidValue;
    if (a.hd == 128) return a.kv_f16 ? attention_rows_dispatch<128, true>(a, r, st) : attention_rows_dispatch<128, false>(a, r, st);
    if (a.hd == 64) return a.kv_f16 ? attention_rows_dispatch<64, true>(a, r, st) : attention_rows_dispatch<64, false>(a, r, st);
    return hipErrorInvalidValue;
}

hipError_t launch_rope_rows(const float* inv_freq, int rot, const DecodeRows& r, hipStream_t st) {
    rope_rows_kernel<<<r.rows, kThreads, 0, st>>>(inv_freq, rot / 2, r);
    return hipGetLastError();
}

hipError_t launch_gather_row_tokens(const uint32_t* tokens, int ld, const DecodeRows& r, uint32_t* out,
                                    hipStream_t st) {
    gather_row_tokens_kernel<<<(r.rows + 63) / 64, 64, 0, st>>>(tokens, ld, r, out);
    return hipGetLastError();
}

hipError_t launch_rows_argmax_commit(const float* logits, int V, const DecodeRows& r, SeqState* slots,
                                     uint64_t* part, hipStream_t st) {
    static_assert(kArgChunks == 64, "one lane per chunk in the commit kernel");
    rows_argmax_part_kernel<<<dim3(kArgChunks, r.rows), 256, 0, st>>>(logits, V, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    rows_argmax_commit_kernel<<<r.rows, 64, 0, st>>>(part, r, slots);
    return hipGetLastError();
}

hipError_t launch_embed(const EmbedArgs& a, hipStream_t st) {
    if (a.half_rot > kThreads) return hipErrorInvalidValue;
    embed_kernel<<<(a.hidden + kThreads - 1) / kThreads, kThreads, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_advance(const StepCtl* ctl, hipStream_t st) {
    advance_kernel<<<1, 64, 0, st>>>(ctl);
    return hipGetLastError();
}

hipError_t launch_dequant_f16(const QMat& w, uint16_t* out, hipStream_t st) {
    const size_t total = (size_t)w.rows * w.k;
    if (total == 0) return hipSuccess;
    dequant_f16_kernel<<<(unsigned)((total + kThreads - 1) / kThreads), kThreads, 0, st>>>(w, out);
    return hipGetLastError();
}

hipError_t launch_dequant(const QMat& w, float* out, hipStream_t st) {
    const size_t total = (size_t)w.rows * w.k;
    dequant_kernel<<<(unsigned)((total + kThreads - 1) / kThreads), kThreads, 0, st>>>(w, out);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, uint32_t n, uint64_t* partial, uint32_t* counter, uint32_t* out,
                         hipStream_t st) {
    unsigned blocks = (n + kThreads * 8 - 1) / (kThreads * 8);
    if (blocks < 1) blocks = 1;
    if (blocks > 1024) blocks = 1024;
    argmax_kernel<<<blocks, kThreads, 0, st>>>(logits, n, partial, counter, out);
    return hipGetLastError();
}

}  // namespace ribn
