// Chunked prefill: the prompt's rows run through every layer together, so each
// weight matrix is read once per chunk and the projections are dense GEMMs on
// the matrix cores (prefill_chunk / run_prefill_chunk, nvidia/src/decode.rs:2124,
// 2360; the reference batches 8 rows through warp GEMVs, this build uses MFMA).
//
//  * prefill_gemm: Y[M][N] = X[M][K] deq(W)^T. X is binary16 (the RMSNorm'd or
//    activation rows), W stays in its GGUF planes and each 256-wide K slice of a
//    128-row tile is dequantized (exactly as dequantize_block, then rounded to
//    binary16) into LDS; v_mfma_f32_16x16x32_f16 accumulates in fp32.
//  * rows_rms_f16, embed_rows, qk_rope_append, prefill_attention, silu_mul_f16:
//    the per-row steps around the GEMMs, same equations as the decode kernels.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "kernels.h"
#include "lanes.h"

namespace ribn {
namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef unsigned u4v_t __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
constexpr int kTileM = 128;   // chunk rows per workgroup
constexpr int kTileN = 128;   // weight rows per workgroup
constexpr int kTileK = 128;   // half a Q4_K / Q6_K super-block, four Q8_0 blocks
#ifndef RIBN_PG_PAD
#define RIBN_PG_PAD 8
#endif
#ifndef RIBN_PG_REMAP
#define RIBN_PG_REMAP 0
#endif
#ifndef RIBN_PG_DEPTH
#define RIBN_PG_DEPTH 1
#endif
constexpr int kLdsRow = kTileK + RIBN_PG_PAD;   // halves per LDS row (padded against bank conflicts)

__device__ __forceinline__ float h2f_bits(uint32_t b) { return __half2float(__ushort_as_half((unsigned short)(b & 0xffffu))); }
__device__ __forceinline__ float canon(uint32_t b) {
    const float v = h2f_bits(b);
    return v != v ? __uint_as_float(0x7fc00000u) : v;
}
__device__ __forceinline__ uint16_t f2h_bits(float f) { return __half_as_ushort(__float2half_rn(f)); }

// Dequantize 64 consecutive values of one weight row into LDS as binary16:
// values [128 kt + 64 q, +64) of the row (kt = 128-wide K tile, q = quarter of
// it), computed exactly as dequantize_block (gguf/src/lib.rs:584-649) and then
// rounded to binary16.
// The bytes of one quarter are fetched into registers one K tile ahead
// (QuarterRaw<T>::fetch) and converted into LDS when that tile is staged
// (QuarterRaw<T>::convert), so the weight loads are in flight during the MFMA
// phase of the previous tile.
template <int T>
struct QuarterRaw;

__device__ __forceinline__ void store16(uint16_t* dst, const uint32_t (&o)[8]) {
    u4v_t* out = reinterpret_cast<u4v_t*>(dst);
    out[0] = u4v_t{o[0], o[1], o[2], o[3]};
    out[1] = u4v_t{o[4], o[5], o[6], o[7]};
}
__device__ __forceinline__ uint32_t lane_of(const u4v_t& v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; }

template <>
struct QuarterRaw<12> {
    // group pair p = 2 (kt % 2) + q of block kt / 2: group 2p = low nibbles of qs
    // bytes 32p..32p+31, group 2p+1 = their high nibbles; scale dword p holds
    // sc(2p), sc(2p+1), m(2p), m(2p+1)
    uint32_t dd, s;
    u4v_t qv[2];
    __device__ __forceinline__ void fetch(const QMat& w, size_t row, int kt, int q) {
        const size_t bi = row * w.nb + (kt >> 1);
        const int p = 2 * (kt & 1) + q;
        dd = *reinterpret_cast<const uint32_t*>(w.c + bi * 4);
        s = reinterpret_cast<const uint32_t*>(w.b + bi * 16)[p];
        const u4v_t* qs = reinterpret_cast<const u4v_t*>(w.a + bi * 128 + 32 * p);
        qv[0] = qs[0];
        qv[1] = qs[1];
    }
    __device__ __forceinline__ void convert(uint16_t* dst) const {
        const float d = canon(dd), dmin = canon(dd >> 16);
        const float g0 = __fmul_rn(d, (float)(s & 0xffu)), g1 = __fmul_rn(d, (float)((s >> 8) & 0xffu));
        const float m0 = __fmul_rn(dmin, (float)((s >> 16) & 0xffu)), m1 = __fmul_rn(dmin, (float)(s >> 24));
#pragma unroll
        for (int c = 0; c < 2; c++) {
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t v = lane_of(qv[c], j);
                uint32_t a[4], bb[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    a[e] = f2h_bits(__fsub_rn(__fmul_rn(g0, (float)((v >> (8 * e)) & 15u)), m0));
                    bb[e] = f2h_bits(__fsub_rn(__fmul_rn(g1, (float)((v >> (8 * e + 4)) & 15u)), m1));
                }
                lo[2 * j] = a[0] | (a[1] << 16);
                lo[2 * j + 1] = a[2] | (a[3] << 16);
                hi[2 * j] = bb[0] | (bb[1] << 16);
                hi[2 * j + 1] = bb[2] | (bb[3] << 16);
            }
            store16(dst + 16 * c, lo);
            store16(dst + 32 + 16 * c, hi);
        }
    }
};

template <>
struct QuarterRaw<14> {
    // chunk h = kt % 2 of block kt / 2 (ql bytes 64h.., qh bytes 32h..); value
    // 32v + l of the chunk: ((ql[32 (v%2) + l] >> 4 (v/2)) & 15) | (((qh[l] >> 2v) & 3) << 4),
    // minus 32, times d * sc(8h + 2v + l/16); the quarter q holds v = 2q, 2q + 1.
    // Sub-block scale s sits at c-plane byte 2c + slot, c = 4 (s/8) + s%4, slot = (s/4) % 2.
    uint32_t d16, sc4;   // d; the quarter's four sub-block scales (int8, order vv * 2 + lc)
    int q;
    u4v_t ql[4], qh[2];
    __device__ __forceinline__ void fetch(const QMat& w, size_t row, int kt, int qq) {
        const size_t bi = row * w.nb + (kt >> 1);
        const int h = kt & 1;
        q = qq;
        d16 = *reinterpret_cast<const uint16_t*>(w.d + bi * 2);
        const uint8_t* sp = w.c + bi * 16;
        sc4 = 0;
#pragma unroll
        for (int vv = 0; vv < 2; vv++)
#pragma unroll
            for (int lc = 0; lc < 2; lc++) {
                const int sb = 8 * h + 2 * (2 * qq + vv) + lc;
                sc4 |= (uint32_t)sp[2 * (4 * (sb / 8) + sb % 4) + (sb / 4) % 2] << (8 * (2 * vv + lc));
            }
        const u4v_t* ql4 = reinterpret_cast<const u4v_t*>(w.a + bi * 128 + 64 * h);
        const u4v_t* qh4 = reinterpret_cast<const u4v_t*>(w.b + bi * 64 + 32 * h);
#pragma unroll
        for (int i = 0; i < 4; i++) ql[i] = ql4[i];
        qh[0] = qh4[0];
        qh[1] = qh4[1];
    }
    __device__ __forceinline__ void convert(uint16_t* dst) const {
        const float d = canon(d16);
#pragma unroll
        for (int vv = 0; vv < 2; vv++) {
            const int v = 2 * q + vv;
#pragma unroll
            for (int lc = 0; lc < 2; lc++) {
                const float gsc = __fmul_rn(d, (float)(int8_t)(sc4 >> (8 * (2 * vv + lc))));
                const u4v_t qlv = ql[2 * vv + lc], qhv = qh[lc];
                uint32_t o[8];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t lw = lane_of(qlv, j), hw = lane_of(qhv, j);
                    uint32_t e[4];
#pragma unroll
                    for (int b = 0; b < 4; b++) {
                        const int qq = (int)((((lw >> (8 * b)) >> (4 * q)) & 15u) | ((((hw >> (8 * b)) >> (2 * v)) & 3u) << 4)) - 32;
                        e[b] = f2h_bits(__fmul_rn(gsc, (float)qq));
                    }
                    o[2 * j] = e[0] | (e[1] << 16);
                    o[2 * j + 1] = e[2] | (e[3] << 16);
                }
                store16(dst + 32 * vv + 16 * lc, o);
            }
        }
    }
};

template <>
struct QuarterRaw<8> {
    // Q8_0 blocks 4 kt + 2q and 4 kt + 2q + 1; past the row's end (k % 128 != 0): zeros
    uint32_t d16[2];
    u4v_t qv[2][2];
    bool present[2];
    __device__ __forceinline__ void fetch(const QMat& w, size_t row, int kt, int q) {
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int qb = 4 * kt + 2 * q + b;
            present[b] = qb < (int)w.nb;
            d16[b] = 0u;
            qv[b][0] = qv[b][1] = u4v_t{0u, 0u, 0u, 0u};
            if (present[b]) {
                const size_t bi = row * w.nb + (size_t)qb;
                d16[b] = *reinterpret_cast<const uint16_t*>(w.b + bi * 2);
                const u4v_t* qs = reinterpret_cast<const u4v_t*>(w.a + bi * 32);
                qv[b][0] = qs[0];
                qv[b][1] = qs[1];
            }
        }
    }
    __device__ __forceinline__ void convert(uint16_t* dst) const {
#pragma unroll
        for (int b = 0; b < 2; b++) {
            uint32_t o[2][8];
            const float d = canon(d16[b]);
#pragma unroll
            for (int c = 0; c < 2; c++) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t v = lane_of(qv[b][c], j);
                    uint32_t e[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) e[k] = present[b] ? f2h_bits(__fmul_rn(d, (float)(int8_t)(v >> (8 * k)))) : 0u;
                    o[c][2 * j] = e[0] | (e[1] << 16);
                    o[c][2 * j + 1] = e[2] | (e[3] << 16);
                }
            }
            store16(dst + 32 * b, o[0]);
            store16(dst + 32 * b + 16, o[1]);
        }
    }
};

// Workgroup tile: 128 chunk rows x 128 weight rows of one segment; wave w owns
// weight rows 32w..32w+31 of the tile (two 16-column MFMA blocks) for all 128
// chunk rows (eight 16-row blocks): 16 accumulators of 4 floats. K runs in
// tiles of 128 (X slice and dequantized W slice in LDS, 70 KB: two workgroups
// per CU, so one stages while the other multiplies).
// MFMA 16x16x32 f16 operand layout (lane l): A[m = l%16][k = 8(l/16) .. +8],
// B[k = 8(l/16) .. +8][n = l%16]; result C[m = 4(l/16) + i][n = l%16], i < 4.
// MT (128 or 32) is the workgroup's chunk rows: 32 for batched decode rows,
// where a 128-row tile would mostly multiply padding.
template <int TA, int TB, int MT>
__global__ __launch_bounds__(kGemmThreads) void prefill_gemm_kernel(PrefillGemm g) {
    constexpr int MB = MT / 16;                // 16-row MFMA blocks
    constexpr int XR = MT * 16 / kGemmThreads; // X chunks per thread per K tile
    extern __shared__ __attribute__((aligned(16))) uint16_t plds[];
    uint16_t* xs = plds;                       // [MT][kLdsRow]
    uint16_t* ws = plds + MT * kLdsRow;        // [kTileN][kLdsRow]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int si = 0;
    if (g.nseg > 1 && (int)blockIdx.x >= g.seg[1].tile0) si = 1;
    if (g.nseg > 2 && (int)blockIdx.x >= g.seg[2].tile0) si = 2;
    const PrefillSeg sg = g.seg[si];
    const int m0 = blockIdx.y * MT, n0 = ((int)blockIdx.x - sg.tile0) * kTileN;
    const int n_rows = (int)sg.w.rows;
    f4_t acc[MB][2];
#pragma unroll
    for (int i = 0; i < MB; i++) {
        acc[i][0] = f4_t{0.f, 0.f, 0.f, 0.f};
        acc[i][1] = f4_t{0.f, 0.f, 0.f, 0.f};
    }
    const int n_kt = (g.k + kTileK - 1) / kTileK;
    const int ks = max(1, g.ksplit), z = blockIdx.z;
    const int kt0 = (int)((long)n_kt * z / ks), kt1 = (int)((long)n_kt * (z + 1) / ks);
    // dequant: row of the tile, quarter of the K tile
    const int wr = RIBN_PG_REMAP ? 32 * wave + (lane & 31) : tid >> 1, wq = RIBN_PG_REMAP ? lane >> 5 : tid & 1;
    const size_t wrow = (size_t)min(n0 + wr, n_rows - 1);
    const bool use_b = si == 2 && TB != TA;
    // K tiles in flight in registers: X slice (128 rows x 128 halves = 2048
    // 16-byte chunks, 8 per thread) and this thread's weight quarter
    struct Stage {
        u4v_t xr[XR];
        QuarterRaw<TA> ra;
        QuarterRaw<TB> rb;
    };
    auto fetch = [&](Stage& st, int kt) {
#pragma unroll
        for (int j = 0; j < XR; j++) {
            const int idx = j * kGemmThreads + tid;
            const int r = idx >> 4, c = idx & 15;
            const int col = kt * kTileK + c * 8;
            st.xr[j] = u4v_t{0u, 0u, 0u, 0u};
            if (m0 + r < g.m && col < g.k) st.xr[j] = *reinterpret_cast<const u4v_t*>(g.x + (size_t)(m0 + r) * g.k + col);
        }
        if constexpr (TB != TA) {
            if (use_b) st.rb.fetch(sg.w, wrow, kt, wq);
            else st.ra.fetch(sg.w, wrow, kt, wq);
        } else {
            st.ra.fetch(sg.w, wrow, kt, wq);
        }
    };
    auto stage = [&](const Stage& st) {
#pragma unroll
        for (int j = 0; j < XR; j++) {
            const int idx = j * kGemmThreads + tid;
            *reinterpret_cast<u4v_t*>(xs + (idx >> 4) * kLdsRow + (idx & 15) * 8) = st.xr[j];
        }
        if constexpr (TB != TA) {
            if (use_b) st.rb.convert(ws + wr * kLdsRow + 64 * wq);
            else st.ra.convert(ws + wr * kLdsRow + 64 * wq);
        } else {
            st.ra.convert(ws + wr * kLdsRow + 64 * wq);
        }
    };
    auto multiply = [&]() {
#pragma unroll
        for (int ks = 0; ks < kTileK / 32; ks++) {
            const int kk = ks * 32 + 8 * (lane >> 4);
            h8_t b[2];
#pragma unroll
            for (int nb = 0; nb < 2; nb++)
                b[nb] = *reinterpret_cast<const h8_t*>(ws + (32 * wave + 16 * nb + (lane & 15)) * kLdsRow + kk);
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
                const h8_t a = *reinterpret_cast<const h8_t*>(xs + (16 * mb + (lane & 15)) * kLdsRow + kk);
                acc[mb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[0], acc[mb][0], 0, 0, 0);
                acc[mb][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[1], acc[mb][1], 0, 0, 0);
            }
        }
    };
#if RIBN_PG_DEPTH == 2
    // two tiles ahead: the loads of tile kt + 2 are issued while tile kt is multiplied
    Stage s0, s1;
    if (kt0 < kt1) fetch(s0, kt0);
    if (kt0 + 1 < kt1) fetch(s1, kt0 + 1);
    for (int kt = kt0; kt < kt1; kt += 2) {
        __syncthreads();   // the previous tile's MFMA reads are done
        stage(s0);
        __syncthreads();
        if (kt + 2 < kt1) fetch(s0, kt + 2);
        multiply();
        if (kt + 1 >= kt1) break;
        __syncthreads();
        stage(s1);
        __syncthreads();
        if (kt + 3 < kt1) fetch(s1, kt + 3);
        multiply();
    }
#else
    Stage s0;
    if (kt0 < kt1) fetch(s0, kt0);
    for (int kt = kt0; kt < kt1; kt++) {
        __syncthreads();   // the previous tile's MFMA reads are done
        stage(s0);
        __syncthreads();
        if (kt + 1 < kt1) fetch(s0, kt + 1);
        multiply();
    }
#endif
    // epilogue: C[m][n] of block (mb, nb): m = 16 mb + 4 (lane / 16) + i, n = 16 nb + lane % 16
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
        const int n = n0 + 32 * wave + 16 * nb + (lane & 15);
        if (n >= n_rows) continue;
        const float bias = sg.bias && z == 0 ? sg.bias[n] : 0.f;
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 16 * mb + 4 * (lane >> 4) + i;
                if (m >= g.m) continue;
                const float v = (i == 0 ? acc[mb][nb].x : i == 1 ? acc[mb][nb].y : i == 2 ? acc[mb][nb].z : acc[mb][nb].w) + bias;
                const size_t o = (size_t)m * g.ldy + sg.col0 + n;
                if (ks > 1) g.part[(size_t)z * g.m * g.ldy + o] = v;
                else if (g.mode == MV_ADD) g.y[o] = g.res[o] + v;
                else g.y[o] = v;
            }
        }
    }
}

// y = (res) + sum over z of part[z] (fixed order: deterministic)
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* part, int ks, size_t n, const float* res,
                                                            float* y, int add) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v = add ? res[i] : 0.f;
    for (int z = 0; z < ks; z++) v += part[(size_t)z * n + i];
    y[i] = v;
}

// rows x[m][k] -> f16(rms_norm(x) * w) (rms_norm, model_ops.rs:108-157); w may be null
// (plain conversion). One workgroup per row.
__global__ __launch_bounds__(256) void rows_rms_f16_kernel(const float* x, int k, const float* w, float eps, int norm,
                                                           uint16_t* out, int ldo) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (size_t)r * k;
    float inv = 1.0f;
    if (norm) {
        float ss = 0.f;
        for (int i = tid; i < k; i += 256) ss += xr[i] * xr[i];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        ss = red[0] + red[1] + red[2] + red[3];
        inv = 1.0f / sqrtf(ss / (float)k + eps);
    }
    for (int i = tid; i < k; i += 256) {
        const float v = w ? xr[i] * inv * w[i] : xr[i] * inv;
        out[(size_t)r * ldo + i] = f2h_bits(v);
    }
}

// token rows: h[r][e] = dequantized token_embd row of tokens[r] (q4_k_embedding)
__global__ __launch_bounds__(256) void embed_rows_kernel(QMat w, const uint32_t* tokens, int hidden, float* h) {
    const int r = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= hidden) return;
    const uint32_t tok = tokens[r];
    // same exact element dequantization as the decode embedding
    const size_t nb = w.nb;
    const uint32_t be = w.type == 8 ? 32u : 256u;
    const uint32_t blk = (uint32_t)e / be, i = (uint32_t)e % be;
    const size_t bi = (size_t)tok * nb + blk;
    float v;
    if (w.type == 8) {
        v = __fmul_rn(canon(*reinterpret_cast<const uint16_t*>(w.b + bi * 2)), (float)(int8_t)w.a[bi * 32 + i]);
    } else if (w.type == 12) {
        const uint8_t* dd = w.c + bi * 4;
        const float d = canon(dd[0] | (dd[1] << 8)), dmin = canon(dd[2] | (dd[3] << 8));
        const uint32_t g = i / 32, j = i % 32;
        const uint8_t* sp = w.b + bi * 16 + (g / 2) * 4;
        const uint32_t sc = sp[g % 2], mn = sp[2 + g % 2];
        const uint32_t q = (w.a[bi * 128 + (g / 2) * 32 + j] >> ((g % 2) * 4)) & 15u;
        v = __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)q), __fmul_rn(dmin, (float)mn));
    } else {
        const uint32_t g = i / 32, pos = i % 32, chunk = g / 4, variant = g % 4;
        const uint32_t lo = (w.a[bi * 128 + chunk * 64 + (variant % 2) * 32 + pos] >> (variant < 2 ? 0 : 4)) & 15u;
        const uint32_t hi = (w.b[bi * 64 + chunk * 32 + pos] >> (2 * variant)) & 3u;
        const float d = canon(*reinterpret_cast<const uint16_t*>(w.d + bi * 2));
        const uint32_t sidx = g * 2 + pos / 16;
        const int8_t sc = (int8_t)w.c[bi * 16 + 2 * (4 * (sidx / 8) + sidx % 4) + (sidx / 4) % 2];
        v = __fmul_rn(__fmul_rn(d, (float)sc), (float)((int)(lo | (hi << 4)) - 32));
    }
    h[(size_t)r * hidden + e] = v;
}

// Per row and head: q/k RMSNorm (qwen_reference.rs:382-400), NeoX rope at the
// row's position (theta = pos * inv_freq, as the decode table), K/V append to
// the paged cache (kv_append_f16, model_ops.rs:1258-1276). q goes to qout (fp32,
// for the attention); one workgroup of 64 threads per (row, head), heads
// 0..hq-1 are q heads, hq..hq+hkv-1 the k/v heads.
__global__ __launch_bounds__(64) void qk_rope_append_kernel(PrefillRows p) {
    __shared__ float v[128];
    const int r = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
    const int hd = p.hd, qd = p.hq * hd, kd = p.hkv * hd;
    const int pos = p.pos0 + r;
    const bool is_q = head < p.hq;
    const int kvh = head - p.hq;
    const float* src = p.qkv + (size_t)r * p.ld_qkv + (is_q ? head * hd : qd + kvh * hd);
    for (int d = lane; d < hd; d += 64) v[d] = src[d];
    __syncthreads();
    const float* nw = is_q ? p.q_norm : p.k_norm;
    if (nw) {
        float ss = 0.f;
        for (int d = lane; d < hd; d += 64) ss += v[d] * v[d];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        const float inv = 1.0f / sqrtf(ss / (float)hd + p.eps);
        __syncthreads();
        for (int d = lane; d < hd; d += 64) v[d] = v[d] * inv * nw[d];
        __syncthreads();
    }
    const int half = p.rot / 2;
    float outv[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int d = lane + 64 * j;
        outv[j] = d < hd ? v[d] : 0.f;
        if (d < 2 * half) {
            const int pp = d < half ? d : d - half;
            const float theta = (float)pos * p.inv_freq[pp];
            const float c = cosf(theta), sn = sinf(theta);
            outv[j] = d < half ? v[d] * c - v[d + half] * sn : v[d - half] * sn + v[d] * c;
        }
    }
    if (is_q) {
        for (int j = 0; j < 2; j++) {
            const int d = lane + 64 * j;
            if (d < hd) p.qout[(size_t)r * qd + head * hd + d] = outv[j];
        }
        return;
    }
    const int page = p.pages[pos / kPageTokens];
    const size_t base = ((size_t)(page * p.hkv + kvh) * kPageTokens + pos % kPageTokens) * hd;
    const float* vsrc = p.qkv + (size_t)r * p.ld_qkv + qd + kd + kvh * hd;
    for (int j = 0; j < 2; j++) {
        const int d = lane + 64 * j;
        if (d >= hd) continue;
        const float kv = outv[j], vv = vsrc[d];
        if (p.kv_f16) {
            p.kcache[base + d] = f2h_bits(kv);
            p.vcache[base + d] = f2h_bits(vv);
        } else {
            uint32_t ku = __float_as_uint(kv), vu = __float_as_uint(vv);
            ku = (ku & 0x7fffffffu) > 0x7f800000u ? (ku >> 16) | 0x40u : (ku + 0x7fffu + ((ku >> 16) & 1u)) >> 16;
            vu = (vu & 0x7fffffffu) > 0x7f800000u ? (vu >> 16) | 0x40u : (vu + 0x7fffu + ((vu >> 16) & 1u)) >> 16;
            p.kcache[base + d] = (uint16_t)ku;
            p.vcache[base + d] = (uint16_t)vu;
        }
    }
}


// Causal attention of a chunk's rows over the paged cache (positions 0 .. own
// position; attn_score_gqa_paged rows > 1, model_ops.rs:442-554), flash style
// on MFMA. Workgroup = RB blocks of 16 chunk rows x the G query heads of one
// KV head; a (row block, head) tile belongs to one wave. Per 32-key tile:
//   S^T[key][q] = K Q^T   (v_mfma_f32_16x16x32_f16, A = K rows from LDS,
//                          B = q in registers, binary16 with log2(e)/sqrt(hd) folded in)
//   online softmax per query in fp32 (exp2), P rounded to binary16
//   O^T[dim][q] += V^T P^T (A = V^T from a transposed LDS tile, B = P^T taken
//                          straight from the S^T accumulators)
// The S^T / O^T orientation keeps every per-query quantity in lane % 16, so the
// softmax needs no transposes: a lane's P^T entries are keys 4j..4j+3 and
// 16+4j..16+4j+3 (j = lane / 16), and V^T is read in the same key order.
// A binary16 cache is used as stored; a bfloat16 cache is converted to binary16
// when staged (exact for values in binary16's normal range).
constexpr int kAttKeys = 32;

template <int HD, int G, bool F16KV>
__global__ __launch_bounds__(256) void prefill_attention_kernel(PrefillRows p) {
    constexpr int RB = G >= 4 ? 1 : 4 / G;     // 16-row blocks per workgroup
    constexpr int NT = RB * G;                  // tiles
    constexpr int TPW = (NT + 3) / 4;           // tiles per wave
    constexpr int NC = HD / 32;                 // 32-dim chunks of q.k
    constexpr int ND = HD / 16;                 // 16-dim blocks of the output
    constexpr int KLD = HD + 8;                 // K tile row, halves
    constexpr int VLD = kAttKeys + 4;           // V^T row, halves (8-byte aligned rows)
    constexpr int CPR = HD / 8;                 // 16-byte chunks per cache row
    constexpr int KCH = kAttKeys * CPR / 256;   // K chunks per thread per tile
    constexpr int VIT = (kAttKeys / 2) * CPR;   // V (key pair, chunk) items per tile
    __shared__ __attribute__((aligned(16))) _Float16 ks[kAttKeys][KLD];
    __shared__ __attribute__((aligned(16))) _Float16 vts[HD][VLD];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int qn = lane & 15, j = lane >> 4;
    const int kvh = blockIdx.y;
    const int row0 = blockIdx.x * 16 * RB;
    const int last_pos = p.pos0 + min(p.m, row0 + 16 * RB) - 1;
    const int ldq = p.hq * HD;
    const float qscale = 1.44269504088896341f / sqrtf((float)HD);

    h8_t qb[TPW][NC];
    f4_t acc[TPW][ND];
    float mrun[TPW], lrun[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        const int tile = wave + 4 * t, rb = tile / G, h = tile % G;
        const int r = row0 + rb * 16 + qn;
        const bool ok = tile < NT && r < p.m;
        const float* q = p.qout + (size_t)r * ldq + (kvh * G + h) * HD + 8 * j;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float4 lo = float4{0.f, 0.f, 0.f, 0.f}, hi = lo;
            if (ok) {
                lo = *reinterpret_cast<const float4*>(q + 32 * c);
                hi = *reinterpret_cast<const float4*>(q + 32 * c + 4);
            }
            qb[t][c] = h8_t{(_Float16)(lo.x * qscale), (_Float16)(lo.y * qscale), (_Float16)(lo.z * qscale),
                            (_Float16)(lo.w * qscale), (_Float16)(hi.x * qscale), (_Float16)(hi.y * qscale),
                            (_Float16)(hi.z * qscale), (_Float16)(hi.w * qscale)};
        }
#pragma unroll
        for (int d = 0; d < ND; d++) acc[t][d] = f4_t{0.f, 0.f, 0.f, 0.f};
        mrun[t] = -INFINITY;
        lrun[t] = 0.f;
    }

    // cache tile in registers: K chunks, and V as key pairs for the transposed store
    u4v_t kr[KCH], vr[2];
    auto cache_off = [&](int pos, int c8) {
        const int page = p.pages[pos / kPageTokens];
        return ((size_t)(page * p.hkv + kvh) * kPageTokens + pos % kPageTokens) * HD + c8 * 8;
    };
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int e = 0; e < KCH; e++) {
            const int idx = e * 256 + tid, key = idx / CPR, c8 = idx % CPR, pos = t0 + key;
            kr[e] = pos <= last_pos ? *reinterpret_cast<const u4v_t*>(p.kcache + cache_off(pos, c8)) : u4v_t{0u, 0u, 0u, 0u};
        }
        if (tid < VIT) {
            const int kp = tid / CPR, c8 = tid % CPR;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int pos = t0 + 2 * kp + e;
                vr[e] = pos <= last_pos ? *reinterpret_cast<const u4v_t*>(p.vcache + cache_off(pos, c8)) : u4v_t{0u, 0u, 0u, 0u};
            }
        }
    };
    // bfloat16 pair (one dword) -> binary16 pair
    auto to_f16x2 = [](uint32_t w) -> uint32_t {
        if constexpr (F16KV) return w;
        const _Float16 a = (_Float16)__uint_as_float(w << 16), b = (_Float16)__uint_as_float(w & 0xffff0000u);
        return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int e = 0; e < KCH; e++) {
            const int idx = e * 256 + tid, key = idx / CPR, c8 = idx % CPR;
            *reinterpret_cast<u4v_t*>(&ks[key][c8 * 8]) =
                u4v_t{to_f16x2(kr[e].x), to_f16x2(kr[e].y), to_f16x2(kr[e].z), to_f16x2(kr[e].w)};
        }
        if (tid < VIT) {
            const int kp = tid / CPR, c8 = tid % CPR;
            const uint32_t a[4] = {to_f16x2(vr[0].x), to_f16x2(vr[0].y), to_f16x2(vr[0].z), to_f16x2(vr[0].w)};
            const uint32_t b[4] = {to_f16x2(vr[1].x), to_f16x2(vr[1].y), to_f16x2(vr[1].z), to_f16x2(vr[1].w)};
#pragma unroll
            for (int d = 0; d < 8; d++) {
                const uint32_t lo = (a[d / 2] >> (16 * (d & 1))) & 0xffffu, hi = (b[d / 2] >> (16 * (d & 1))) & 0xffffu;
                *reinterpret_cast<uint32_t*>(&vts[c8 * 8 + d][2 * kp]) = lo | (hi << 16);
            }
        }
    };

    load_tile(0);
    for (int t0 = 0; t0 <= last_pos; t0 += kAttKeys) {
        __syncthreads();   // the previous tile is consumed
        store_tile();
        __syncthreads();
        if (t0 + kAttKeys <= last_pos) load_tile(t0 + kAttKeys);
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            const int tile = wave + 4 * t, rb = tile / G;
            // wave-uniform: an absent tile, or a row block whose rows all precede the keys
            if (tile >= NT || t0 > p.pos0 + row0 + rb * 16 + 15) continue;
            const int qpos = p.pos0 + row0 + rb * 16 + qn;
            f4_t s[2] = {f4_t{0.f, 0.f, 0.f, 0.f}, f4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int blk = 0; blk < 2; blk++)
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const h8_t a = *reinterpret_cast<const h8_t*>(&ks[16 * blk + qn][32 * c + 8 * j]);
                    s[blk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qb[t][c], s[blk], 0, 0, 0);
                }
            // s[blk][i] = S^T[key t0 + 16 blk + 4 j + i][query qn] (log2 domain)
            float tmax = -INFINITY;
#pragma unroll
            for (int blk = 0; blk < 2; blk++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (t0 + 16 * blk + 4 * j + i > qpos) s[blk][i] = -INFINITY;
                    tmax = fmaxf(tmax, s[blk][i]);
                }
            tmax = xor32_max(xor16_max(tmax));
            const float mnew = fmaxf(mrun[t], tmax);
            const float corr = exp2f(mrun[t] - mnew);
            float psum = 0.f;
            _Float16 ph[8];
#pragma unroll
            for (int blk = 0; blk < 2; blk++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float pv = exp2f(s[blk][i] - mnew);
                    psum += pv;
                    ph[4 * blk + i] = (_Float16)pv;
                }
            psum = xor32_sum(xor16_sum(psum));
            lrun[t] = lrun[t] * corr + psum;
            mrun[t] = mnew;
            const h8_t pb = h8_t{ph[0], ph[1], ph[2], ph[3], ph[4], ph[5], ph[6], ph[7]};
#pragma unroll
            for (int d = 0; d < ND; d++) {
                acc[t][d] *= corr;
                const uint2 lo = *reinterpret_cast<const uint2*>(&vts[16 * d + qn][4 * j]);
                const uint2 hi = *reinterpret_cast<const uint2*>(&vts[16 * d + qn][16 + 4 * j]);
                const h8_t a = __builtin_bit_cast(h8_t, u4v_t{lo.x, lo.y, hi.x, hi.y});
                acc[t][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, acc[t][d], 0, 0, 0);
            }
        }
    }
    // acc[t][d][i] = O^T[dim 16 d + 4 j + i][query qn]
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        const int tile = wave + 4 * t, rb = tile / G, h = tile % G;
        const int r = row0 + rb * 16 + qn;
        if (tile >= NT || r >= p.m) continue;
        const float il = 1.0f / lrun[t];
        uint16_t* out = p.attn16 + (size_t)r * ldq + (kvh * G + h) * HD + 4 * j;
#pragma unroll
        for (int d = 0; d < ND; d++) {
            const uint32_t w0 = f2h_bits(acc[t][d][0] * il) | ((uint32_t)f2h_bits(acc[t][d][1] * il) << 16);
            const uint32_t w1 = f2h_bits(acc[t][d][2] * il) | ((uint32_t)f2h_bits(acc[t][d][3] * il) << 16);
            *reinterpret_cast<uint2*>(out + 16 * d) = uint2{w0, w1};
        }
    }
}

// act16[r][j] = f16(silu(gu[r][j]) * gu[r][F + j]) (silu_mul, model_ops.rs:318-330)
__global__ __launch_bounds__(256) void silu_mul_f16_kernel(const float* gu, int f, int m, uint16_t* act) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)m * f) return;
    const size_t r = i / f, j = i % f;
    const float g = gu[r * 2 * f + j], u = gu[r * 2 * f + f + j];
    act[i] = f2h_bits(g / (1.0f + expf(-g)) * u);
}

__global__ void set_pos_kernel(SeqState* s, int pos) {
    if (threadIdx.x == 0) s->pos = pos;
}

template <int HD, int G>
hipError_t attention_launch_prefill(const PrefillRows& p, hipStream_t st) {
    constexpr int RB = G >= 4 ? 1 : 4 / G;
    const dim3 grid((p.m + 16 * RB - 1) / (16 * RB), p.hkv);
    if (p.kv_f16) prefill_attention_kernel<HD, G, true><<<grid, 256, 0, st>>>(p);
    else prefill_attention_kernel<HD, G, false><<<grid, 256, 0, st>>>(p);
    return hipGetLastError();
}

template <int HD>
hipError_t attention_dispatch_prefill(const PrefillRows& p, hipStream_t st) {
    switch (p.hq / p.hkv) {
    case 1: return attention_launch_prefill<HD, 1>(p, st);
    case 2: return attention_launch_prefill<HD, 2>(p, st);
    case 3: return attention_launch_prefill<HD, 3>(p, st);
    case 4: return attention_launch_prefill<HD, 4>(p, st);
    case 5: return attention_launch_prefill<HD, 5>(p, st);
    case 6: return attention_launch_prefill<HD, 6>(p, st);
    case 7: return attention_launch_prefill<HD, 7>(p, st);
    case 8: return attention_launch_prefill<HD, 8>(p, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

int gemm_rows_tile(int m) { return m <= 32 ? 32 : kTileM; }

int prefill_gemm_splits(int m, int k, int n_tiles) {
    // enough workgroups for two per CU on 256 CUs, at least 4 K tiles per split, at most 8 splits
    const int mt = gemm_rows_tile(m);
    const int wgs = n_tiles * ((m + mt - 1) / mt);
    const int n_kt = (k + kTileK - 1) / kTileK;
    int ks = 1;
    while (ks < 8 && wgs * ks < 512 && n_kt / (2 * ks) >= 4) ks *= 2;
    return ks;
}

size_t prefill_gemm_lds_bytes() { return (size_t)(kTileM + kTileN) * kLdsRow * 2; }

hipError_t launch_prefill_gemm(const PrefillGemm& g, hipStream_t st) {
    if (g.m <= 0 || g.k <= 0 || g.k % 32 || g.nseg < 1 || g.nseg > 3) return hipErrorInvalidValue;
    int tiles = 0;
    for (int i = 0; i < g.nseg; i++) {
        const QMat& w = g.seg[i].w;
        // K-quant rows are whole 256-value super-blocks; Q8_0 rows may end inside a tile
        if (w.k != (uint32_t)g.k || w.rows == 0 || (w.type != 8 && g.k % 256) || g.seg[i].tile0 != tiles)
            return hipErrorInvalidValue;
        if (i < 2 && w.type != g.seg[0].w.type) return hipErrorInvalidValue;
        tiles += (int)((w.rows + kTileN - 1) / kTileN);
    }
    const uint32_t ta = g.seg[0].w.type, tb = g.seg[g.nseg - 1].w.type;
    const int ks = g.part ? max(1, g.ksplit) : 1;
    if (ks > 1 && ks > (g.k + kTileK - 1) / kTileK) return hipErrorInvalidValue;
    const int mt = gemm_rows_tile(g.m);
    const dim3 grid(tiles, (g.m + mt - 1) / mt, ks);
    PrefillGemm gg = g;
    gg.ksplit = ks;
    const size_t lds = (size_t)(mt + kTileN) * kLdsRow * 2;
#define RIBN_PG(A, B)                                                                                           \
    if (ta == A && tb == B) {                                                                                   \
        hipError_t e;                                                                                           \
        if (mt == 32) {                                                                                         \
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_gemm_kernel<A, B, 32>),              \
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);                      \
            if (e != hipSuccess) return e;                                                                      \
            prefill_gemm_kernel<A, B, 32><<<grid, kGemmThreads, lds, st>>>(gg);                                 \
        } else {                                                                                                \
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_gemm_kernel<A, B, kTileM>),          \
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);                      \
            if (e != hipSuccess) return e;                                                                      \
            prefill_gemm_kernel<A, B, kTileM><<<grid, kGemmThreads, lds, st>>>(gg);                             \
        }                                                                                                       \
        e = hipGetLastError();                                                                                  \
        if (e != hipSuccess || ks == 1) return e;                                                               \
        const size_t n = (size_t)g.m * g.ldy;                                                                   \
        splitk_reduce_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(g.part, ks, n, g.res, g.y,            \
                                                                          g.mode == MV_ADD ? 1 : 0);            \
        return hipGetLastError();                                                                               \
    }
    RIBN_PG(12, 12) RIBN_PG(14, 14) RIBN_PG(8, 8) RIBN_PG(12, 14) RIBN_PG(14, 12) RIBN_PG(12, 8) RIBN_PG(8, 12)
    RIBN_PG(14, 8) RIBN_PG(8, 14)
#undef RIBN_PG
    return hipErrorInvalidValue;
}

hipError_t launch_rows_rms_f16(const float* x, int m, int k, const float* w, float eps, bool norm, uint16_t* out,
                               int ldo, hipStream_t st) {
    if (m <= 0) return hipErrorInvalidValue;
    rows_rms_f16_kernel<<<m, 256, 0, st>>>(x, k, w, eps, norm ? 1 : 0, out, ldo);
    return hipGetLastError();
}

hipError_t launch_embed_rows(const QMat& w, const uint32_t* tokens, int m, int hidden, float* h, hipStream_t st) {
    if (m <= 0) return hipErrorInvalidValue;
    embed_rows_kernel<<<dim3((hidden + 255) / 256, m), 256, 0, st>>>(w, tokens, hidden, h);
    return hipGetLastError();
}

hipError_t launch_qk_rope_append(const PrefillRows& p, hipStream_t st) {
    if (p.m <= 0 || p.hd > 128 || p.rot > p.hd) return hipErrorInvalidValue;
    qk_rope_append_kernel<<<dim3(p.m, p.hq + p.hkv), 64, 0, st>>>(p);
    return hipGetLastError();
}

hipError_t launch_prefill_attention(const PrefillRows& p, hipStream_t st) {
    if (p.m <= 0 || p.hq % p.hkv) return hipErrorInvalidValue;
    if (p.hd == 128) return attention_dispatch_prefill<128>(p, st);
    if (p.hd == 64) return attention_dispatch_prefill<64>(p, st);
    return hipErrorInvalidValue;
}

hipError_t launch_silu_mul_f16(const float* gu, int f, int m, uint16_t* act, hipStream_t st) {
    const size_t n = (size_t)m * f;
    silu_mul_f16_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(gu, f, m, act);
    return hipGetLastError();
}

hipError_t launch_set_pos(SeqState* s, int pos, hipStream_t st) {
    set_pos_kernel<<<1, 64, 0, st>>>(s, pos);
    return hipGetLastError();
}

}  // namespace ribn
