// Chunked prefill: the prompt's rows run through every layer together, so each
// weight matrix is read once per chunk and the projections are dense GEMMs on
// the matrix cores (prefill_chunk / run_prefill_chunk, nvidia/src/decode.rs:2124,
// 2360; the reference batches 8 rows through warp GEMVs, this build uses MFMA).
//
//  * prefill_gemm: Y[M][N] = X[M][K] deq(W)^T. X is binary16 (the RMSNorm'd or
//    activation rows), W stays in its GGUF planes and every lane dequantizes
//    its weight values straight into MFMA operand registers (exactly as
//    dequantize_block, then rounded to binary16); v_mfma_f32_16x16x32_f16
//    accumulates in fp32.
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
constexpr int kTileK = 128;   // half a Q4_K / Q6_K super-block, four Q8_0 blocks
constexpr int kLdsRow = kTileK + 8;   // halves per LDS row (padded against bank conflicts)

__device__ __forceinline__ float h2f_bits(uint32_t b) { return __half2float(__ushort_as_half((unsigned short)(b & 0xffffu))); }
__device__ __forceinline__ float canon(uint32_t b) {
    const float v = h2f_bits(b);
    return v != v ? __uint_as_float(0x7fc00000u) : v;
}
__device__ __forceinline__ uint16_t f2h_bits(float f) { return __half_as_ushort(__float2half_rn(f)); }

// Weight fragments straight from the GGUF planes. In a 128-wide K tile, lane
// (bn, bj) of a 16-row weight block dequantizes 32 values of row bn into the
// MFMA B operand of the four 32-wide K steps (8 values each): the values it
// can load contiguously. Which 8 values step ks gets is fixed per type by
// xoff(ks, bj), the offset of the matching 8 contiguous X values in the tile
// (the contraction does not depend on how K is ordered inside a step, only on
// both operands using the same order). Each value follows dequantize_block
// (gguf/src/lib.rs:584-649) exactly, then rounded to binary16: the quant
// integer is built exactly as binary16 (1024 + q with v_perm_b32, minus the
// bias in one packed add for two values) and v_fma_mix computes the fp32
// result from it and rounds that to binary16 (about two VALU instructions per
// value). The raw bytes of the next K tile are fetched while the current one
// is multiplied.
template <int T>
struct WFrag;

typedef _Float16 h2v_t __attribute__((ext_vector_type(2)));
typedef float f2v_t __attribute__((ext_vector_type(2)));
// two fp32 values -> binary16 pair, round to nearest even (v_cvt_pk_f16_f32)
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v_t{a, b}), h2v_t));
}
// Four small unsigned integers (the bytes of v, each < 1024) -> two binary16
// pairs holding 1024 + byte, exact (0x64 is the high byte of 1024.0):
// lo = bytes 0, 1, hi = bytes 2, 3 (v_perm_b32 with 0x64 bytes from the other source).
__device__ __forceinline__ h2v_t bias1024_lo(uint32_t v) {
    return __builtin_bit_cast(h2v_t, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u));
}
__device__ __forceinline__ h2v_t bias1024_hi(uint32_t v) {
    return __builtin_bit_cast(h2v_t, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u));
}
// round16(round32(q * g + c)) for a pair of exact binary16 integers q: the
// reference's fp32 result rounded to binary16 (v_fma_mixlo/mixhi_f16)
__device__ __forceinline__ uint32_t mix2(h2v_t q, float g, float c) {
    const h2v_t r{(_Float16)__builtin_fmaf((float)q[0], g, c), (_Float16)__builtin_fmaf((float)q[1], g, c)};
    return __builtin_bit_cast(uint32_t, r);
}

template <>
struct WFrag<12> {
    // Q4_K: the tile's group pair p = 2 (kt % 2) + bj / 2 of block kt / 2; the
    // lane's 16 bytes are qs[32p + 16 (bj % 2) ..]: low nibbles = values
    // 64 (bj/2) + 16 (bj%2) + b of the tile, high nibbles = the same + 32.
    // Scale dword p = sc(2p), sc(2p+1), m(2p), m(2p+1).
    uint32_t dd, s;
    u4v_t qv;
    __device__ static __forceinline__ int xoff(int ks, int j) { return 64 * (j >> 1) + 16 * (j & 1) + 8 * (ks & 1) + 32 * (ks >> 1); }
    // the lane's byte offsets into the planes (fixed over K); each fetch adds
    // them to plane bases that depend on the K tile only (wave-uniform), so the
    // loads take scalar-base + vector-offset addressing with no address math
    struct Off { uint32_t a, b, c; };
    __device__ static __forceinline__ Off lane_off(const QMat& w, size_t row, int j) {
        const uint32_t rb = (uint32_t)(row * w.nb);
        return Off{rb * 128u + 32u * (uint32_t)(j >> 1) + 16u * (uint32_t)(j & 1), rb * 16u + 4u * (uint32_t)(j >> 1), rb * 4u};
    }
    __device__ __forceinline__ void fetch(const QMat& w, const Off& o, int kt) {
        const int kb = kt >> 1, h = kt & 1;
        dd = *reinterpret_cast<const uint32_t*>(w.c + (size_t)kb * 4 + o.c);
        s = *reinterpret_cast<const uint32_t*>(w.b + (size_t)kb * 16 + 8 * h + o.b);
        qv = *reinterpret_cast<const u4v_t*>(w.a + (size_t)kb * 128 + 64 * h + o.a);
    }
    // the same bytes from the GEMM-ordered copy: `blk` is the block of this
    // lane's 16-row group and K tile (QMat::g)
    __device__ __forceinline__ void fetch_g(const uint8_t* blk) {
        const int lane = threadIdx.x & 63, bn = lane & 15, bj = lane >> 4;
        qv = *reinterpret_cast<const u4v_t*>(blk + lane * 16);
        s = *reinterpret_cast<const uint32_t*>(blk + 1024 + (bn * 2 + (bj >> 1)) * 4);
        dd = *reinterpret_cast<const uint32_t*>(blk + 1152 + bn * 4);
    }
    static constexpr size_t kBlk = kGemmBlkQ4;
    // value = round16(fma(q, sc*d, -m*dmin)): g * q is exact in fp32 (d has
    // 11 significant bits, sc 6, q 4), so the fma rounds once, as the
    // reference's multiply-then-subtract does
    __device__ __forceinline__ h8_t frag(int ks) const {
        const float d = canon(dd), dmin = canon(dd >> 16);
        const int hi = ks >> 1;   // 0: low nibbles (group 2p), 1: high nibbles (group 2p + 1)
        const float g = __fmul_rn(d, (float)((s >> (8 * hi)) & 0xffu));
        const float m = __fmul_rn(dmin, (float)((s >> (16 + 8 * hi)) & 0xffu));
        const uint32_t w0 = (ks & 1) ? qv.z : qv.x, w1 = (ks & 1) ? qv.w : qv.y;
        const uint32_t n0 = (w0 >> (4 * hi)) & 0x0f0f0f0fu, n1 = (w1 >> (4 * hi)) & 0x0f0f0f0fu;
        const h2v_t k1024 = h2v_t{(_Float16)1024.0f, (_Float16)1024.0f};
        const u4v_t o{mix2(bias1024_lo(n0) - k1024, g, -m), mix2(bias1024_hi(n0) - k1024, g, -m),
                      mix2(bias1024_lo(n1) - k1024, g, -m), mix2(bias1024_hi(n1) - k1024, g, -m)};
        return __builtin_bit_cast(h8_t, o);
    }
};

template <>
struct WFrag<14> {
    // Q6_K: chunk h = kt % 2 of block kt / 2 (ql bytes 64h.., qh bytes 32h..);
    // value 32v + l of the chunk is ((ql[32 (v%2) + l] >> 4 (v/2)) & 15) |
    // (((qh[l] >> 2v) & 3) << 4), minus 32, times d * sc(8h + 2v + l/16).
    // Lane bj holds l = 8 bj .. 8 bj + 7 for v = 0..3 (step ks = v). Sub-block
    // scale s sits at c-plane byte 2c + slot, c = 4 (s/8) + s%4, slot = (s/4) % 2:
    // for s = 8h + 2v + bj/2 that is byte 8h + 4 (v%2) + 2 (bj/2) + v/2.
    uint32_t d16, sc01, sc23;   // scale bytes (v=0, v=2) and (v=1, v=3)
    uint2 ql0, ql1, qh;
    __device__ static __forceinline__ int xoff(int ks, int j) { return 32 * ks + 8 * j; }
    struct Off { uint32_t a, b, c, d; };
    __device__ static __forceinline__ Off lane_off(const QMat& w, size_t row, int j) {
        const uint32_t rb = (uint32_t)(row * w.nb);
        return Off{rb * 128u + 8u * (uint32_t)j, rb * 64u + 8u * (uint32_t)j, rb * 16u + 2u * (uint32_t)(j >> 1), rb * 2u};
    }
    __device__ __forceinline__ void fetch(const QMat& w, const Off& o, int kt) {
        const int kb = kt >> 1, h = kt & 1;
        d16 = *reinterpret_cast<const uint16_t*>(w.d + (size_t)kb * 2 + o.d);
        const uint8_t* sp = w.c + (size_t)kb * 16 + 8 * h + o.c;
        sc01 = *reinterpret_cast<const uint16_t*>(sp);
        sc23 = *reinterpret_cast<const uint16_t*>(sp + 4);
        const uint8_t* ap = w.a + (size_t)kb * 128 + 64 * h + o.a;
        ql0 = *reinterpret_cast<const uint2*>(ap);
        ql1 = *reinterpret_cast<const uint2*>(ap + 32);
        qh = *reinterpret_cast<const uint2*>(w.b + (size_t)kb * 64 + 32 * h + o.b);
    }
    __device__ __forceinline__ void fetch_g(const uint8_t* blk) {
        const int lane = threadIdx.x & 63, bn = lane & 15, bj = lane >> 4;
        const u4v_t q = *reinterpret_cast<const u4v_t*>(blk + lane * 16);
        ql0 = uint2{q.x, q.y};
        ql1 = uint2{q.z, q.w};
        qh = *reinterpret_cast<const uint2*>(blk + 1024 + lane * 8);
        const uint32_t sc = *reinterpret_cast<const uint32_t*>(blk + 1536 + (bn * 2 + (bj >> 1)) * 4);
        sc01 = sc & 0xffffu;
        sc23 = sc >> 16;
        d16 = *reinterpret_cast<const uint16_t*>(blk + 1664 + bn * 2);
    }
    static constexpr size_t kBlk = kGemmBlkQ6;
    // value = round16(round32(d*sc * (q - 32))), q - 32 exact in binary16
    __device__ __forceinline__ h8_t frag(int v) const {
        const float d = canon(d16);
        const uint32_t scb = (v & 1) ? sc23 : sc01;
        const float gsc = __fmul_rn(d, (float)(int8_t)(scb >> (8 * (v >> 1))));
        const uint2 l = (v & 1) ? ql1 : ql0;
        // bytes of q (0..63) for positions e = 0..3 (x) and 4..7 (y)
        const uint32_t qx = ((l.x >> (4 * (v >> 1))) & 0x0f0f0f0fu) | (((qh.x >> (2 * v)) & 0x03030303u) << 4);
        const uint32_t qy = ((l.y >> (4 * (v >> 1))) & 0x0f0f0f0fu) | (((qh.y >> (2 * v)) & 0x03030303u) << 4);
        const h2v_t k1056 = h2v_t{(_Float16)1056.0f, (_Float16)1056.0f};
        const u4v_t o{mix2(bias1024_lo(qx) - k1056, gsc, 0.f), mix2(bias1024_hi(qx) - k1056, gsc, 0.f),
                      mix2(bias1024_lo(qy) - k1056, gsc, 0.f), mix2(bias1024_hi(qy) - k1056, gsc, 0.f)};
        return __builtin_bit_cast(h8_t, o);
    }
};

template <>
struct WFrag<8> {
    // Q8_0: lane bj holds block 4 kt + bj (step ks = its bytes 8 ks ..);
    // past the row's end (k % 128 != 0): zeros
    uint32_t d16;
    u4v_t qv[2];
    __device__ static __forceinline__ int xoff(int ks, int j) { return 32 * j + 8 * ks; }
    struct Off { uint32_t blk; int j; };   // block index of the lane's row and K slot
    __device__ static __forceinline__ Off lane_off(const QMat& w, size_t row, int j) {
        return Off{(uint32_t)(row * w.nb) + (uint32_t)j, j};
    }
    // K a multiple of the 128-wide tile: every block exists, no condition
    __device__ __forceinline__ void fetch_full(const QMat& w, const Off& o, int kt) {
        d16 = *reinterpret_cast<const uint16_t*>(w.b + (size_t)kt * 8 + o.blk * 2u);
        const u4v_t* qs = reinterpret_cast<const u4v_t*>(w.a + (size_t)kt * 128 + o.blk * 32u);
        qv[0] = qs[0];
        qv[1] = qs[1];
    }
    __device__ __forceinline__ void fetch(const QMat& w, const Off& o, int kt) {
        d16 = 0u;
        qv[0] = qv[1] = u4v_t{0u, 0u, 0u, 0u};
        if (4 * kt + o.j < (int)w.nb) fetch_full(w, o, kt);
    }
    // value = round16(d * q) (d * q is exact in fp32), q exact in binary16
    // (int8 as q + 128 unsigned)
    __device__ __forceinline__ h8_t frag(int ks) const {
        const float d = canon(d16);
        const u4v_t& v = qv[ks >> 1];
        const uint32_t w0 = ((ks & 1) ? v.z : v.x) ^ 0x80808080u, w1 = ((ks & 1) ? v.w : v.y) ^ 0x80808080u;
        const h2v_t k1152 = h2v_t{(_Float16)1152.0f, (_Float16)1152.0f};
        const u4v_t o{mix2(bias1024_lo(w0) - k1152, d, 0.f), mix2(bias1024_hi(w0) - k1152, d, 0.f),
                      mix2(bias1024_lo(w1) - k1152, d, 0.f), mix2(bias1024_hi(w1) - k1152, d, 0.f)};
        return __builtin_bit_cast(h8_t, o);
    }
};

// Workgroup tile: MT chunk rows x kGemmTileN (128) weight rows of one segment;
// wave w owns weight rows 32w..32w+31 of the tile (two 16-row blocks, whose B
// fragments it dequantizes itself) for all MT chunk rows (MT/16 blocks of A
// fragments from the X tile in LDS). K runs in tiles of 128; the X slice is
// staged through two LDS buffers (MT x 128 binary16 each, one barrier per
// tile) and the next tile's X chunks and raw weight bytes are fetched into
// registers during the current tile's MFMAs. Two workgroups share a CU.
// MFMA 16x16x32 f16 operand layout (lane l): A[m = l%16][k = 8(l/16) .. +8],
// B[k = 8(l/16) .. +8][n = l%16]; result C[m = 4(l/16) + i][n = l%16], i < 4.
// MT (128 or 32) is the workgroup's chunk rows: 32 for batched decode rows,
// where a 128-row tile would mostly multiply padding.
// GP: the weights come from the GEMM-ordered copy (QMat::g; Q4_K / Q6_K).
template <int T, int MT, bool FULL, bool GP = false>
__device__ __forceinline__ void gemm_tile(const PrefillGemm& g, const PrefillSeg& sg, int m0, int n0, int kt0, int kt1,
                                          int z, uint16_t* xs) {
    static_assert(!GP || T == 12 || T == 14, "GEMM-ordered copies exist for Q4_K and Q6_K");
    constexpr int MB = MT / 16;                // 16-row blocks of chunk rows
    constexpr int NB = kGemmTileN / 64;        // 16-row weight blocks per wave
    constexpr int XR = MT * 16 / kGemmThreads; // X chunks per thread per K tile
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bn = lane & 15, bj = lane >> 4;
    const int n_rows = (int)sg.w.rows;
    f4_t acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) acc[i][nb] = f4_t{0.f, 0.f, 0.f, 0.f};
    typename WFrag<T>::Off woff[NB];
    const uint8_t* gblk[NB];   // GP: the copy's blocks of this wave's 16-row groups at K tile 0
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        if constexpr (GP) {
            // groups past the matrix read its last group (their outputs are not stored)
            const int n16 = min((n0 >> 4) + NB * wave + nb, (n_rows + 15) / 16 - 1);
            gblk[nb] = sg.w.g + (size_t)n16 * (sg.w.k / kTileK) * WFrag<T>::kBlk;
        } else {
            woff[nb] = WFrag<T>::lane_off(sg.w, (size_t)min(n0 + 16 * NB * wave + 16 * nb + bn, n_rows - 1), bj);
        }
    }
    u4v_t xr[XR];
    WFrag<T> w0[NB], w1[NB];   // raw weight bytes of tiles kt and kt + 1
    auto fetch_x = [&](int kt) {
#pragma unroll
        for (int j = 0; j < XR; j++) {
            const int idx = j * kGemmThreads + tid;
            const int r = idx >> 4, c = idx & 15;
            const int col = kt * kTileK + c * 8;
            if constexpr (FULL) {
                // every column is inside X; rows past the chunk re-read its last row (their
                // outputs are not stored), so the load needs no condition
                xr[j] = *reinterpret_cast<const u4v_t*>(g.x + (size_t)min(m0 + r, g.m - 1) * g.k + col);
            } else {
                xr[j] = u4v_t{0u, 0u, 0u, 0u};
                if (m0 + r < g.m && col < g.k) xr[j] = *reinterpret_cast<const u4v_t*>(g.x + (size_t)(m0 + r) * g.k + col);
            }
        }
    };
    auto store_x = [&](uint16_t* buf) {
#pragma unroll
        for (int j = 0; j < XR; j++) {
            const int idx = j * kGemmThreads + tid;
            *reinterpret_cast<u4v_t*>(buf + (idx >> 4) * kLdsRow + (idx & 15) * 8) = xr[j];
        }
    };
    auto fetch_w = [&](WFrag<T> (&wf)[NB], int kt) {
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            if constexpr (GP) wf[nb].fetch_g(gblk[nb] + (size_t)kt * WFrag<T>::kBlk);
            else if constexpr (FULL && T == 8) wf[nb].fetch_full(sg.w, woff[nb], kt);
            else wf[nb].fetch(sg.w, woff[nb], kt);
        }
    };
    // FULL: the fetches of the next tiles are unconditional (past the last tile
    // they re-read it), so the compiler can count the loads in flight behind each
    // use and wait for exactly the ones it needs; under a condition it assumes
    // none was issued and waits for all of them.
    const int kt_last = kt1 - 1;
    if (kt0 < kt1) {
        fetch_x(kt0);
        fetch_w(w0, kt0);
        store_x(xs);
        if (FULL) fetch_x(min(kt0 + 1, kt_last));
        else if (kt0 + 1 < kt1) fetch_x(kt0 + 1);
        __syncthreads();
    }
    for (int kt = kt0; kt < kt1; kt++) {
        if (FULL) fetch_w(w1, min(kt + 1, kt_last));
        else if (kt + 1 < kt1) fetch_w(w1, kt + 1);
        const uint16_t* xb = xs + (size_t)((kt - kt0) & 1) * MT * kLdsRow;
        // scheduling hint: interleave the LDS reads of X with the MFMAs (the
        // 512-token prefill measured 28.0k -> 28.5k tok/s with it; the
        // MFMA-priority and wider-LDS-row variants measured no gain)
        __builtin_amdgcn_iglp_opt(0);
#pragma unroll
        for (int ks = 0; ks < kTileK / 32; ks++) {
            const int kk = WFrag<T>::xoff(ks, bj);
            h8_t a[MB];
#pragma unroll
            for (int mb = 0; mb < MB; mb++) a[mb] = *reinterpret_cast<const h8_t*>(xb + (16 * mb + bn) * kLdsRow + kk);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                const h8_t b = w0[nb].frag(ks);
#pragma unroll
                for (int mb = 0; mb < MB; mb++) acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mb], b, acc[mb][nb], 0, 0, 0);
            }
        }
        if (FULL) {
            // the other buffer was last read in the previous tile, before its barrier
            // (after the last tile it is not read again)
            store_x(xs + (size_t)((kt + 1 - kt0) & 1) * MT * kLdsRow);
            fetch_x(min(kt + 2, kt_last));
#pragma unroll
            for (int nb = 0; nb < NB; nb++) w0[nb] = w1[nb];
        } else if (kt + 1 < kt1) {
            store_x(xs + (size_t)((kt + 1 - kt0) & 1) * MT * kLdsRow);
            if (kt + 2 < kt1) fetch_x(kt + 2);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) w0[nb] = w1[nb];
        }
        __syncthreads();
    }
    // epilogue: C[m][n] of block (mb, nb): m = 16 mb + 4 bj + i, n = 64 wave + 16 nb + bn
    const int ks = max(1, g.ksplit);
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const int n = n0 + 16 * NB * wave + 16 * nb + bn;
        if (n >= n_rows) continue;
        const float bias = sg.bias && z == 0 ? sg.bias[n] : 0.f;
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 16 * mb + 4 * bj + i;
                if (m >= g.m) continue;
                const float v = acc[mb][nb][i] + bias;
                const size_t o = (size_t)m * g.ldy + sg.col0 + n;
                if (ks > 1) g.part[(size_t)z * g.m * g.ldy + o] = v;
                else if (g.mode == MV_ADD) g.y[o] = g.res[o] + v;
                else g.y[o] = v;
            }
        }
    }
}

template <int TA, int TB, int MT, bool GP = false>
__global__ __launch_bounds__(kGemmThreads) void prefill_gemm_kernel(PrefillGemm g) {
    extern __shared__ __attribute__((aligned(16))) uint16_t plds[];   // X tiles [2][MT][kLdsRow]
    int si = 0;
    if (g.nseg > 1 && (int)blockIdx.x >= g.seg[1].tile0) si = 1;
    if (g.nseg > 2 && (int)blockIdx.x >= g.seg[2].tile0) si = 2;
    const PrefillSeg& sg = g.seg[si];
    const int m0 = blockIdx.y * MT, n0 = ((int)blockIdx.x - sg.tile0) * kGemmTileN;
    const int n_kt = (g.k + kTileK - 1) / kTileK;
    const int ks = max(1, g.ksplit), z = blockIdx.z;
    const int kt0 = (int)((long)n_kt * z / ks), kt1 = (int)((long)n_kt * (z + 1) / ks);
    // Unconditional fetches with exact waits pay at 32-row tiles (batched decode
    // rows: configs[3] decode phase 4.24k -> 4.47k tok/s) and cost at 128-row
    // tiles (512-token prefill 27.2k -> 23.4k tok/s), so only the former use them.
    if (MT != 32 || g.k % kTileK) {   // uniform: a partial last K tile needs the conditional fetches
        if (si == 2 && TB != TA) gemm_tile<TB, MT, false, GP>(g, sg, m0, n0, kt0, kt1, z, plds);
        else gemm_tile<TA, MT, false, GP>(g, sg, m0, n0, kt0, kt1, z, plds);
        return;
    }
    if constexpr (TA == TB) {
        gemm_tile<TA, MT, true, GP>(g, sg, m0, n0, kt0, kt1, z, plds);
    } else {
        if (si == 2) gemm_tile<TB, MT, true, GP>(g, sg, m0, n0, kt0, kt1, z, plds);
        else gemm_tile<TA, MT, true, GP>(g, sg, m0, n0, kt0, kt1, z, plds);
    }
}

// acc + part[0][i] + part[stride][i] + ... + part[(ks - 1) stride][i], added in
// split order; the loads of four splits are issued before any is added, so a
// reduction waits for ks / 4 L2 round trips instead of ks.
__device__ __forceinline__ float4 add_splits(float4 a, const float* part, size_t stride, size_t i, int ks) {
    int z = 0;
    for (; z + 8 <= ks; z += 8) {
        float4 p[8];
#pragma unroll
        for (int q = 0; q < 8; q++) p[q] = *reinterpret_cast<const float4*>(part + (size_t)(z + q) * stride + i);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            a.x += p[q].x; a.y += p[q].y; a.z += p[q].z; a.w += p[q].w;
        }
    }
    for (; z + 4 <= ks; z += 4) {
        float4 p[4];
#pragma unroll
        for (int q = 0; q < 4; q++) p[q] = *reinterpret_cast<const float4*>(part + (size_t)(z + q) * stride + i);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            a.x += p[q].x; a.y += p[q].y; a.z += p[q].z; a.w += p[q].w;
        }
    }
    for (; z < ks; z++) {
        const float4 p = *reinterpret_cast<const float4*>(part + (size_t)z * stride + i);
        a.x += p.x; a.y += p.y; a.z += p.z; a.w += p.w;
    }
    return a;
}

// y = (res) + part[0] + ... + part[ks - 1], in split order (deterministic).
// Four values per thread; n is a multiple of 4.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* part, int ks, size_t n, const float* res,
                                                            float* y) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const float4 v = add_splits(res ? *reinterpret_cast<const float4*>(res + i) : float4{0.f, 0.f, 0.f, 0.f}, part, n, i, ks);
    *reinterpret_cast<float4*>(y + i) = v;
}

// Split-K reduction with the RMSNorm of the next GEMM's input fused: one
// workgroup per row r: y[r] = (res[r]) + part[0][r] + ... (split order), then
// out[r][i] = f16(y[r][i] * inv * w[i]), inv = 1/sqrt(sum(y^2)/n + eps)
// (rms_norm, model_ops.rs:108-157). n is a multiple of 4 and at most 8192.
__global__ __launch_bounds__(256) void splitk_reduce_rms_kernel(const float* part, int ks, int m, int n, const float* res,
                                                                float* y, const float* w, float eps, uint16_t* out) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    const size_t plane = (size_t)m * n, row = (size_t)r * n;
    float4 v[8];
    float ss = 0.f;
    // every sum first (no store in between, so the loads of all of a thread's
    // groups and splits can be in flight together), then the stores
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = 4 * tid + 1024 * j;
        if (i < n)
            v[j] = add_splits(res ? *reinterpret_cast<const float4*>(res + row + i) : float4{0.f, 0.f, 0.f, 0.f}, part,
                              plane, row + i, ks);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = 4 * tid + 1024 * j;
        if (i < n) {
            const float4 a = v[j];
            *reinterpret_cast<float4*>(y + row + i) = a;
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = 4 * tid + 1024 * j;
        if (i < n) {
            const float4 wv = *reinterpret_cast<const float4*>(w + i);
            *reinterpret_cast<uint2*>(out + row + i) =
                uint2{pack_h2(v[j].x * inv * wv.x, v[j].y * inv * wv.y), pack_h2(v[j].z * inv * wv.z, v[j].w * inv * wv.w)};
        }
    }
}

// Split-K reduction of a gate | up GEMM with SwiGLU fused (silu_mul,
// model_ops.rs:318-330): act[r][j] = f16(g / (1 + exp(-g)) * u) for the summed
// g = y[r][j], u = y[r][f + j] (split order); the sums themselves are not
// stored. Four columns per thread; f is a multiple of 4.
__global__ __launch_bounds__(256) void splitk_reduce_silu_kernel(const float* part, int ks, int m, int f, uint16_t* act) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t per_row = (size_t)f / 4;
    if (t >= (size_t)m * per_row) return;
    const size_t r = t / per_row, j = (t % per_row) * 4;
    const size_t plane = (size_t)m * 2 * f, gi = r * 2 * f + j, ui = gi + f;
    const float4 g = add_splits(float4{0.f, 0.f, 0.f, 0.f}, part, plane, gi, ks);
    const float4 u = add_splits(float4{0.f, 0.f, 0.f, 0.f}, part, plane, ui, ks);
    auto sw = [](float a, float b) { return a / (1.0f + expf(-a)) * b; };
    *reinterpret_cast<uint2*>(act + r * f + j) = uint2{pack_h2(sw(g.x, u.x), sw(g.y, u.y)), pack_h2(sw(g.z, u.z), sw(g.w, u.w))};
}

// rows x[m][k] -> f16(rms_norm(x) * w) (rms_norm, model_ops.rs:108-157); w may be null
// (plain conversion). One workgroup per row.
__global__ __launch_bounds__(256) void rows_rms_f16_kernel(const float* x, int k, const float* w, float eps, int norm,
                                                           uint16_t* out, int ldo) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (size_t)r * k;
    // four values per thread and pass, four passes' loads in flight (k is a multiple of 4)
    float inv = 1.0f;
    if (norm) {
        float ss = 0.f;
#pragma unroll 4
        for (int i = 4 * tid; i < k; i += 1024) {
            const float4 a = *reinterpret_cast<const float4*>(xr + i);
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        ss = red[0] + red[1] + red[2] + red[3];
        inv = 1.0f / sqrtf(ss / (float)k + eps);
    }
#pragma unroll 4
    for (int i = 4 * tid; i < k; i += 1024) {
        const float4 a = *reinterpret_cast<const float4*>(xr + i);
        const float4 wv = w ? *reinterpret_cast<const float4*>(w + i) : float4{1.f, 1.f, 1.f, 1.f};
        float v0 = a.x * inv, v1 = a.y * inv, v2 = a.z * inv, v3 = a.w * inv;
        if (w) { v0 = v0 * wv.x; v1 = v1 * wv.y; v2 = v2 * wv.z; v3 = v3 * wv.w; }
        *reinterpret_cast<uint2*>(out + (size_t)r * ldo + i) = uint2{pack_h2(v0, v1), pack_h2(v2, v3)};
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
// 16-row blocks per workgroup: about four (row block, head) tiles, one per wave
// (8 or 16 tiles per workgroup measured slower: one workgroup per CU)
template <int G>
__host__ __device__ constexpr int att_row_blocks() { return G >= 4 ? 1 : 4 / G; }

template <int HD, int G, bool F16KV, int NW>
__global__ __launch_bounds__(64 * NW) void prefill_attention_kernel(PrefillRows p) {
    constexpr int NTH = 64 * NW;                // threads
    constexpr int RB = att_row_blocks<G>() * NW / 4;   // 16-row blocks per workgroup
    constexpr int NT = RB * G;                  // tiles
    constexpr int TPW = (NT + NW - 1) / NW;     // tiles per wave
    constexpr int NC = HD / 32;                 // 32-dim chunks of q.k
    constexpr int ND = HD / 16;                 // 16-dim blocks of the output
    constexpr int KLD = HD + 8;                 // K tile row, halves
    constexpr int VLD = kAttKeys + 4;           // V^T row, halves (8-byte aligned rows)
    constexpr int CPR = HD / 8;                 // 16-byte chunks per cache row
    constexpr int KCH = kAttKeys * CPR / NTH;   // K chunks per thread per tile
    static_assert(KCH >= 1 && KCH * NTH == kAttKeys * CPR, "K tile chunks per thread");
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
        const int tile = wave + NW * t, rb = tile / G, h = tile % G;
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

    // cache tiles in registers (a ring of two: tile t0 + 32 is in flight while
    // tile t0 is computed): K chunks, and V as key pairs for the transposed store.
    // Every load is unconditional: a key past the last position re-reads the last
    // position (written, finite data: its score is masked to -inf and its value
    // meets a zero probability), so the compiler waits for exactly the tile it
    // stores, not for the one behind it.
    struct Tile { u4v_t k[KCH], v[2]; };
    Tile tb[2];
    auto cache_off = [&](int pos, int c8) {
        const int page = p.pages[pos / kPageTokens];
        return ((size_t)(page * p.hkv + kvh) * kPageTokens + pos % kPageTokens) * HD + c8 * 8;
    };
    auto load_tile = [&](Tile& tl, int t0) {
#pragma unroll
        for (int e = 0; e < KCH; e++) {
            const int idx = e * NTH + tid, key = idx / CPR, c8 = idx % CPR, pos = min(t0 + key, last_pos);
            tl.k[e] = *reinterpret_cast<const u4v_t*>(p.kcache + cache_off(pos, c8));
        }
        // threads past VIT load a valid row too (unused), so no load is conditional
        const int kp = (tid % VIT) / CPR, c8 = tid % CPR;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int pos = min(t0 + 2 * kp + e, last_pos);
            tl.v[e] = *reinterpret_cast<const u4v_t*>(p.vcache + cache_off(pos, c8));
        }
    };
    // bfloat16 pair (one dword) -> binary16 pair
    auto to_f16x2 = [](uint32_t w) -> uint32_t {
        if constexpr (F16KV) return w;
        const _Float16 a = (_Float16)__uint_as_float(w << 16), b = (_Float16)__uint_as_float(w & 0xffff0000u);
        return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
    };
    auto store_tile = [&](const Tile& tl) {
#pragma unroll
        for (int e = 0; e < KCH; e++) {
            const int idx = e * NTH + tid, key = idx / CPR, c8 = idx % CPR;
            *reinterpret_cast<u4v_t*>(&ks[key][c8 * 8]) =
                u4v_t{to_f16x2(tl.k[e].x), to_f16x2(tl.k[e].y), to_f16x2(tl.k[e].z), to_f16x2(tl.k[e].w)};
        }
        if (tid < VIT) {
            const int kp = tid / CPR, c8 = tid % CPR;
            const uint32_t a[4] = {to_f16x2(tl.v[0].x), to_f16x2(tl.v[0].y), to_f16x2(tl.v[0].z), to_f16x2(tl.v[0].w)};
            const uint32_t b[4] = {to_f16x2(tl.v[1].x), to_f16x2(tl.v[1].y), to_f16x2(tl.v[1].z), to_f16x2(tl.v[1].w)};
#pragma unroll
            for (int d = 0; d < 8; d++) {
                const uint32_t lo = (a[d / 2] >> (16 * (d & 1))) & 0xffffu, hi = (b[d / 2] >> (16 * (d & 1))) & 0xffffu;
                *reinterpret_cast<uint32_t*>(&vts[c8 * 8 + d][2 * kp]) = lo | (hi << 16);
            }
        }
    };

    // the tiles past the last one re-read the last tile (their loads stay
    // unconditional; they are never stored)
    const int t_last = last_pos / kAttKeys * kAttKeys;
    auto compute = [&](int t0) {
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            const int tile = wave + NW * t, rb = tile / G;
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
    };
    load_tile(tb[0], 0);
    load_tile(tb[1], min(kAttKeys, t_last));
    // tile t0 goes from the register ring into LDS, its slot refills with tile
    // t0 + 64, then tile t0 is computed
    auto step = [&](Tile& tl, int t0) {
        __syncthreads();   // the previous tile is consumed
        store_tile(tl);
        __syncthreads();
        load_tile(tl, min(t0 + 2 * kAttKeys, t_last));
        compute(t0);
    };
    for (int t0 = 0; t0 <= last_pos; t0 += 2 * kAttKeys) {
        step(tb[0], t0);
        if (t0 + kAttKeys > last_pos) break;
        step(tb[1], t0 + kAttKeys);
    }
    // acc[t][d][i] = O^T[dim 16 d + 4 j + i][query qn]
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        const int tile = wave + NW * t, rb = tile / G, h = tile % G;
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

template <int HD, int G, int NW>
hipError_t attention_launch_prefill_nw(const PrefillRows& p, hipStream_t st) {
    constexpr int RB = att_row_blocks<G>() * NW / 4;
    const dim3 grid((p.m + 16 * RB - 1) / (16 * RB), p.hkv);
    if (p.kv_f16) prefill_attention_kernel<HD, G, true, NW><<<grid, 64 * NW, 0, st>>>(p);
    else prefill_attention_kernel<HD, G, false, NW><<<grid, 64 * NW, 0, st>>>(p);
    return hipGetLastError();
}

// Every workgroup streams the whole key range of its rows' KV head through
// LDS, so the K/V bytes read per chunk are (key range) x (workgroups per KV
// head). Over long contexts (a chunk whose last key is past kAttWideKeys)
// 8-wave workgroups take twice the rows, halving those re-reads (configs[4],
// 32K context: the launch is bound by them); short prompts keep 4-wave
// workgroups, which give the GPU more of them.
constexpr int kAttWideKeys = 4096;

template <int HD, int G>
hipError_t attention_launch_prefill(const PrefillRows& p, hipStream_t st) {
    if constexpr (HD == 128) {
        if (p.pos0 + p.m > kAttWideKeys) return attention_launch_prefill_nw<HD, G, 8>(p, st);
    }
    return attention_launch_prefill_nw<HD, G, 4>(p, st);
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
    // The split count with the shortest makespan in K tiles: rounds of
    // resident workgroups (two per CU on 256 CUs, four with 32-row tiles) times K tiles per
    // split, at least 2 K tiles per split, at most 8 splits; ties go to fewer.
    const int mt = gemm_rows_tile(m);
    const int wgs = n_tiles * ((m + mt - 1) / mt);
    const int n_kt = (k + kTileK - 1) / kTileK;
    const int slots = 256 * (mt == 32 ? 4 : 2);
    int best = 1;
    long best_t = -1;
    for (int ks = 1; ks <= 8 && (ks == 1 || n_kt / ks >= 2); ks++) {
        const long rounds = ((long)wgs * ks + slots - 1) / slots;
        const long t = rounds * ((n_kt + ks - 1) / ks);
        if (best_t < 0 || t < best_t) {
            best_t = t;
            best = ks;
        }
    }
    return best;
}

size_t prefill_gemm_lds_bytes() { return (size_t)2 * kTileM * kLdsRow * 2; }

// After the GEMM: the split-K reduction (with the fused step, if any), or the
// fused step on its own for an unsplit GEMM.
static hipError_t gemm_post(const PrefillGemm& g, int ks, hipStream_t st) {
    const float* res = g.mode == MV_ADD ? g.res : nullptr;
    if (ks == 1) {
        if (g.post == GEMM_POST_RMS_F16) return launch_rows_rms_f16(g.y, g.m, g.ldy, g.post_w, g.post_eps, true, g.post_out, g.ldy, st);
        if (g.post == GEMM_POST_SILU_F16) return launch_silu_mul_f16(g.y, g.ldy / 2, g.m, g.post_out, st);
        return hipSuccess;
    }
    if (g.post == GEMM_POST_RMS_F16) {
        splitk_reduce_rms_kernel<<<(unsigned)g.m, 256, 0, st>>>(g.part, ks, g.m, g.ldy, res, g.y, g.post_w, g.post_eps,
                                                                 g.post_out);
        return hipGetLastError();
    }
    if (g.post == GEMM_POST_SILU_F16) {
        const size_t t = (size_t)g.m * (g.ldy / 2) / 4;
        splitk_reduce_silu_kernel<<<(unsigned)((t + 255) / 256), 256, 0, st>>>(g.part, ks, g.m, g.ldy / 2, g.post_out);
        return hipGetLastError();
    }
    const size_t n = (size_t)g.m * g.ldy;
    splitk_reduce_kernel<<<(unsigned)((n / 4 + 255) / 256), 256, 0, st>>>(g.part, ks, n, res, g.y);
    return hipGetLastError();
}

hipError_t launch_prefill_gemm(const PrefillGemm& g, hipStream_t st) {
    if (g.m <= 0 || g.k <= 0 || g.k % 32 || g.nseg < 1 || g.nseg > 3) return hipErrorInvalidValue;
    int tiles = 0;
    for (int i = 0; i < g.nseg; i++) {
        const QMat& w = g.seg[i].w;
        // K-quant rows are whole 256-value super-blocks; Q8_0 rows may end inside a tile
        if (w.k != (uint32_t)g.k || w.rows == 0 || (w.type != 8 && g.k % 256) || g.seg[i].tile0 != tiles)
            return hipErrorInvalidValue;
        if (i < 2 && w.type != g.seg[0].w.type) return hipErrorInvalidValue;
        tiles += gemm_tiles((int)w.rows);
    }
    const uint32_t ta = g.seg[0].w.type, tb = g.seg[g.nseg - 1].w.type;
    // split-K needs the partial workspace and whole float4s of y for the reduction
    if (g.post == GEMM_POST_RMS_F16 && (!g.post_w || !g.post_out || g.ldy > 8192)) return hipErrorInvalidValue;
    if (g.post == GEMM_POST_SILU_F16 && (!g.post_out || g.mode != MV_STORE || g.ldy % 8)) return hipErrorInvalidValue;
    const bool can_split = g.part && ((size_t)g.m * g.ldy) % 4 == 0 && (reinterpret_cast<uintptr_t>(g.y) & 15) == 0 &&
                           (reinterpret_cast<uintptr_t>(g.res) & 15) == 0;
    const int ks = can_split ? max(1, g.ksplit) : 1;
    if (ks > 1 && ks > (g.k + kTileK - 1) / kTileK) return hipErrorInvalidValue;
    const int mt = gemm_rows_tile(g.m);
    const dim3 grid(tiles, (g.m + mt - 1) / mt, ks);
    PrefillGemm gg = g;
    gg.ksplit = ks;
    const size_t lds = (size_t)2 * mt * kLdsRow * 2;
    // the GEMM-ordered copies (QMat::g) when every segment has one
    bool gp = true;
    for (int i = 0; i < g.nseg; i++) gp = gp && g.seg[i].w.g != nullptr && (g.seg[i].w.type == 12 || g.seg[i].w.type == 14);
#define RIBN_PG_LAUNCH(A, B, P)                                                                                 \
    {                                                                                                           \
        hipError_t e;                                                                                           \
        if (mt == 32) {                                                                                         \
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_gemm_kernel<A, B, 32, P>),           \
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);                      \
            if (e != hipSuccess) return e;                                                                      \
            prefill_gemm_kernel<A, B, 32, P><<<grid, kGemmThreads, lds, st>>>(gg);                              \
        } else {                                                                                                \
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_gemm_kernel<A, B, kTileM, P>),       \
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);                      \
            if (e != hipSuccess) return e;                                                                      \
            prefill_gemm_kernel<A, B, kTileM, P><<<grid, kGemmThreads, lds, st>>>(gg);                          \
        }                                                                                                       \
        e = hipGetLastError();                                                                                  \
        if (e != hipSuccess) return e;                                                                          \
        return gemm_post(g, ks, st);                                                                            \
    }
#define RIBN_PG(A, B) \
    if (ta == A && tb == B) RIBN_PG_LAUNCH(A, B, false)
#define RIBN_PG2(A, B)                           \
    if (ta == A && tb == B) {                    \
        if (gp) RIBN_PG_LAUNCH(A, B, true)       \
        RIBN_PG_LAUNCH(A, B, false)              \
    }
    RIBN_PG2(12, 12) RIBN_PG2(14, 14) RIBN_PG(8, 8) RIBN_PG2(12, 14) RIBN_PG2(14, 12) RIBN_PG(12, 8) RIBN_PG(8, 12)
    RIBN_PG(14, 8) RIBN_PG(8, 14)
#undef RIBN_PG
#undef RIBN_PG2
#undef RIBN_PG_LAUNCH
    return hipErrorInvalidValue;
}

hipError_t launch_rows_rms_f16(const float* x, int m, int k, const float* w, float eps, bool norm, uint16_t* out,
                               int ldo, hipStream_t st) {
    if (m <= 0 || k % 4 || ldo % 4) return hipErrorInvalidValue;
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
