// Hand-written HIP kernels for gfx950 (CDNA4, wave64) on ribn's decode path.
//
// Decode at batch 1 streams every weight once per token, so the matvec is the
// hot path and it is HBM-bound. Design:
//  * weights stay in their GGUF block encoding, re-tiled at load into
//    16-byte-aligned planes (kernels.h, QMat) so each lane issues 128-bit
//    non-temporal loads and a wave reads 1 KiB of contiguous quants;
//  * the input vector is staged once per workgroup in LDS as fp16 with a
//    power-of-two scale, plus fp32 sums of every 16 staged values;
//  * quants become fp16 by byte permutes (1024 + q has q in the low mantissa
//    bits) and meet x in v_dot2_f32_f16 with fp32 accumulation; the constant
//    1024 (and the Q6_K/Q8_0 offsets) is removed with the 16-element sums,
//    and the Q4_K minimum term uses the same sums;
//  * RMSNorm is a workgroup prologue; residual add, SwiGLU, q/k head norm +
//    NeoX rope + BF16 KV append, and the vocab argmax are epilogues, so one
//    layer is 5 launches.
// Reference semantics followed: gguf_gemv (nvidia/src/qwen_reference.rs:31-40),
// rms_norm_raw (:550-556), rope (:406-425), attention (:431-461), ffn (:529-539),
// argmax (nvidia/src/model_ops.rs:203-260), dequant (gguf/src/lib.rs:577-649).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "kernels.h"

namespace ribn {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef unsigned u4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kTailBytes = 2048;   // LDS tail: reductions + head-epilogue staging

__device__ __forceinline__ u4_t ld_nt16(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p));
}
__device__ __forceinline__ u4_t ld16(const uint8_t* p) { return *reinterpret_cast<const u4_t*>(p); }
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}
__device__ __forceinline__ uint32_t byte_at(uint32_t v, uint32_t j) { return (v >> (8u * j)) & 0xffu; }
__device__ __forceinline__ uint32_t dword_at(const u4_t& v, uint32_t i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Bytes b0..b3 of `v` (each < 256) -> two fp16 pairs (1024 + b0, 1024 + b1), (1024 + b2, 1024 + b3).
__device__ __forceinline__ h2_t lo_pair(uint32_t v) {
    return __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u));
}
__device__ __forceinline__ h2_t hi_pair(uint32_t v) {
    return __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u));
}
__device__ __forceinline__ float fdot2(h2_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(a, __builtin_bit_cast(h2_t, b), c, false);
}
// sum_{j<16} (1024 + byte_j(q)) * x_j with x as 8 fp16 pairs in xa, xb.
__device__ __forceinline__ float dot16(uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3, const u4_t& xa,
                                       const u4_t& xb) {
    float s = 0.f;
    s = fdot2(lo_pair(q0), xa.x, s);
    s = fdot2(hi_pair(q0), xa.y, s);
    s = fdot2(lo_pair(q1), xa.z, s);
    s = fdot2(hi_pair(q1), xa.w, s);
    s = fdot2(lo_pair(q2), xb.x, s);
    s = fdot2(hi_pair(q2), xb.y, s);
    s = fdot2(lo_pair(q3), xb.z, s);
    s = fdot2(hi_pair(q3), xb.w, s);
    return s;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
// KV cache element encode (bf16 RNE, or binary16 RNE like kv_append_f16, model_ops.rs:1210-1276).
__device__ __forceinline__ uint16_t kv_encode(float f, int f16) {
    return f16 ? __half_as_ushort(__float2half_rn(f)) : f32_to_bf16(f);
}
template <bool F16>
__device__ __forceinline__ float kv_decode(uint32_t b) {
    if constexpr (F16) return __half2float(__ushort_as_half((unsigned short)b));
    else return bf16_to_f32(b);
}

// Monotone key of model_ops.rs:193-199 packed with the inverted index, so
// the u64 maximum is the largest logit with the lowest index. NaN -> 0.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    if (v != v) return 0ull;
    uint32_t bits = __float_as_uint(v);
    uint32_t key = (bits >> 31) ? ~bits : (bits ^ 0x80000000u);
    return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - idx);
}

__device__ __forceinline__ void fence_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }
__device__ __forceinline__ void fence_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

// ---------------------------------------------------------------------------
// Exact dequantization of one element, bit-identical to dequantize_block
// (gguf/src/lib.rs:577-649): separate roundings, no contraction.
__device__ __forceinline__ float canon_f16(uint32_t bits) {
    float v = h2f(bits);
    return (v != v) ? __uint_as_float(0x7fc00000u) : v;   // f16_to_f32: any NaN -> f32::NAN
}

__device__ float deq_elem(const QMat& w, uint32_t row, uint32_t e) {
    const size_t nb = w.nb;
    uint32_t blk = e / (w.type == 8 ? 32u : 256u);
    uint32_t i = e % (w.type == 8 ? 32u : 256u);
    size_t bi = (size_t)row * nb + blk;
    if (w.type == 8) {
        float d = canon_f16(*reinterpret_cast<const uint16_t*>(w.b + bi * 2));
        int8_t q = (int8_t)w.a[bi * 32 + i];
        return __fmul_rn(d, (float)q);
    }
    if (w.type == 12) {
        const uint8_t* h = w.b + bi * 16;
        float d = canon_f16(h[0] | (h[1] << 8)), dmin = canon_f16(h[2] | (h[3] << 8));
        const uint8_t* e12 = h + 4;
        uint32_t g = i / 32, j = i % 32, sc, mn;
        if (g < 4) {
            sc = e12[g] & 63u;
            mn = e12[4 + g] & 63u;
        } else {
            sc = (e12[8 + g - 4] & 15u) | ((e12[g - 4] >> 2) & 0x30u);
            mn = (e12[8 + g - 4] >> 4) | ((e12[4 + g - 4] >> 2) & 0x30u);
        }
        uint32_t q = (w.a[bi * 128 + (g / 2) * 32 + j] >> ((g % 2) * 4)) & 15u;
        float gs = __fmul_rn(d, (float)sc), gm = __fmul_rn(dmin, (float)mn);
        return __fsub_rn(__fmul_rn(gs, (float)q), gm);
    }
    // Q6_K
    uint32_t g = i / 32, pos = i % 32, chunk = g / 4, variant = g % 4;
    uint32_t lo = (w.a[bi * 128 + chunk * 64 + (variant % 2) * 32 + pos] >> (variant < 2 ? 0 : 4)) & 15u;
    uint32_t hi = (w.b[bi * 64 + chunk * 32 + pos] >> (2 * variant)) & 3u;
    float d = canon_f16(*reinterpret_cast<const uint16_t*>(w.d + bi * 2));
    int8_t sc = (int8_t)w.c[bi * 16 + g * 2 + pos / 16];
    float gs = __fmul_rn(d, (float)sc);
    return __fmul_rn(gs, (float)((int)(lo | (hi << 4)) - 32));
}

__global__ __launch_bounds__(kThreads) void dequant_kernel(QMat w, float* out) {
    size_t idx = (size_t)blockIdx.x * kThreads + threadIdx.x;
    size_t total = (size_t)w.rows * w.k;
    if (idx >= total) return;
    out[idx] = deq_elem(w, (uint32_t)(idx / w.k), (uint32_t)(idx % w.k));
}

// Token embedding: one row of token_embd dequantized exactly
// (q4_k_embedding, kernels/quantized/q4_k.cu:1; reference decode.rs:577-582).
__global__ __launch_bounds__(kThreads) void embed_kernel(QMat w, int hidden, float* h, const StepCtl* ctl) {
    const SeqState* s = ctl->seq;
    uint32_t tok = s->tokens[s->pos];
    int e = blockIdx.x * kThreads + threadIdx.x;
    if (e < hidden) h[e] = deq_elem(w, tok, (uint32_t)e);
}

__global__ void advance_kernel(const StepCtl* ctl) {
    if (threadIdx.x == 0) ctl->seq->pos += 1;
}

// ---------------------------------------------------------------------------
// Matvec input staging: x (optionally RMS-normalised, rms_norm model_ops.rs:108)
// -> fp16 in LDS scaled by 2^e so that max|x| lies in [2^14, 2^15), plus fp32
// sums of each 16 staged values. Returns 2^-e, the output scale.
__device__ float stage_x(const MvArgs& a, _Float16* xs, float* gs, float* red) {
    const int k = a.k, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
    const bool norm = a.norm_w != nullptr;
    float ss = 0.f, am = 0.f;
    for (int i = tid; i < k / 4; i += kThreads) {
        float4 v = x4[i];
        if (norm) {
            float4 w = w4[i];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x * w.x), fabsf(v.y * w.y)), fmaxf(fabsf(v.z * w.z), fabsf(v.w * w.w))));
        } else {
            am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    }
    ss = wave_sum(ss);
    am = wave_max(am);
    if (lane == 0) { red[wave] = ss; red[kWaves + wave] = am; }
    __syncthreads();
    ss = 0.f; am = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; i++) { ss += red[i]; am = fmaxf(am, red[kWaves + i]); }
    const float inv = norm ? 1.0f / sqrtf(ss / (float)k + a.eps) : 1.0f;
    float amax = am * inv * 1.0001f;
    int ex = 0;
    if (amax > 0.f && amax < 3.0e38f) frexpf(amax, &ex);
    ex = min(max(15 - ex, -100), 100);
    const float scale = ldexpf(1.0f, ex);
    for (int g = tid; g < k / 16; g += kThreads) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float4 t = x4[g * 4 + j];
            v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
        }
        if (norm) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float4 t = w4[g * 4 + j];
                v[4 * j] = v[4 * j] * inv * t.x;
                v[4 * j + 1] = v[4 * j + 1] * inv * t.y;
                v[4 * j + 2] = v[4 * j + 2] * inv * t.z;
                v[4 * j + 3] = v[4 * j + 3] * inv * t.w;
            }
        }
        float sum = 0.f;
        _Float16 hv[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            hv[j] = (_Float16)(v[j] * scale);
            sum += (float)hv[j];
        }
        u4_t* dst = reinterpret_cast<u4_t*>(xs + g * 16);
        dst[0] = *reinterpret_cast<u4_t*>(&hv[0]);
        dst[1] = *reinterpret_cast<u4_t*>(&hv[8]);
        gs[g] = sum;
    }
    __syncthreads();
    return 1.0f / scale;
}

// ---------------------------------------------------------------------------
// Per-lane work units. A unit is 16 bytes of quants of one row:
//  Q4_K: 8 units per block; unit c holds nibble pairs of groups 2p, 2p+1 (p = c/2),
//        elements 16*(c%2) .. +16 of each group (lib.rs:584-600 layout).
//  Q6_K: 8 units per block; unit c holds ql bytes 16c..16c+15: low nibbles are
//        group 4*(c/4) + (c/2)%2, high nibbles that group + 2 (lib.rs:623-649).
//  Q8_0: 2 units per block (16 int8 each).
template <int T>
struct Unit;

template <>
struct Unit<12> {
    static constexpr int kPerBlock = 8;
    struct Raw { u4_t q, h; };
    static __device__ __forceinline__ Raw load(const QMat& w, size_t row, int u) {
        const size_t nb = w.nb;
        Raw r;
        r.q = ld_nt16(w.a + (row * nb * 128) + (size_t)u * 16);
        r.h = ld16(w.b + (row * nb + (u >> 3)) * 16);
        return r;
    }
    static __device__ __forceinline__ float apply(const Raw& r, int u, const u4_t* xs4, const float* gs, float acc) {
        const int blk = u >> 3, c = u & 7, p = c >> 1, hf = c & 1;
        const uint32_t g0 = 2 * p, g1 = 2 * p + 1;
        uint32_t sc0, sc1, m0, m1;
        if (p < 2) {
            sc0 = byte_at(r.h.y, g0) & 63u; sc1 = byte_at(r.h.y, g1) & 63u;
            m0 = byte_at(r.h.z, g0) & 63u;  m1 = byte_at(r.h.z, g1) & 63u;
        } else {
            const uint32_t j0 = g0 - 4, j1 = g1 - 4;
            sc0 = (byte_at(r.h.w, j0) & 15u) | ((byte_at(r.h.y, j0) >> 2) & 0x30u);
            sc1 = (byte_at(r.h.w, j1) & 15u) | ((byte_at(r.h.y, j1) >> 2) & 0x30u);
            m0 = (byte_at(r.h.w, j0) >> 4) | ((byte_at(r.h.z, j0) >> 2) & 0x30u);
            m1 = (byte_at(r.h.w, j1) >> 4) | ((byte_at(r.h.z, j1) >> 2) & 0x30u);
        }
        const float d = h2f(r.h.x), dmin = h2f(r.h.x >> 16);
        const int xo = blk * 256 + 64 * p + 16 * hf;   // in halves
        const u4_t xa = xs4[xo / 8], xb = xs4[xo / 8 + 1];
        const u4_t ya = xs4[xo / 8 + 4], yb = xs4[xo / 8 + 5];
        const float X0 = gs[xo / 16], X1 = gs[xo / 16 + 2];
        const uint32_t m = 0x0f0f0f0fu;
        const float s0 = dot16(r.q.x & m, r.q.y & m, r.q.z & m, r.q.w & m, xa, xb);
        const float s1 = dot16((r.q.x >> 4) & m, (r.q.y >> 4) & m, (r.q.z >> 4) & m, (r.q.w >> 4) & m, ya, yb);
        acc = fmaf(d * (float)sc0, fmaf(-1024.f, X0, s0), acc);
        acc = fmaf(d * (float)sc1, fmaf(-1024.f, X1, s1), acc);
        acc = fmaf(-dmin * (float)m0, X0, acc);
        acc = fmaf(-dmin * (float)m1, X1, acc);
        return acc;
    }
};

template <>
struct Unit<14> {
    static constexpr int kPerBlock = 8;
    struct Raw { u4_t ql, qh, sc; uint32_t d; };
    static __device__ __forceinline__ Raw load(const QMat& w, size_t row, int u) {
        const size_t nb = w.nb, bi = row * nb + (u >> 3);
        const int c = u & 7;
        Raw r;
        r.ql = ld_nt16(w.a + row * nb * 128 + (size_t)u * 16);
        r.qh = ld_nt16(w.b + bi * 64 + 16 * (2 * (c >> 2) + (c & 1)));
        r.sc = ld16(w.c + bi * 16);
        r.d = *reinterpret_cast<const uint16_t*>(w.d + bi * 2);
        return r;
    }
    static __device__ __forceinline__ float apply(const Raw& r, int u, const u4_t* xs4, const float* gs, float acc) {
        const int blk = u >> 3, c = u & 7, chunk = c >> 2, vb = (c >> 1) & 1, hf = c & 1;
        const uint32_t sl = 2 * vb, sh = 2 * vb + 4;
        const uint32_t m4 = 0x0f0f0f0fu, m2 = 0x03030303u;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t l = dword_at(r.ql, i), h = dword_at(r.qh, i);
            lo[i] = (l & m4) | (((h >> sl) & m2) << 4);
            hi[i] = ((l >> 4) & m4) | (((h >> sh) & m2) << 4);
        }
        const int il = (chunk * 4 + vb) * 2 + hf, ih = il + 4;
        const float scl = (float)(int8_t)byte_at(dword_at(r.sc, il >> 2), il & 3);
        const float sch = (float)(int8_t)byte_at(dword_at(r.sc, ih >> 2), ih & 3);
        const float d = h2f(r.d);
        const int xo = blk * 256 + chunk * 128 + vb * 32 + 16 * hf;
        const u4_t xa = xs4[xo / 8], xb = xs4[xo / 8 + 1];
        const u4_t ya = xs4[xo / 8 + 8], yb = xs4[xo / 8 + 9];
        const float X0 = gs[xo / 16], X1 = gs[xo / 16 + 4];
        const float s0 = dot16(lo[0], lo[1], lo[2], lo[3], xa, xb);
        const float s1 = dot16(hi[0], hi[1], hi[2], hi[3], ya, yb);
        acc = fmaf(d * scl, fmaf(-1056.f, X0, s0), acc);
        acc = fmaf(d * sch, fmaf(-1056.f, X1, s1), acc);
        return acc;
    }
};

template <>
struct Unit<8> {
    static constexpr int kPerBlock = 2;
    struct Raw { u4_t q; uint32_t d; };
    static __device__ __forceinline__ Raw load(const QMat& w, size_t row, int u) {
        const size_t nb = w.nb;
        Raw r;
        r.q = ld_nt16(w.a + row * nb * 32 + (size_t)u * 16);
        r.d = *reinterpret_cast<const uint16_t*>(w.b + (row * nb + (u >> 1)) * 2);
        return r;
    }
    static __device__ __forceinline__ float apply(const Raw& r, int u, const u4_t* xs4, const float* gs, float acc) {
        const uint32_t f = 0x80808080u;
        const int xo = u * 16;
        const float s = dot16(r.q.x ^ f, r.q.y ^ f, r.q.z ^ f, r.q.w ^ f, xs4[xo / 8], xs4[xo / 8 + 1]);
        return fmaf(h2f(r.d), fmaf(-1152.f, gs[u], s), acc);
    }
};

// Two rows (A, B) at once; lanes stride over units, two units in flight per row.
template <int T>
__device__ __forceinline__ void rows2(const QMat& wa, size_t ra, const QMat& wb, size_t rb, const u4_t* xs4,
                                      const float* gs, float& acc_a, float& acc_b) {
    using U = Unit<T>;
    const int n_units = (int)wa.nb * U::kPerBlock;
    const int lane = threadIdx.x & 63;
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
    int u = lane;
    for (; u + 64 < n_units; u += 128) {
        auto pa0 = U::load(wa, ra, u), pb0 = U::load(wb, rb, u);
        auto pa1 = U::load(wa, ra, u + 64), pb1 = U::load(wb, rb, u + 64);
        a0 = U::apply(pa0, u, xs4, gs, a0);
        b0 = U::apply(pb0, u, xs4, gs, b0);
        a1 = U::apply(pa1, u + 64, xs4, gs, a1);
        b1 = U::apply(pb1, u + 64, xs4, gs, b1);
    }
    if (u < n_units) {
        auto pa = U::load(wa, ra, u), pb = U::load(wb, rb, u);
        a0 = U::apply(pa, u, xs4, gs, a0);
        b0 = U::apply(pb, u, xs4, gs, b0);
    }
    acc_a = wave_sum(a0 + a1);
    acc_b = wave_sum(b0 + b1);
}

__device__ __forceinline__ void rows2_any(const QMat& wa, size_t ra, const QMat& wb, size_t rb, const u4_t* xs4,
                                          const float* gs, float& ya, float& yb) {
    switch (wa.type) {
    case 12: rows2<12>(wa, ra, wb, rb, xs4, gs, ya, yb); break;
    case 14: rows2<14>(wa, ra, wb, rb, xs4, gs, ya, yb); break;
    default: rows2<8>(wa, ra, wb, rb, xs4, gs, ya, yb); break;
    }
}

// q/k head epilogue, run by wave 0 of the last workgroup of a head: per-head
// RMSNorm (qwen_reference.rs:382-400, dense Qwen3: stride hd) and NeoX rope
// (:406-425) with theta = pos * base^(-2p/rot); q -> q_out, k -> BF16 cache.
__device__ void head_finish(const MvArgs& a, int kind, int head, float* tmp) {
    const QkvEpi& e = a.qkv;
    const int hd = e.hd, lane = threadIdx.x & 63;
    const SeqState* s = a.ctl->seq;
    const int pos = s->pos;
    const float* src = e.raw + (kind == 0 ? head * hd : e.hq * hd + head * hd);
    const float* nw = kind == 0 ? e.q_norm : e.k_norm;
    float v[4];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = lane + 64 * j;
        v[j] = i < hd ? __builtin_nontemporal_load(src + i) : 0.f;
        ss += v[j] * v[j];
    }
    if (nw) {
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)hd + e.eps);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = lane + 64 * j;
            if (i < hd) v[j] = v[j] * inv * nw[i];
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = lane + 64 * j;
        if (i < hd) tmp[i] = v[j];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const int half = e.rot / 2;
    const int page = s->pages[pos / kPageTokens], off = pos % kPageTokens;
    uint16_t* kdst = e.kcache + ((size_t)(page * e.hkv + head) * kPageTokens + off) * hd;
    float* qdst = e.q_out + head * hd;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = lane + 64 * j;
        if (i >= hd) continue;
        float r;
        if (i < e.rot) {
            const int p = i < half ? i : i - half;
            const float theta = (float)pos * powf(e.rope_base, -(2.0f * (float)p) / (float)e.rot);
            const float sn = sinf(theta), cs = cosf(theta);
            const float x0 = tmp[p], x1 = tmp[p + half];
            r = i < half ? x0 * cs - x1 * sn : x0 * sn + x1 * cs;
        } else {
            r = tmp[i];
        }
        if (kind == 0) qdst[i] = r;
        else kdst[i] = kv_encode(r, e.kv_f16);
    }
}

__global__ __launch_bounds__(kThreads) void matvec_kernel(MvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    _Float16* xs = reinterpret_cast<_Float16*>(lds);
    float* gs = reinterpret_cast<float*>(lds + (size_t)a.k * 2);
    float* tail = gs + a.k / 16;
    const float oscale = stage_x(a, xs, gs, tail);
    const u4_t* xs4 = reinterpret_cast<const u4_t*>(xs);

    const int wg = blockIdx.x;
    int si = 0;
    if (a.nseg > 1 && wg >= a.seg[1].wg_begin) si = 1;
    if (a.nseg > 2 && wg >= a.seg[2].wg_begin) si = 2;
    const MvSeg& sg = a.seg[si];
    const int lwg = wg - sg.wg_begin;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ipw = a.items_per_wave;
    const bool pair = a.mode == MV_SILU;
    const int rows_per_item = pair ? 1 : 2;
    const int n_rows = (int)sg.w.rows;
    uint64_t best = 0ull;

    for (int it = 0; it < ipw; it++) {
        const int item = (lwg * ipw + it) * kWaves + wave;
        const int ra = item * rows_per_item;
        if (ra >= n_rows) break;
        const int rb = pair ? ra : min(ra + 1, n_rows - 1);
        float ya, yb;
        rows2_any(sg.w, (size_t)ra, pair ? sg.w2 : sg.w, (size_t)rb, xs4, gs, ya, yb);
        ya *= oscale;
        yb *= oscale;
        if (lane == 0) {
            const bool has_b = !pair && ra + 1 < n_rows;
            if (sg.bias) {
                ya += sg.bias[ra];
                if (has_b) yb += sg.bias[rb];
            }
            switch (a.mode) {
            case MV_ADD:
                sg.out[ra] += ya;
                if (has_b) sg.out[rb] += yb;
                break;
            case MV_SILU:
                sg.out[ra] = ya / (1.0f + expf(-ya)) * yb;
                break;
            case MV_HEAD:
                sg.out[ra] = ya;
                if (has_b) sg.out[rb] = yb;
                best = max(best, argmax_key(ya, (uint32_t)ra));
                if (has_b) best = max(best, argmax_key(yb, (uint32_t)rb));
                break;
            default:
                sg.out[ra] = ya;
                if (has_b) sg.out[rb] = yb;
                if (a.mode == MV_QKV && sg.kind == 2) {
                    const SeqState* s = a.ctl->seq;
                    const int pos = s->pos, hd = a.qkv.hd;
                    const int page = s->pages[pos / kPageTokens], off = pos % kPageTokens;
                    const int h0 = ra / hd, h1 = rb / hd;
                    a.qkv.vcache[((size_t)(page * a.qkv.hkv + h0) * kPageTokens + off) * hd + ra % hd] = kv_encode(ya, a.qkv.kv_f16);
                    if (has_b)
                        a.qkv.vcache[((size_t)(page * a.qkv.hkv + h1) * kPageTokens + off) * hd + rb % hd] =
                            kv_encode(yb, a.qkv.kv_f16);
                }
                break;
            }
        }
    }

    if (a.mode == MV_QKV && sg.kind < 2) {
        // Last workgroup of a head finishes it (rows per workgroup divide hd).
        __shared__ int is_last;
        const int rows_wg = ipw * kWaves * 2;
        const int head = (lwg * rows_wg) / a.qkv.hd;
        const int per_head = a.qkv.hd / rows_wg;
        uint32_t* ctr = a.qkv.counters + (sg.kind == 0 ? head : a.qkv.hq + head);
        fence_release();   // every wave's row stores complete before the arrival
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t old = atomicAdd(ctr, 1u);
            is_last = (old == (uint32_t)per_head - 1);
        }
        __syncthreads();
        if (is_last) {
            fence_acquire();
            if (wave == 0) head_finish(a, sg.kind, head, tail + 64);
            if (threadIdx.x == 0) *ctr = 0u;
        }
    } else if (a.mode == MV_HEAD) {
        __shared__ uint64_t wbest[kWaves];
        __shared__ int is_last;
        if (lane == 0) wbest[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t b = wbest[0];
            for (int i = 1; i < kWaves; i++) b = max(b, wbest[i]);
            a.head.partial[wg] = b;
            fence_release();
            const uint32_t old = atomicAdd(a.head.counter, 1u);
            is_last = (old == gridDim.x - 1);
        }
        __syncthreads();
        if (is_last) {
            fence_acquire();
            uint64_t b = 0ull;
            for (int i = threadIdx.x; i < (int)gridDim.x; i += kThreads)
                b = max(b, __builtin_nontemporal_load(a.head.partial + i));
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const uint64_t other = __shfl_xor(b, o);
                b = max(b, other);
            }
            if (lane == 0) wbest[wave] = b;
            __syncthreads();
            if (threadIdx.x == 0) {
                b = wbest[0];
                for (int i = 1; i < kWaves; i++) b = max(b, wbest[i]);
                const uint32_t tok = b ? 0xffffffffu - (uint32_t)(b & 0xffffffffu) : 0u;
                SeqState* s = a.ctl->seq;
                const int pos = s->pos;
                if (pos + 1 <= s->max_ctx) s->tokens[pos + 1] = tok;
                s->last_token = tok;
                s->pos = pos + 1;
                *a.head.counter = 0u;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GQA decode attention over the paged BF16 cache with split-K over the
// context (attn_score_gqa_paged, model_ops.rs:442-590; host equations
// qwen_reference.rs:431-461). Workgroup (split, kv head); the G = hq/hkv query
// heads of a KV head share every K/V load. Lanes: LPT = hd/8 lanes per token,
// 8 dims each. Per split: online softmax in base 2; the last workgroup of a KV
// head merges the splits by log-sum-exp.
template <int HD, int G, bool F16>
__global__ __launch_bounds__(kThreads) void attention_kernel(AttnArgs a) {
    constexpr int LPT = HD / 8, TPW = 64 / LPT, NG = kWaves * TPW;
    __shared__ float sm[kWaves][G][HD + 2];
    __shared__ int is_last;
    const int split = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tg = wave * TPW + lane / LPT, dl = lane % LPT;
    const SeqState* s = a.ctl->seq;
    const int ctx = s->pos + 1;
    int per = (ctx + a.n_splits - 1) / a.n_splits;
    per = (per + kPageTokens - 1) / kPageTokens * kPageTokens;
    const int t0 = split * per, t1 = min(ctx, t0 + per);

    float q[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float* qp = a.q + (size_t)(kvh * G + g) * HD + dl * 8;
        const float4 q0 = *reinterpret_cast<const float4*>(qp), q1 = *reinterpret_cast<const float4*>(qp + 4);
        q[g][0] = q0.x * a.scale_log2; q[g][1] = q0.y * a.scale_log2;
        q[g][2] = q0.z * a.scale_log2; q[g][3] = q0.w * a.scale_log2;
        q[g][4] = q1.x * a.scale_log2; q[g][5] = q1.y * a.scale_log2;
        q[g][6] = q1.z * a.scale_log2; q[g][7] = q1.w * a.scale_log2;
    }
    float m[G], l[G], o[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY; l[g] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) o[g][i] = 0.f;
    }
    for (int t = t0 + tg; t < t1; t += NG) {
        const int page = s->pages[t / kPageTokens];
        const size_t base = ((size_t)(page * a.hkv + kvh) * kPageTokens + (t % kPageTokens)) * HD + dl * 8;
        const u4_t kr = *reinterpret_cast<const u4_t*>(a.kcache + base);
        const u4_t vr = *reinterpret_cast<const u4_t*>(a.vcache + base);
        float kf[8], vf[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t kw = dword_at(kr, i), vw = dword_at(vr, i);
            kf[2 * i] = kv_decode<F16>(kw & 0xffffu); kf[2 * i + 1] = kv_decode<F16>(kw >> 16);
            vf[2 * i] = kv_decode<F16>(vw & 0xffffu); vf[2 * i + 1] = kv_decode<F16>(vw >> 16);
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            float sc = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) sc = fmaf(q[g][i], kf[i], sc);
#pragma unroll
            for (int off = 1; off < LPT; off <<= 1) sc += __shfl_xor(sc, off);
            const float mn = fmaxf(m[g], sc);
            const float corr = exp2f(m[g] - mn), p = exp2f(sc - mn);
            l[g] = l[g] * corr + p;
#pragma unroll
            for (int i = 0; i < 8; i++) o[g][i] = fmaf(o[g][i], corr, p * vf[i]);
            m[g] = mn;
        }
    }
    // merge the token groups of a wave
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float mo = __shfl_xor(m[g], off), lo = __shfl_xor(l[g], off);
            const float mn = fmaxf(m[g], mo);
            const float ca = mn == -INFINITY ? 0.f : exp2f(m[g] - mn);
            const float cb = mn == -INFINITY ? 0.f : exp2f(mo - mn);
            l[g] = l[g] * ca + lo * cb;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float oo = __shfl_xor(o[g][i], off);
                o[g][i] = o[g][i] * ca + oo * cb;
            }
            m[g] = mn;
        }
    }
    if (lane < LPT) {
#pragma unroll
        for (int g = 0; g < G; g++) {
#pragma unroll
            for (int i = 0; i < 8; i++) sm[wave][g][dl * 8 + i] = o[g][i];
            if (dl == 0) { sm[wave][g][HD] = m[g]; sm[wave][g][HD + 1] = l[g]; }
        }
    }
    __syncthreads();
    const bool direct = a.n_splits == 1;
    for (int idx = tid; idx < G * HD; idx += kThreads) {
        const int g = idx / HD, d = idx % HD;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; w++) mx = fmaxf(mx, sm[w][g][HD]);
        float lt = 0.f, ot = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float c = mx == -INFINITY ? 0.f : exp2f(sm[w][g][HD] - mx);
            lt += sm[w][g][HD + 1] * c;
            ot += sm[w][g][d] * c;
        }
        const int qh = kvh * G + g;
        if (direct) {
            a.out[qh * HD + d] = ot / lt;
        } else {
            float* p = a.part + ((size_t)qh * a.n_splits + split) * (HD + 2);
            p[d] = ot;
            if (d == 0) { p[HD] = mx; p[HD + 1] = lt; }
        }
    }
    if (direct) return;
    fence_release();   // every wave's partial stores complete before the arrival
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = atomicAdd(a.counters + kvh, 1u);
        is_last = (old == (uint32_t)a.n_splits - 1);
    }
    __syncthreads();
    if (!is_last) return;
    fence_acquire();
    for (int idx = tid; idx < G * HD; idx += kThreads) {
        const int g = idx / HD, d = idx % HD, qh = kvh * G + g;
        const float* p = a.part + (size_t)qh * a.n_splits * (HD + 2);
        float mx = -INFINITY;
        for (int sp = 0; sp < a.n_splits; sp++) mx = fmaxf(mx, __builtin_nontemporal_load(p + sp * (HD + 2) + HD));
        float lt = 0.f, ot = 0.f;
        for (int sp = 0; sp < a.n_splits; sp++) {
            const float ms = __builtin_nontemporal_load(p + sp * (HD + 2) + HD);
            const float c = ms == -INFINITY ? 0.f : exp2f(ms - mx);
            lt += __builtin_nontemporal_load(p + sp * (HD + 2) + HD + 1) * c;
            ot += __builtin_nontemporal_load(p + sp * (HD + 2) + d) * c;
        }
        a.out[qh * HD + d] = ot / lt;
    }
    if (tid == 0) a.counters[kvh] = 0u;
}

// Standalone greedy argmax (model_ops.rs:203-260) used by tests.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* logits, uint32_t n, uint64_t* partial,
                                                          uint32_t* counter, uint32_t* out) {
    __shared__ uint64_t wbest[kWaves];
    __shared__ int is_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t b = 0ull;
    for (uint32_t i = blockIdx.x * kThreads + tid; i < n; i += gridDim.x * kThreads) b = max(b, argmax_key(logits[i], i));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) b = max(b, (uint64_t)__shfl_xor(b, o));
    if (lane == 0) wbest[wave] = b;
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < kWaves; i++) wbest[0] = max(wbest[0], wbest[i]);
        partial[blockIdx.x] = wbest[0];
        fence_release();
        is_last = atomicAdd(counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!is_last) return;
    fence_acquire();
    b = 0ull;
    for (int i = tid; i < (int)gridDim.x; i += kThreads) b = max(b, __builtin_nontemporal_load(partial + i));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) b = max(b, (uint64_t)__shfl_xor(b, o));
    __syncthreads();
    if (lane == 0) wbest[wave] = b;
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < kWaves; i++) wbest[0] = max(wbest[0], wbest[i]);
        *out = wbest[0] ? 0xffffffffu - (uint32_t)(wbest[0] & 0xffffffffu) : 0u;
        *counter = 0u;
    }
}

template <int HD, bool F16>
hipError_t attention_dispatch(const AttnArgs& a, hipStream_t st) {
    dim3 grid(a.n_splits, a.hkv);
    switch (a.hq / a.hkv) {
    case 1: attention_kernel<HD, 1, F16><<<grid, kThreads, 0, st>>>(a); break;
    case 2: attention_kernel<HD, 2, F16><<<grid, kThreads, 0, st>>>(a); break;
    case 3: attention_kernel<HD, 3, F16><<<grid, kThreads, 0, st>>>(a); break;
    case 4: attention_kernel<HD, 4, F16><<<grid, kThreads, 0, st>>>(a); break;
    case 5: attention_kernel<HD, 5, F16><<<grid, kThreads, 0, st>>>(a); break;
    case 6: attention_kernel<HD, 6, F16><<<grid, kThreads, 0, st>>>(a); break;
    case 7: attention_kernel<HD, 7, F16><<<grid, kThreads, 0, st>>>(a); break;
    case 8: attention_kernel<HD, 8, F16><<<grid, kThreads, 0, st>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

size_t matvec_lds_bytes(int k) { return (size_t)k * 2 + (size_t)(k / 16) * 4 + kTailBytes; }

int matvec_rows_per_wg(const MvArgs& a) { return a.items_per_wave * kWaves * (a.mode == MV_SILU ? 1 : 2); }

hipError_t launch_matvec(const MvArgs& a, int n_wg, hipStream_t st) {
    if (n_wg <= 0) return hipErrorInvalidValue;
    matvec_kernel<<<n_wg, kThreads, matvec_lds_bytes(a.k), st>>>(a);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
    if (a.n_splits < 1 || a.n_splits > kMaxSplits || a.hq % a.hkv) return hipErrorInvalidValue;
    if (a.hd == 128) return a.kv_f16 ? attention_dispatch<128, true>(a, st) : attention_dispatch<128, false>(a, st);
    if (a.hd == 64) return a.kv_f16 ? attention_dispatch<64, true>(a, st) : attention_dispatch<64, false>(a, st);
    return hipErrorInvalidValue;
}

hipError_t launch_embed(const QMat& w, int hidden, float* h, const StepCtl* ctl, hipStream_t st) {
    embed_kernel<<<(hidden + kThreads - 1) / kThreads, kThreads, 0, st>>>(w, hidden, h, ctl);
    return hipGetLastError();
}

hipError_t launch_advance(const StepCtl* ctl, hipStream_t st) {
    advance_kernel<<<1, 64, 0, st>>>(ctl);
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
