// Device code shared by the standalone kernels (kernels.hip) and the persistent
// decode step (step.hip): value-type units, input staging, the matvec ring,
// the decode-attention work item and the cross-workgroup hand-off helpers.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <type_traits>

#include "kernels.h"
#include "lanes.h"

namespace ribn {
namespace {

typedef unsigned u4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
// matvec launches run 4 or 8 waves per workgroup (MvArgs::waves)
constexpr int kMaxMvWaves = 8;
constexpr int kMaxMvThreads = kMaxMvWaves * 64;

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

// Cross-workgroup hand-off inside one kernel. The eight XCD-local L2 caches are
// not coherent with each other and an agent-scope fence writes back or
// invalidates a whole L2 (buffer_wbl2 / buffer_inv), which costs tens of
// microseconds across a grid. Instead, handed-off values move with agent-scope
// atomic stores and loads (coherent per access), each wave waits until its
// stores are acknowledged before its workgroup's arrival is counted, and the
// arrival counter is a device-scope atomic.
template <typename T>
__device__ __forceinline__ void st_agent(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_agent(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Count this workgroup's arrival; true in the last of `total` workgroups,
// which also rearms the counter for the next launch.
__device__ __forceinline__ bool arrive_last(uint32_t* ctr, uint32_t total) {
    __shared__ int last;
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = atomicAdd(ctr, 1u);
        last = old == total - 1;
        if (last) st_agent(ctr, 0u);
    }
    __syncthreads();
    return last != 0;
}

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
        // planes: a = qs, b = unpacked scales (dword p = sc(2p), sc(2p+1), m(2p), m(2p+1)), c = d | dmin
        const uint8_t* dd = w.c + bi * 4;
        float d = canon_f16(dd[0] | (dd[1] << 8)), dmin = canon_f16(dd[2] | (dd[3] << 8));
        uint32_t g = i / 32, j = i % 32;
        const uint8_t* sp = w.b + bi * 16 + (g / 2) * 4;
        uint32_t sc = sp[g % 2], mn = sp[2 + g % 2];
        uint32_t q = (w.a[bi * 128 + (g / 2) * 32 + j] >> ((g % 2) * 4)) & 15u;
        float gs = __fmul_rn(d, (float)sc), gm = __fmul_rn(dmin, (float)mn);
        return __fsub_rn(__fmul_rn(gs, (float)q), gm);
    }
    // Q6_K: scale s of sub-block s is at byte 2c + slot, c = 4(s/8) + s%4, slot = (s/4)%2
    uint32_t g = i / 32, pos = i % 32, chunk = g / 4, variant = g % 4;
    uint32_t lo = (w.a[bi * 128 + chunk * 64 + (variant % 2) * 32 + pos] >> (variant < 2 ? 0 : 4)) & 15u;
    uint32_t hi = (w.b[bi * 64 + chunk * 32 + pos] >> (2 * variant)) & 3u;
    float d = canon_f16(*reinterpret_cast<const uint16_t*>(w.d + bi * 2));
    const uint32_t sidx = g * 2 + pos / 16;
    int8_t sc = (int8_t)w.c[bi * 16 + 2 * (4 * (sidx / 8) + sidx % 4) + (sidx / 4) % 2];
    float gs = __fmul_rn(d, (float)sc);
    return __fmul_rn(gs, (float)((int)(lo | (hi << 4)) - 32));
}

// ---------------------------------------------------------------------------
// Matvec input staging. x (optionally the RMSNorm input: rms_norm model_ops.rs:108,
// x * (1/sqrt(sum/n + eps)) * w) is stored in 16-bit fixed point: each block of
// 64 values has an fp32 scale s = max|v| / 32512 and v ~ s v16 with v16 =
// rint(v / s) (resolution 3e-5 of the block maximum), kept as two signed bytes
// v16 = 256 hi + lo. Every group of 16 values also keeps the fp32 sum X of its
// values (for the Q4_K minima and the Q6_K offset). Products with the quants run
// on v_dot4_i32_i8 and are exact in int32. For an RMSNorm input the blocks hold
// x*w and the normalisation factor 1/sqrt(mean(x^2)+eps) is returned as an
// output multiplier, so x is read once.
//
// LDS layout: [k] int8 parts in unit planes | [k/16] (s, X) pairs | 64 fp32
// reduction slots. Unit planes: plane j (Q4_K/Q6_K: 0..3, Q8_0: 0..1) holds,
// for every unit u of the value type, the 16 bytes that unit's lane reads j-th
// (hi then lo of its first 16 values, then hi and lo of its second 16), so
// lane i of a wave reads the i-th 16 bytes of a plane (no bank conflicts).
__host__ __device__ constexpr size_t mv_red_offset(int k) {
    return ((size_t)k * 2 + (size_t)(k / 16) * 8 + 15) / 16 * 16;
}

// Unit, first plane (hi part; lo part in the next plane) and scale slot of the
// 16 values x[16g .. 16g+16).
template <int T>
__device__ __forceinline__ void plane_of_group(int g, int& unit, int& plane, int& slot) {
    if constexpr (T == 8) {
        unit = g; plane = 0; slot = 0;
    } else if constexpr (T == 12) {
        const int blk = g >> 4, o = (g & 15) * 16, grp = o >> 5, hf = (o & 31) >> 4;
        unit = blk * 8 + (grp >> 1) * 2 + hf;
        plane = (grp & 1) * 2;
        slot = grp & 1;
    } else {
        const int blk = g >> 4, o = (g & 15) * 16, chunk = o >> 7, v = (o & 127) >> 5, hf = (o & 31) >> 4;
        unit = blk * 8 + chunk * 4 + (v & 1) * 2 + hf;
        plane = (v >> 1) * 2;
        slot = v >> 1;
    }
}

// The input of the first NP staging passes (x of groups 0..256 NP - 1, and the
// norm weights of the first pass), loaded before the weight stream of a
// standalone launch so it returns ahead of the weights (loads complete in order).
template <int NP>
struct XPre {
    float4 x[NP][4];
    float4 w[4];
};
template <int NP>
__device__ __forceinline__ void stage_pre(const float* x, const float* norm_w, int k, XPre<NP>& p) {
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const int g = q * (int)blockDim.x + threadIdx.x;
        const bool valid = g < k / 16;
#pragma unroll
        for (int j = 0; j < 4; j++)
            p.x[q][j] = valid ? reinterpret_cast<const float4*>(x)[g * 4 + j] : float4{0.f, 0.f, 0.f, 0.f};
    }
    const bool valid = (int)threadIdx.x < k / 16;
#pragma unroll
    for (int j = 0; j < 4; j++)
        p.w[j] = valid && norm_w ? reinterpret_cast<const float4*>(norm_w)[threadIdx.x * 4 + j] : float4{1.f, 1.f, 1.f, 1.f};
}

// One thread's group g of 16 inputs: x (times the norm weights, when given)
// quantized to 16-bit fixed point into the unit planes, the block scale and the
// group sum into gs; ss gathers the sum of squares of x. All lanes take part
// (the block maximum is a quad reduction).
template <int T>
__device__ __forceinline__ void stage_group(int g, int k, const float4 (&xv)[4], const float4 (&wv)[4], bool norm,
                                            int8_t* xs, float* gs, float& ss) {
    const int n_units = T == 8 ? k / 16 : k / 32;
    const bool valid = g < k / 16;
    u4_t* planes = reinterpret_cast<u4_t*>(xs);
    float v[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float4 t = valid ? xv[j] : float4{0.f, 0.f, 0.f, 0.f};
        ss += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
        if (norm && valid) {
            const float4 w = wv[j];
            t.x *= w.x; t.y *= w.y; t.z *= w.z; t.w *= w.w;
        }
        v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
    }
    float am = 0.f, sum = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        am = fmaxf(am, fabsf(v[j]));
        sum += v[j];
    }
    // maximum over the 4 lanes of a quad (the four groups of a 64-value block)
    am = fmaxf(am, dpp_f<0xB1>(am));
    am = fmaxf(am, dpp_f<0x4E>(am));
    // x ~ s * v16 with v16 = rint(x / s) in [-32512, 32512], s = max|x| / 32512
    // over the 64-value block; v16 = 256 hi + lo with hi, lo signed bytes
    const float sc = am * (1.0f / 32512.0f);
    const float is = am > 0.f ? 32512.0f / am : 0.f;
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t h4 = 0, l4 = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int q = (int)rintf(v[4 * j + b] * is);
            const int hi = (q + 128) >> 8, lo = q - (hi << 8);
            h4 |= ((uint32_t)hi & 0xffu) << (8 * b);
            l4 |= ((uint32_t)lo & 0xffu) << (8 * b);
        }
        hw[j] = h4;
        lw[j] = l4;
    }
    if (valid) {
        int unit, plane, slot;
        plane_of_group<T>(g, unit, plane, slot);
        planes[plane * n_units + unit] = u4_t{hw[0], hw[1], hw[2], hw[3]};
        planes[(plane + 1) * n_units + unit] = u4_t{lw[0], lw[1], lw[2], lw[3]};
        if constexpr (T == 8) {
            gs[unit * 2] = sc;
            gs[unit * 2 + 1] = sum;
        } else {
            gs[unit * 4 + slot] = sc;
            gs[unit * 4 + 2 + slot] = sum;
        }
    }
}

// Stage x (k values, RMSNorm weights optional) into LDS for the matvec; returns
// the RMSNorm inverse 1/sqrt(mean x^2 + eps) (1 without norm), which the
// epilogue applies to the row sums. The first NP passes take their input from
// `pre` (loaded by stage_pre).
template <int T, int NP = 0>
__device__ __forceinline__ float stage_x(const float* x, const float* norm_w, float eps, int k, int8_t* xs, float* gs, float* red,
                         const XPre<NP == 0 ? 1 : NP>* pre = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = (int)blockDim.x;   // 256 or 512 threads (matvec launches choose)
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* w4 = reinterpret_cast<const float4*>(norm_w);
    const bool norm = norm_w != nullptr;
    const int n16 = k / 16;
    float ss = 0.f;
    // thread = one group of 16 values; the four groups of a 64-value block sit in
    // four consecutive lanes, which share the block's scale
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const int g = q * nt + tid;
        if (q * nt < n16) {   // uniform
            float4 wl[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                wl[j] = q == 0 ? pre->w[j] : norm && g < n16 ? w4[g * 4 + j] : float4{1.f, 1.f, 1.f, 1.f};
            stage_group<T>(g, k, pre->x[q], wl, norm, xs, gs, ss);
        }
    }
    for (int base = NP * nt; base < n16; base += nt) {
        const int g = base + tid;
        float4 xl[4], wl[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            xl[j] = g < n16 ? x4[g * 4 + j] : float4{0.f, 0.f, 0.f, 0.f};
            wl[j] = norm && g < n16 ? w4[g * 4 + j] : float4{1.f, 1.f, 1.f, 1.f};
        }
        stage_group<T>(g, k, xl, wl, norm, xs, gs, ss);
    }
    float inv = 1.0f;
    if (norm) {
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        ss = 0.f;
#pragma unroll
        for (int i = 0; i < (nt >> 6); i++) ss += red[i];
        inv = 1.0f / sqrtf(ss / (float)k + eps);
    }
    __syncthreads();
    return inv;
}

// sum_j q_j v16_j over 16 values, exact in int32: q are bytes (4 per dword),
// v16 = 256 hi + lo with the hi and lo bytes in xh and xl. The lo products
// accumulate onto the hi sum shifted by 8.
__device__ __forceinline__ int dot16v(uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3, const u4_t& xh,
                                      const u4_t& xl) {
    int h = __builtin_amdgcn_sdot4((int)q0, (int)xh.x, 0, false);
    h = __builtin_amdgcn_sdot4((int)q1, (int)xh.y, h, false);
    h = __builtin_amdgcn_sdot4((int)q2, (int)xh.z, h, false);
    h = __builtin_amdgcn_sdot4((int)q3, (int)xh.w, h, false);
    int t = h << 8;
    t = __builtin_amdgcn_sdot4((int)q0, (int)xl.x, t, false);
    t = __builtin_amdgcn_sdot4((int)q1, (int)xl.y, t, false);
    t = __builtin_amdgcn_sdot4((int)q2, (int)xl.z, t, false);
    t = __builtin_amdgcn_sdot4((int)q3, (int)xl.w, t, false);
    return t;
}

// ---------------------------------------------------------------------------
// Per-lane work units. A unit is 16 bytes of quants of one row:
//  Q4_K: 8 units per block; unit c holds nibble pairs of groups 2p, 2p+1 (p = c/2),
//        elements 16*(c%2) .. +16 of each group (lib.rs:584-600 layout).
//  Q6_K: 8 units per block; unit c holds ql bytes 16c..16c+15: low nibbles are
//        group 4*(c/4) + (c/2)%2, high nibbles that group + 2 (lib.rs:623-649).
//  Q8_0: 2 units per block (16 int8 each).
// A wave walks 128 consecutive units of a row per load group (two halves of 64:
// lane l takes units g0 + l and g0 + 64 + l), so every row offset is
// wave-uniform and only the lane's fixed offset lives in a vector register.
__device__ __forceinline__ uint32_t ld_nt32(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}
__device__ __forceinline__ uint32_t ld_nt16b(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
}

// base: wave-uniform pointer (scalar registers); off: the lane's 32-bit byte
// offset, so the load uses scalar-base + vector-offset addressing.
__device__ __forceinline__ u4_t ldo_nt16(const uint8_t* base, uint32_t off) { return ld_nt16(base + off); }

template <int T>
struct Unit;

template <>
struct Unit<12> {
    static constexpr int kPerBlock = 8;
    struct Raw { u4_t q; uint32_t s, dd; };
    // unit u of `row`: quants, the lane's scale dword [sc(2p), sc(2p+1), m(2p), m(2p+1)], d|dmin
    // units g0 + lane (g0 a multiple of 64, wave-uniform)
    static __device__ __forceinline__ Raw load_full(const QMat& w, size_t row, int g0, int lane) {
        const size_t bi0 = row * w.nb + (size_t)(g0 >> 3);
        const uint8_t* qa = w.a + (row * w.nb * 128 + (size_t)g0 * 16);
        const uint8_t* sb = w.b + bi0 * 16;
        const uint8_t* dc = w.c + bi0 * 4;
        Raw r;
        r.q = ld_nt16(qa + (uint32_t)(lane * 16));
        r.s = ld_nt32(sb + (uint32_t)((lane >> 3) * 16 + ((lane & 7) >> 1) * 4));
        r.dd = ld_nt32(dc + (uint32_t)((lane >> 3) * 4));
        return r;
    }
    static __device__ __forceinline__ float apply(const Raw& r, int u, const u4_t* xs4, int U, const float* gs, float acc) {
        const float d = h2f(r.dd), dmin = h2f(r.dd >> 16);
        const float4 G = reinterpret_cast<const float4*>(gs)[u];   // s, s, X_a, X_b
        const uint32_t m = 0x0f0f0f0fu;
        // q in [0, 15], |v16| <= 32639: |t| < 2^23, so 24-bit products are exact
        const int ta = dot16v(r.q.x & m, r.q.y & m, r.q.z & m, r.q.w & m, xs4[u], xs4[U + u]);
        const int tb = dot16v((r.q.x >> 4) & m, (r.q.y >> 4) & m, (r.q.z >> 4) & m, (r.q.w >> 4) & m, xs4[2 * U + u],
                              xs4[3 * U + u]);
        // both halves of a unit lie in one 64-value block of x (one scale s):
        // sum_j x_j ((d sc) q_j - dmin m) = d s (sc_a t_a + sc_b t_b) - dmin (m_a X_a + m_b X_b)
        const int comb = __mul24((int)(r.s & 0xffu), ta) + __mul24((int)((r.s >> 8) & 0xffu), tb);
        acc = fmaf(d * G.x, (float)comb, acc);
        const float mins = fmaf((float)(r.s >> 24), G.w, (float)((r.s >> 16) & 0xffu) * G.z);
        return fmaf(-dmin, mins, acc);
    }
};

template <>
struct Unit<14> {
    static constexpr int kPerBlock = 8;
    struct Raw { u4_t ql, qh; uint32_t sc, d; };
    static __device__ __forceinline__ Raw load_full(const QMat& w, size_t row, int g0, int lane) {
        const size_t bi0 = row * w.nb + (size_t)(g0 >> 3);
        const int c = lane & 7;
        Raw r;
        r.ql = ld_nt16(w.a + (row * w.nb * 128 + (size_t)g0 * 16) + (uint32_t)(lane * 16));
        r.qh = ld_nt16(w.b + bi0 * 64 + (uint32_t)((lane >> 3) * 64 + 16 * (2 * (c >> 2) + (c & 1))));
        r.sc = ld_nt16b(w.c + bi0 * 16 + (uint32_t)((lane >> 3) * 16 + 2 * c));
        r.d = ld_nt16b(w.d + bi0 * 2 + (uint32_t)((lane >> 3) * 2));
        return r;
    }
    static __device__ __forceinline__ float apply(const Raw& r, int u, const u4_t* xs4, int U, const float* gs, float acc) {
        const int vb = ((u & 7) >> 1) & 1;
        const uint32_t s1 = 4 - 2 * vb, s2 = 2 * vb;
        const uint32_t m4 = 0x0f0f0f0fu, m30 = 0x30303030u;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t l = dword_at(r.ql, i), h = dword_at(r.qh, i);
            lo[i] = (l & m4) | ((h << s1) & m30);
            hi[i] = ((l >> 4) & m4) | ((h >> s2) & m30);
        }
        const float d = h2f(r.d);
        const float scl = (float)(int8_t)(r.sc & 0xffu), sch = (float)(int8_t)(r.sc >> 8);
        const float4 G = reinterpret_cast<const float4*>(gs)[u];
        const float t0 = (float)dot16v(lo[0], lo[1], lo[2], lo[3], xs4[u], xs4[U + u]);
        const float t1 = (float)dot16v(hi[0], hi[1], hi[2], hi[3], xs4[2 * U + u], xs4[3 * U + u]);
        // sum_j x_j (d sc)(q_j - 32) = (d sc)(s t - 32 X), per 16-value sub-block
        acc = fmaf(d * scl, fmaf(G.x, t0, -32.0f * G.z), acc);
        acc = fmaf(d * sch, fmaf(G.y, t1, -32.0f * G.w), acc);
        return acc;
    }
};

template <>
struct Unit<8> {
    static constexpr int kPerBlock = 2;
    struct Raw { u4_t q; uint32_t d; };
    static __device__ __forceinline__ Raw load_full(const QMat& w, size_t row, int g0, int lane) {
        Raw r;
        r.q = ld_nt16(w.a + (row * w.nb * 32 + (size_t)g0 * 16) + (uint32_t)(lane * 16));
        r.d = ld_nt16b(w.b + (row * w.nb + (size_t)(g0 >> 1)) * 2 + (uint32_t)((lane >> 1) * 2));
        return r;
    }
    static __device__ __forceinline__ float apply(const Raw& r, int u, const u4_t* xs4, int U, const float* gs, float acc) {
        const float2 G = reinterpret_cast<const float2*>(gs)[u];
        const float t = (float)dot16v(r.q.x, r.q.y, r.q.z, r.q.w, xs4[u], xs4[U + u]);
        return fmaf(h2f(r.d) * G.x, t, acc);
    }
};

// A load group: two units of each of the two rows of an item, per lane.
template <int T>
struct Group {
    typename Unit<T>::Raw a0, b0, a1, b1;
};

// Where a wave's work lives: items (two rows each, or one gate/up pair) of one
// segment, walked as a flat sequence of load groups. Every field is wave-uniform.
struct WaveWork {
    QMat wa;
    QMat wb;               // second row's matrix (the up matrix for gate/up pairs)
    int first_item, n_items, n_rows, ngr, n_units;
    int stride;            // waves per workgroup: a wave's items are strided by it
    bool pair;
};

// Loads of one group: wave-uniform row/group base (scalar registers) plus the
// lane's 32-bit offset. Lanes past the end of a row (the last group of a row
// whose unit count is not a multiple of 128) load a valid unit of the same row
// and are masked out in mv_body.
template <int T>
__device__ __forceinline__ void load_group(Group<T>& g, const WaveWork& w, int it, int gi) {
    using U = Unit<T>;
    const int item = w.first_item + it * w.stride;
    const int ra = w.pair ? item : 2 * item;
    const int rb = w.pair ? item : min(ra + 1, w.n_rows - 1);
    const int lane = threadIdx.x & 63;
    const int g0 = gi * 128, g1 = g0 + 64 < w.n_units ? g0 + 64 : 0;
    const int l0 = g0 + lane < w.n_units ? lane : 0, l1 = g1 + lane < w.n_units ? lane : 0;
    g.a0 = U::load_full(w.wa, (size_t)ra, g0, l0);
    g.b0 = U::load_full(w.wb, (size_t)rb, g0, l0);
    g.a1 = U::load_full(w.wa, (size_t)ra, g1, l1);
    g.b1 = U::load_full(w.wb, (size_t)rb, g1, l1);
}

// Position (item, group) of a wave's walk, advanced one load group at a time.
struct Cursor {
    int it, gi;
    __device__ __forceinline__ void next(int ngr) {
        if (++gi == ngr) { gi = 0; ++it; }
    }
};

// The wave's load groups live in a ring of D register slots: slot j is
// computed, then refilled with the group D positions ahead, so D-1 groups of
// 128-bit loads are in flight while one is computed. Every full round issues
// the same D refills (the last one's refills past the end reload the wave's
// last group, which the L2 still holds) and the final round issues none, so
// the compiler's wait counting sees a fixed number of loads behind each slot
// and waits for that slot only. With refills that depend on the position it
// has to assume none was issued and waits for every load in flight.
// Addend of each output row a wave produces (residual for MV_ADD plus bias),
// loaded before the wave's first weight loads so that its latency overlaps
// them: lane 2i holds item i's first row, lane 2i+1 its second (a gate/up
// item's single row in lane 2i). Needs at most 32 items per wave.
__device__ __forceinline__ float mv_addend(const MvSeg& sg, const WaveWork& w, int mode, size_t roff = 0) {
    const int lane = threadIdx.x & 63;
    float v = 0.f;
    if (lane < 2 * w.n_items) {
        const int item = w.first_item + (lane >> 1) * w.stride;
        const int row = w.pair ? item : 2 * item + (lane & 1);
        if (row < w.n_rows && !(w.pair && (lane & 1))) {
            if (mode == MV_ADD) v = sg.res[roff + row];
            if (sg.bias) v += sg.bias[row];
        }
    }
    return v;
}

template <int T, int MODE, int R>
__device__ __forceinline__ void mv_finish(const MvSeg& sg, const WaveWork& w, const Cursor& c, float (&a0)[R],
                                          float (&b0)[R], const float (&oscale)[R], const float (&addend)[R],
                                          uint64_t& best, size_t ldo) {
    if (c.gi != w.ngr - 1) return;
    const int lane = threadIdx.x & 63;
    const int item = w.first_item + c.it * w.stride;
    const int ra = w.pair ? item : 2 * item;
    const int rb = w.pair ? item : ra + 1;
    // (the host keeps a launch with addends at <= 32 items per wave)
    const int al = (2 * c.it) & 63;
#pragma unroll
    for (int r = 0; r < R; r++) {
        // both row sums in one reduction: the permlane32 swap of (a0, b0) leaves
        // {a0[l], a0[l + 32]} in lanes 0-31 and {b0[l - 32], b0[l]} in lanes 32-63,
        // then DPP sums within each half
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(a0[r]), __float_as_uint(b0[r]), false, false);
        float v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        v = xor16_sum(group_sum<16>(v));
        const float ya = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) * oscale[r];
        const float yb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) * oscale[r];
        a0[r] = b0[r] = 0.f;
        const float add_a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(addend[r]), al));
        const float add_b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(addend[r]), al + 1));
        float* const out = sg.out + (size_t)r * ldo;
        if (lane == 0) {
            const bool has_b = !w.pair && rb < w.n_rows;
            // outputs are written through to memory (agent-scope stores) so
            // workgroups on other XCDs read them after a grid barrier
            if constexpr (MODE == MV_ADD) {
                st_agent(out + ra, add_a + ya);
                if (has_b) st_agent(out + rb, add_b + yb);
            } else if constexpr (MODE == MV_SILU) {
                st_agent(out + ra, ya / (1.0f + expf(-ya)) * yb);
            } else {
                const float oa = ya + add_a, ob = yb + add_b;
                st_agent(out + ra, oa);
                if (has_b) st_agent(out + rb, ob);
                if constexpr (MODE == MV_HEAD) {
                    static_assert(R == 1, "the head's argmax epilogue takes one row");
                    best = max(best, argmax_key(oa, (uint32_t)ra));
                    if (has_b) best = max(best, argmax_key(ob, (uint32_t)rb));
                }
            }
        }
    }
}

// R input rows staged rb bytes apart: each weight unit is applied to every row.
template <int T, int R>
__device__ __forceinline__ void mv_group(const Group<T>& g, const WaveWork& w, const Cursor& c, const u4_t* xs4,
                                         const float* gs, size_t rb, float (&a0)[R], float (&b0)[R]) {
    using U = Unit<T>;
    const int u0 = c.gi * 128 + (threadIdx.x & 63), u1 = u0 + 64;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const u4_t* x4 = reinterpret_cast<const u4_t*>(reinterpret_cast<const uint8_t*>(xs4) + r * rb);
        const float* gr = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(gs) + r * rb);
        if (u0 < w.n_units) {
            a0[r] = U::apply(g.a0, u0, x4, w.n_units, gr, a0[r]);
            b0[r] = U::apply(g.b0, u0, x4, w.n_units, gr, b0[r]);
        }
        if (u1 < w.n_units) {
            a0[r] = U::apply(g.a1, u1, x4, w.n_units, gr, a0[r]);
            b0[r] = U::apply(g.b1, u1, x4, w.n_units, gr, b0[r]);
        }
    }
}

// Rows of 129-160 units (k = 4352 ... 5120 for Q4_K / Q6_K, e.g. the 32B
// shape's hidden 5120) take two load groups per item, the second holding at
// most 32 units of each row. That tail group runs with one unit per lane:
// lanes 0-31 take row a's tail units, lanes 32-63 row b's, in slot a0 only,
// so it costs a quarter of a full group's loads and arithmetic.
template <int T>
__device__ __forceinline__ void load_tail(Group<T>& g, const WaveWork& w, int it) {
    using U = Unit<T>;
    const int item = w.first_item + it * w.stride;
    const int ra = w.pair ? item : 2 * item;
    const int rb = w.pair ? item : min(ra + 1, w.n_rows - 1);
    const int lane = threadIdx.x & 63, hi = lane >> 5;
    const int l = 128 + (lane & 31) < w.n_units ? (lane & 31) : 0;
    g.a0 = U::load_full(hi ? w.wb : w.wa, (size_t)(hi ? rb : ra), 128, l);
}
template <int T, int R>
__device__ __forceinline__ void mv_tail(const Group<T>& g, const WaveWork& w, const u4_t* xs4, const float* gs,
                                        float (&a0)[R], float (&b0)[R]) {
    static_assert(R == 1, "tail groups run for one input row");
    using U = Unit<T>;
    const int lane = threadIdx.x & 63, u = 128 + (lane & 31);
    const float t = u < w.n_units ? U::apply(g.a0, u, xs4, w.n_units, gs, 0.f) : 0.f;
    if (lane < 32) a0[0] += t;
    else b0[0] += t;
}

// The input of an attention-output projection whose attention launch left its
// split partials unmerged (AttnArgs::defer):
//   x[h HD + d] = sum_s w_s o_s[h][d] / sum_s w_s l_s,  w_s = 2^(m_s - max_s m_s)
// for query head h (KV head h / G); (o_s, m_s, l_s) is split s's record:
// unnormalized output (binary16), base-2 score maximum, weight sum (m = -inf,
// w = 0 for an empty split). The same log-sum-exp merge as the attention
// launch's own. Each thread merges its group of 16 inputs in registers and
// stages it as stage_x does; the first pass's loads are issued before the
// weight loads (merge_issue), like stage_pre's, as loads complete in order.
struct MergePre {
    u4_t p[kDeferMaxSplits][2];
    float m[kDeferMaxSplits], l[kDeferMaxSplits];
};
__device__ __forceinline__ void merge_issue(const MvArgs& a, int base, MergePre& mp) {
    const int HD = a.parts_hd, G = a.parts_g, ns = a.parts_splits, rec = G * HD + 2 * G;
    const int g = min(base + (int)threadIdx.x, a.k / 16 - 1);
    const int h = 16 * g / HD, d = 16 * g % HD, j = h / G, gg = h % G;
#pragma unroll
    for (int s = 0; s < kDeferMaxSplits; s++) {
        const float* r = a.parts + (size_t)(j * ns + min(s, ns - 1)) * rec;
        const u4_t* q = reinterpret_cast<const u4_t*>(reinterpret_cast<const uint16_t*>(r) + gg * HD + d);
        mp.p[s][0] = q[0];
        mp.p[s][1] = q[1];
        mp.m[s] = r[G * HD + gg];
        mp.l[s] = r[G * HD + G + gg];
    }
}
template <int T>
__device__ __forceinline__ float stage_merged(const MvArgs& a, MergePre& mp, int8_t* xs, float* gs) {
    const int ns = a.parts_splits, nt = (int)blockDim.x, n16 = a.k / 16;
    const float4 ones[4] = {{1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}};
    float ss = 0.f;
    for (int base = 0; base < n16; base += nt) {   // uniform
        if (base > 0) merge_issue(a, base, mp);
        float mx = -INFINITY;
#pragma unroll
        for (int s = 0; s < kDeferMaxSplits; s++)
            if (s < ns) mx = fmaxf(mx, mp.m[s]);
        float den = 0.f, o[16];
#pragma unroll
        for (int e = 0; e < 16; e++) o[e] = 0.f;
#pragma unroll
        for (int s = 0; s < kDeferMaxSplits; s++) {
            const float w = s < ns && mp.m[s] != -INFINITY ? exp2f(mp.m[s] - mx) : 0.f;
            den = fmaf(w, mp.l[s], den);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t word = dword_at(mp.p[s][e >> 2], e & 3);
                o[2 * e] = fmaf(w, (float)__builtin_bit_cast(_Float16, (uint16_t)(word & 0xffffu)), o[2 * e]);
                o[2 * e + 1] = fmaf(w, (float)__builtin_bit_cast(_Float16, (uint16_t)(word >> 16)), o[2 * e + 1]);
            }
        }
        const float inv = 1.0f / den;
        float4 xv[4];
#pragma unroll
        for (int j = 0; j < 4; j++) xv[j] = float4{o[4 * j] * inv, o[4 * j + 1] * inv, o[4 * j + 2] * inv, o[4 * j + 3] * inv};
        stage_group<T>(base + (int)threadIdx.x, a.k, xv, ones, false, xs, gs, ss);
    }
    __syncthreads();
    return 1.0f;
}

// Ring of depth D for a wave with total >= D groups, after stage_x.
// MODE MV_ADD_MERGED: MV_ADD whose input is merged from attention partials (merge_parts).
// R > 1: R input rows (MvArgs::rows, ldx floats apart) staged rb bytes apart in
// LDS, outputs (and residuals) ldo floats apart; each weight unit is loaded
// once and applied to every row.
// TAIL: every item is one full group and one tail group (two groups a row,
// D = 2), so ring slot 0 always holds full groups and slot 1 tail groups.
template <int T, int MODE_, int D, int R, typename Sync, bool TAIL = false>
__device__ __forceinline__ bool mv_ring(const MvArgs& a, const MvSeg& sg, const WaveWork& w, int8_t* xs, float* gs,
                                        float* red, size_t rb, uint64_t& best, Sync&& sync) {
    static_assert(!TAIL || (D == 2 && R == 1), "tail groups alternate with full ones in a 2-deep ring");
    constexpr bool MERGE = MODE_ == MV_ADD_MERGED;
    static_assert(R == 1 || !MERGE, "merged attention partials take one row");
    constexpr int MODE = MERGE ? MV_ADD : MODE_;
    const int total = w.n_items * w.ngr;
    constexpr bool EARLY = std::remove_reference_t<Sync>::kEarlyX && !MERGE;
    // the residual launches (O, down) take a long input without norm: two passes
    // early (k up to 16384 at 512 threads; the rest is loaded while staging). Their
    // norm weights are a compile-time null, so no staging pass holds a conditional
    // load, whose wait would cover the weight loads in flight as well. Four early
    // passes measured slower on the 8B down launch (11.6 us against 10.7 us with
    // the 2-deep Q6_K ring): the extra loads delay the weight stream behind them.
    constexpr int NP = EARLY ? (MODE == MV_ADD ? 2 : 1) : 0;
    const float* const norm_w = MODE == MV_ADD ? nullptr : a.norm_w;
    XPre<NP == 0 ? 1 : NP> pre;
    if constexpr (NP > 0) stage_pre<NP>(a.x, norm_w, a.k, pre);
    MergePre mp;
    if constexpr (MERGE) merge_issue(a, 0, mp);
    float addend[R];
#pragma unroll
    for (int r = 0; r < R; r++) addend[r] = (MODE == MV_ADD || sg.bias) ? mv_addend(sg, w, MODE, (size_t)r * a.ldo) : 0.f;
    Group<T> ring[D];
    Cursor ld{0, 0};
    // A standalone launch issues one group before staging and the rest after it:
    // every workgroup's first loads go out together, and the fewer there are, the
    // sooner the address unit reaches the staging code (8B decode: 593 -> 598-603
    // tok/s against the whole ring first). The persistent step issues the whole
    // ring before its grid barrier, whose wait it overlaps.
    constexpr int DP = std::remove_reference_t<Sync>::kEarlyX ? 1 : D;
#pragma unroll
    for (int j = 0; j < DP; j++) {
        if (TAIL && (j & 1)) load_tail<T>(ring[j], w, ld.it);
        else load_group<T>(ring[j], w, ld.it, ld.gi);
        ld.next(w.ngr);
    }
    int ldq = D;   // index of the group `ld` points at
    if (!sync()) return false;
    const float* const x = a.x;
    const float eps = a.eps;
    const int k = a.k;
    float oscale[R];
    if constexpr (MERGE) {
        oscale[0] = stage_merged<T>(a, mp, xs, gs);
    } else {
        oscale[0] = stage_x<T, NP>(x, norm_w, eps, k, xs, gs, red, &pre);
#pragma unroll
        for (int r = 1; r < R; r++)
            oscale[r] = stage_x<T>(x + (size_t)r * a.ldx, norm_w, eps, k, xs + r * rb,
                                   reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(gs) + r * rb), red);
    }
    sync.mark();
#pragma unroll
    for (int j = DP; j < D; j++) {
        if (TAIL && (j & 1)) load_tail<T>(ring[j], w, ld.it);
        else load_group<T>(ring[j], w, ld.it, ld.gi);
        ld.next(w.ngr);
    }
    const u4_t* xs4 = reinterpret_cast<const u4_t*>(xs);
    float a0[R], b0[R];
#pragma unroll
    for (int r = 0; r < R; r++) a0[r] = b0[r] = 0.f;
    Cursor c{0, 0};
    int q0 = 0;
    for (; q0 + D < total; q0 += D) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            if (TAIL && (j & 1)) {
                if constexpr (TAIL) mv_tail<T, R>(ring[j], w, xs4, gs, a0, b0);
                load_tail<T>(ring[j], w, ld.it);
            } else {
                mv_group<T, R>(ring[j], w, c, xs4, gs, rb, a0, b0);
                load_group<T>(ring[j], w, ld.it, ld.gi);
            }
            if (ldq + 1 < total) {
                ld.next(w.ngr);
                ++ldq;
            }
            mv_finish<T, MODE, R>(sg, w, c, a0, b0, oscale, addend, best, (size_t)a.ldo);
            c.next(w.ngr);
        }
    }
#pragma unroll
    for (int j = 0; j < D; j++) {
        if (q0 + j < total) {
            if (TAIL && (j & 1)) {
                if constexpr (TAIL) mv_tail<T, R>(ring[j], w, xs4, gs, a0, b0);
            } else {
                mv_group<T, R>(ring[j], w, c, xs4, gs, rb, a0, b0);
            }
            mv_finish<T, MODE, R>(sg, w, c, a0, b0, oscale, addend, best, (size_t)a.ldo);
            c.next(w.ngr);
        }
    }
    return true;
}

// Stage the input and run the wave's groups with a ring of depth P (or less
// for a wave with fewer groups). The first loads are issued before `sync`
// (a grid barrier in the persistent step, nothing in a standalone launch).
// Returns false if sync reports a failed barrier.
template <int T, int MODE, int P, int R, typename Sync>
__device__ __forceinline__ bool mv_run(const MvArgs& a, const MvSeg& sg, WaveWork& w, int8_t* xs, float* gs,
                                       float* red, size_t rb, uint64_t& best, Sync&& sync) {
    w.n_units = (int)sg.w.nb * Unit<T>::kPerBlock;
    w.ngr = (w.n_units + 127) / 128;
    const int total = w.n_items * w.ngr;
    // depth: one that divides the wave's group count (no refill past the end),
    // or the full depth when the count is large enough for a few reloads of the
    // last group not to matter
    if constexpr (R == 1 && P >= 2 && std::remove_reference_t<Sync>::kEarlyX) {
        if (w.ngr == 2 && w.n_units - 128 <= 32)
            return mv_ring<T, MODE, 2, R, std::remove_reference_t<Sync>&, true>(a, sg, w, xs, gs, red, rb, best, sync);
    }
    if (total >= P && (total % P == 0 || total >= 3 * P)) return mv_ring<T, MODE, P, R>(a, sg, w, xs, gs, red, rb, best, sync);
    if constexpr (P > 3) {
        if (total >= 3 && total % 3 == 0) return mv_ring<T, MODE, 3, R>(a, sg, w, xs, gs, red, rb, best, sync);
    }
    if constexpr (P > 2) {
        if (total >= 2) return mv_ring<T, MODE, 2, R>(a, sg, w, xs, gs, red, rb, best, sync);
    }
    if (total >= 1) return mv_ring<T, MODE, 1, R>(a, sg, w, xs, gs, red, rb, best, sync);
    // no work: take part in the barrier and the workgroup's staging
    if (!sync()) return false;
#pragma unroll
    for (int r = 0; r < R; r++)
        stage_x<T>(a.x + (size_t)r * a.ldx, a.norm_w, a.eps, a.k, xs + r * rb,
                   reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(gs) + r * rb), red);
    sync.mark();
    return true;
}

struct NoSync {
    static constexpr bool kEarlyX = true;   // the input is ready at launch: load it first
    __device__ __forceinline__ bool operator()() const { return true; }
    __device__ __forceinline__ void mark() const {}
    __device__ __forceinline__ void phase(int) const {}   // profiling hook inside attention_item
};

// One workgroup's share of a matvec launch laid out in `a` (segments, items per
// wave). Workgroups beyond the layout only sync. LDS: staged input at `lds`.
// R > 1: R input rows (see mv_ring), staged mv_red_offset(k) bytes apart.
template <int TA, int TB, int MODE, int PA, int PB, int R = 1, typename Sync>
__device__ __forceinline__ bool mv_wg(const MvArgs& a, int wg, uint8_t* lds, uint64_t& best, Sync&& sync) {
    const size_t rb = mv_red_offset(a.k);
    int8_t* xs = reinterpret_cast<int8_t*>(lds);
    float* gs = reinterpret_cast<float*>(lds + (size_t)a.k * 2);
    float* red = reinterpret_cast<float*>(lds + R * rb);
    int si = 0;
    if (a.nseg > 1 && wg >= a.seg[1].wg_begin) si = 1;
    if (a.nseg > 2 && wg >= a.seg[2].wg_begin) si = 2;
    // descriptors by value: in the persistent step `a` lives in global memory,
    // where the output stores could alias it, so reads through `a` in the loop
    // would be reloaded before every weight load
    const MvSeg sg = a.seg[si];
    const int lwg = wg - sg.wg_begin;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr bool pair = MODE == MV_SILU;
    WaveWork w;
    w.wa = sg.w;
    w.wb = pair ? sg.w2 : sg.w;
    w.pair = pair;
    w.n_rows = (int)sg.w.rows;
    const int nw = (int)blockDim.x >> 6;
    w.stride = nw;
    w.first_item = lwg * sg.ipw * nw + wave;
    const int n_item_total = pair ? w.n_rows : (w.n_rows + 1) / 2;
    w.n_items = max(0, min(sg.ipw, (n_item_total - w.first_item + nw - 1) / nw));
    if (si == 2 && TB != TA) return mv_run<TB, MODE, PB, R>(a, sg, w, xs, gs, red, rb, best, sync);
    return mv_run<TA, MODE, PA, R>(a, sg, w, xs, gs, red, rb, best, sync);
}

// Greedy token of the head launch: first maximum over the vocabulary, NaN
// skipped (model_ops.rs:203-260). Every one of the n_wg workgroups publishes its
// best key; the last to arrive reduces them and writes the token into the
// active sequence (tokens[pos + 1], position advanced).
__device__ __forceinline__ void head_finish(const MvArgs& a, uint64_t best, int wg, int n_wg) {
    __shared__ uint64_t wbest[kMaxMvWaves];
    const int nw = (int)blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) best = max(best, (uint64_t)__shfl_xor(best, o));
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = wbest[0];
        for (int i = 1; i < nw; i++) b = max(b, wbest[i]);
        st_agent(a.head.partial + wg, b);
    }
    if (arrive_last(a.head.counter, n_wg)) {
        uint64_t b = 0ull;
        for (int i = threadIdx.x; i < n_wg; i += (int)blockDim.x) b = max(b, ld_agent(a.head.partial + i));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) b = max(b, (uint64_t)__shfl_xor(b, o));
        __syncthreads();
        if (lane == 0) wbest[wave] = b;
        __syncthreads();
        if (threadIdx.x == 0) {
            b = wbest[0];
            for (int i = 1; i < nw; i++) b = max(b, wbest[i]);
            const uint32_t tok = b ? 0xffffffffu - (uint32_t)(b & 0xffffffffu) : 0u;
            SeqState* s = a.ctl->seq;
            const int pos = s->pos;
            if (pos + 1 <= s->max_ctx) s->tokens[pos + 1] = tok;
            s->last_token = tok;
            s->pos = pos + 1;
        }
    }
}

// ---------------------------------------------------------------------------
// GQA decode attention over the paged KV cache with split-K over the context
// (attn_score_gqa_paged, model_ops.rs:442-590; host equations
// qwen_reference.rs:368-461, dense Qwen3: no gate). Workgroup (split, kv head);
// the G = hq/hkv query heads of a KV head share every K/V load.
//  * each wave streams its own 32-position blocks of the split (16-byte loads
//    straight into registers, the next block issued before the current one is
//    used, a wave's first block before the prologue so its latency overlaps);
//  * prologue: q (G heads) and k of the current token get per-head RMSNorm
//    (qwen_reference.rs:382-400) and NeoX rope from the step table; the
//    workgroup whose split holds the current position appends k, v
//    (kv_append_f16, model_ops.rs:1258);
//  * scores and P.V on MFMA with an online softmax per wave; the waves merge
//    in LDS;
//  * splits are merged by log-sum-exp in the last workgroup of a KV head.
// Every key and value, including the current token's, is used at the cache's
// precision, as the reference reads its F16 cache; q and the probabilities
// enter the MFMAs in binary16.
constexpr int kVtLd = 36;   // halves per row of a wave's transposed V tile (32 positions + pad)

template <int HD, int G>
struct AttnLds {
    float buf[G + 2][HD];                // q heads, k, v of the current token
    float rp[HD];                        // rope cos | sin
    uint16_t kq[HD];                     // the current token's k and v at cache precision
    uint16_t vq[HD];
    uint16_t vts[kWaves][HD][kVtLd];     // per wave: V^T of its current 32-position block
    float red[kWaves][G * HD];           // per wave: unnormalized O rows
    float wst[kWaves][2][G];             // per wave: max, sum; then the merge weights
    float swt[G * kMaxSplits];           // cross-split merge weights
    float stat[2][G];                    // per-head max, sum
    int pg[kMaxSplitTokens / kPageTokens];
};

// One (split, KV head) work item. `pos` is the active position and `pages`
// the sequence's page table. In a standalone launch the raw q/k/v loads go
// first (they do not depend on the position); in the persistent step the first
// K/V tile is fetched before `sync` (the barrier after the QKV projection), as
// cached keys and values do not depend on this step, and q/k/v after it.
// Returns false if sync reports a failed barrier.
template <int HD, int G, bool F16, bool PERSIST, typename Sync>
__device__ bool attention_item(const AttnArgs& a, int split, int kvh, int pos, const int32_t* pages, uint8_t* lds_raw,
                               Sync&& sync) {
    constexpr int CH = HD / 8;                 // 16-byte chunks per row
    constexpr int REC = G * HD + 2 * G;        // partial record floats
    AttnLds<HD, G>& L = *reinterpret_cast<AttnLds<HD, G>*>(lds_raw);
    auto& buf = L.buf;
    auto& red = L.red;
    auto& stat = L.stat;
    auto& pg = L.pg;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int qd = a.hq * HD, kd = a.hkv * HD;
    // prologue layout: LPR lanes per row, 4 consecutive values per lane
    constexpr int LPR = HD / 4;
    constexpr int RPP = kThreads / LPR;              // rows per pass
    constexpr int NP = (G + 2 + RPP - 1) / RPP;      // passes over q heads, k, v
    const int pc = tid % LPR, pr = tid / LPR;
    float4 rawv[NP];
    auto load_rawv = [&]() {
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const int r = j * RPP + pr;
            rawv[j] = float4{0.f, 0.f, 0.f, 0.f};
            if (r < G + 2) {
                const float* src = r < G ? a.raw + (size_t)(kvh * G + r) * HD
                                         : (r == G ? a.raw + qd + kvh * HD : a.raw + qd + kd + kvh * HD);
                rawv[j] = *reinterpret_cast<const float4*>(src + 4 * pc);
            }
        }
    };
    // head-norm weights and rope cos/sin for this lane's columns, fetched with
    // q/k/v so the prologue makes no global load of its own. With rot == HD the
    // rotation pairs column c with c +- HD/2, which sits LPR/2 lanes away.
    const int half = a.rot / 2;
    const bool rope_regs = a.rot == HD;
    float4 nwq{0.f, 0.f, 0.f, 0.f}, nwk{0.f, 0.f, 0.f, 0.f};
    if (a.q_norm) {
        nwq = *reinterpret_cast<const float4*>(a.q_norm + 4 * pc);
        nwk = *reinterpret_cast<const float4*>(a.k_norm + 4 * pc);
    }
    float4 rc{1.f, 1.f, 1.f, 1.f}, rs{0.f, 0.f, 0.f, 0.f};
    float rpv = 0.f;
    auto load_rope = [&]() {
        if (rope_regs) {
            const int p0 = (4 * pc) % half;
            rc = *reinterpret_cast<const float4*>(a.rope + p0);
            rs = *reinterpret_cast<const float4*>(a.rope + half + p0);
        } else if (tid < a.rot) {
            rpv = a.rope[tid];
        }
    };
    if constexpr (!PERSIST) {
        load_rawv();
        load_rope();
    }
    const int ctx = pos + 1;
    int per = (ctx + a.n_splits - 1) / a.n_splits;
    per = (per + kPageTokens - 1) / kPageTokens * kPageTokens;
    if (per > kMaxSplitTokens) {
        // A split wider than the LDS tiles: too few splits for this context.
        // Poison the output instead of touching memory.
        if (split == 0)
            for (int i = tid; i < G * HD; i += kThreads) st_agent(a.out + (size_t)kvh * G * HD + i, __uint_as_float(0x7fc00000u));
        return sync();
    }
    const int t0 = split * per, t1 = min(ctx, t0 + per), n = max(0, t1 - t0);
    const bool owner = t0 <= pos && pos < t1;

    sync.phase(0);
    __syncthreads();   // LDS may still be in use by this workgroup's previous work item
    for (int i = tid; i < n; i += kThreads)
        if ((i & (kPageTokens - 1)) == 0) pg[i / kPageTokens] = pages[(t0 + i) / kPageTokens];
    __syncthreads();
    // The split streams in 32-position blocks, one wave per block (blocks
    // wave, wave + kWaves, ...). Lane (bn, bj) holds the k of positions bn
    // and 16 + bn at dims bj*HD/4 .. +HD/4 (KC 16-byte chunks each), and VIT
    // (position pair, 16-byte chunk) items of v. A wave's first block is in
    // flight during the prologue.
    constexpr int KC = HD / 32;
    constexpr int VIT = CH / 4;
    const int bn = lane & 15, bj = lane >> 4;
    const int nblk = (n + 31) / 32;
    // Every load is unconditional: a position past the split re-reads the split's
    // last position (finite, written data; such positions are masked to -inf
    // before the softmax and their v meets a zero weight), page 0 when the split
    // is empty (then nothing is used). So the same loads are in flight behind each
    // use in every iteration, and the compiler waits for the current block's
    // loads only, not for the next block's prefetch.
    const int nlast = n > 0 ? n - 1 : 0;
    const int nmask = n > 0 ? -1 : 0;
    auto kv_load = [&](int blk, u4_t (&kr)[2][KC], u4_t (&vr)[VIT][2]) {
        const int b0 = blk * 32;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int tc = min(b0 + 16 * h + bn, nlast);
            const int page = pg[tc >> 4] & nmask;
            const uint16_t* src = a.kcache + ((size_t)(page * a.hkv + kvh) * kPageTokens + (tc & 15)) * HD + bj * (HD / 4);
#pragma unroll
            for (int c = 0; c < KC; c++) kr[h][c] = *reinterpret_cast<const u4_t*>(src + 8 * c);
        }
#pragma unroll
        for (int it = 0; it < VIT; it++) {
            const int item = it * 64 + lane, pp = item / CH, c8 = item % CH;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int tc = min(b0 + 2 * pp + e, nlast);
                const int page = pg[tc >> 4] & nmask;
                vr[it][e] = *reinterpret_cast<const u4_t*>(
                    a.vcache + ((size_t)(page * a.hkv + kvh) * kPageTokens + (tc & 15)) * HD + c8 * 8);
            }
        }
    };
    u4_t kr[2][KC], vr[VIT][2];
    kv_load(wave, kr, vr);
    sync.phase(1);
    if (!sync()) return false;
    if constexpr (PERSIST) {
        load_rawv();
        load_rope();
    }
    if (!rope_regs && tid < a.rot) L.rp[tid] = rpv;

    sync.phase(2);
    // -- prologue in registers: per-head norm, rope, q scaled into the log2
    //    domain, the current token's k and v at cache precision
    uint2 cur_k{0u, 0u}, cur_v{0u, 0u};
    bool hold_k = false, hold_v = false;
#pragma unroll
    for (int j = 0; j < NP; j++) {
        const int r = j * RPP + pr;
        float v[4] = {rawv[j].x, rawv[j].y, rawv[j].z, rawv[j].w};
        if (a.q_norm) {
            float ss = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
            ss = group_sum<LPR>(ss);
            const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
            const float4 nw = r < G ? nwq : nwk;
            if (r <= G) {
                v[0] = v[0] * inv * nw.x; v[1] = v[1] * inv * nw.y;
                v[2] = v[2] * inv * nw.z; v[3] = v[3] * inv * nw.w;
            }
        }
        if (rope_regs) {
            float o4[4];
#pragma unroll
            for (int i = 0; i < 4; i++) o4[i] = __shfl_xor(v[i], LPR / 2);
            if (r <= G) {
                const float c[4] = {rc.x, rc.y, rc.z, rc.w}, sn[4] = {rs.x, rs.y, rs.z, rs.w};
                const bool first = 4 * pc < half;
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = first ? v[i] * c[i] - o4[i] * sn[i] : o4[i] * sn[i] + v[i] * c[i];
            }
        }
        if (r < G + 1 && !rope_regs) {
            *reinterpret_cast<float4*>(&buf[r][4 * pc]) = float4{v[0], v[1], v[2], v[3]};
        } else if (r < G) {
            *reinterpret_cast<float4*>(&buf[r][4 * pc]) =
                float4{v[0] * a.scale_log2, v[1] * a.scale_log2, v[2] * a.scale_log2, v[3] * a.scale_log2};
        } else if (r == G) {
            cur_k = uint2{kv_encode(v[0], F16 ? 1 : 0) | (uint32_t)kv_encode(v[1], F16 ? 1 : 0) << 16,
                          kv_encode(v[2], F16 ? 1 : 0) | (uint32_t)kv_encode(v[3], F16 ? 1 : 0) << 16};
            hold_k = true;
        }
        if (r == G + 1) {
            cur_v = uint2{kv_encode(v[0], F16 ? 1 : 0) | (uint32_t)kv_encode(v[1], F16 ? 1 : 0) << 16,
                          kv_encode(v[2], F16 ? 1 : 0) | (uint32_t)kv_encode(v[3], F16 ? 1 : 0) << 16};
            hold_v = true;
        }
    }
    if (!rope_regs) {
        // partial rotary: rotate the first rot columns through LDS
        __syncthreads();
        for (int i = tid; i < (G + 1) * half; i += kThreads) {
            const int r = i / half, p = i % half;
            const float c = L.rp[p], sn = L.rp[half + p];
            const float x0 = buf[r][p], x1 = buf[r][p + half];
            buf[r][p] = x0 * c - x1 * sn;
            buf[r][p + half] = x0 * sn + x1 * c;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const int r = j * RPP + pr;
            if (r == G) {
                const float4 k4 = *reinterpret_cast<const float4*>(&buf[G][4 * pc]);
                cur_k = uint2{kv_encode(k4.x, F16 ? 1 : 0) | (uint32_t)kv_encode(k4.y, F16 ? 1 : 0) << 16,
                              kv_encode(k4.z, F16 ? 1 : 0) | (uint32_t)kv_encode(k4.w, F16 ? 1 : 0) << 16};
                hold_k = true;
            }
        }
        for (int i = tid; i < G * HD; i += kThreads) buf[i / HD][i % HD] *= a.scale_log2;
    }
    if (hold_k) *reinterpret_cast<uint2*>(&L.kq[4 * pc]) = cur_k;
    if (hold_v) *reinterpret_cast<uint2*>(&L.vq[4 * pc]) = cur_v;
    if (owner && (hold_k || hold_v)) {
        const int page = pg[(pos - t0) / kPageTokens], off = pos % kPageTokens;
        uint16_t* dst = (hold_k ? a.kcache : a.vcache) + ((size_t)(page * a.hkv + kvh) * kPageTokens + off) * HD;
        *reinterpret_cast<uint2*>(dst + 4 * pc) = hold_k ? cur_k : cur_v;
    }
    __syncthreads();

    sync.phase(3);
    // -- flash decoding on MFMA (v_mfma_f32_16x16x32_f16), per wave and block:
    //      S^T[pos][head] = K Q^T   A = k chunks, B = q (heads beyond G zero) in
    //                               binary16 with log2(e)/sqrt(hd) folded in;
    //                               step c pairs lane group bj's logical k
    //                               0..7 with dims bj*HD/4 + 8c .. +8
    //      online softmax per head (base 2), P rounded to binary16
    //      O^T[dim][head] += V^T P^T  A = V^T from the wave's transposed LDS
    //                               tile, B = P^T straight from the S^T
    //                               accumulators: lane group bj's logical k
    //                               0..7 are positions 4bj..4bj+3, 16+4bj..+3
    //    The S^T / O^T orientation keeps each head in lane % 16. A bfloat16
    //    cache feeds v_mfma_f32_16x16x32_bf16 as stored; q and P then enter as
    //    two bfloat16 terms each (x = hi + lo, hi = bf16(x), lo = bf16(x - hi):
    //    16 significant bits, finer than binary16), two MFMAs per product.
    //    The current position's k and v come from LDS, not the cache.
    {
        typedef _Float16 h8v_t __attribute__((ext_vector_type(8)));
        typedef __bf16 b8v_t __attribute__((ext_vector_type(8)));
        typedef float f4v_t __attribute__((ext_vector_type(4)));
        constexpr int NDB = HD / 16;   // 16-dim blocks of the output
        // x as bfloat16 hi + lo terms (8 values)
        auto split_bf16 = [](const float (&x)[8], b8v_t& hi, b8v_t& lo) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const __bf16 h = (__bf16)x[e];
                hi[e] = h;
                lo[e] = (__bf16)(x[e] - (float)h);
            }
        };
        h8v_t qb[KC];
        b8v_t qbh[KC], qbl[KC];
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int d = bj * (HD / 4) + 8 * c;
            float4 lo{0.f, 0.f, 0.f, 0.f}, hi{0.f, 0.f, 0.f, 0.f};
            if (bn < G) {
                lo = *reinterpret_cast<const float4*>(&buf[bn][d]);
                hi = *reinterpret_cast<const float4*>(&buf[bn][d + 4]);
            }
            if constexpr (F16) {
                qb[c] = h8v_t{(_Float16)lo.x, (_Float16)lo.y, (_Float16)lo.z, (_Float16)lo.w,
                              (_Float16)hi.x, (_Float16)hi.y, (_Float16)hi.z, (_Float16)hi.w};
            } else {
                const float q8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                split_bf16(q8, qbh[c], qbl[c]);
            }
        }
        const int own = owner ? pos - t0 : -1;   // the current position within the split
        uint32_t* vt = reinterpret_cast<uint32_t*>(&L.vts[wave][0][0]);   // [HD][kVtLd / 2] position pairs
        auto v_stage = [&](int blk, const u4_t (&v)[VIT][2]) {
#pragma unroll
            for (int it = 0; it < VIT; it++) {
                const int item = it * 64 + lane, pp = item / CH, c8 = item % CH;
                const int tl = blk * 32 + 2 * pp;
                const u4_t x = tl == own ? *reinterpret_cast<const u4_t*>(&L.vq[c8 * 8]) : v[it][0];
                const u4_t y = tl + 1 == own ? *reinterpret_cast<const u4_t*>(&L.vq[c8 * 8]) : v[it][1];
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint32_t xw = dword_at(x, w), yw = dword_at(y, w);   // cache precision, as stored
                    vt[(c8 * 8 + 2 * w) * (kVtLd / 2) + pp] = (xw & 0xffffu) | (yw << 16);
                    vt[(c8 * 8 + 2 * w + 1) * (kVtLd / 2) + pp] = (xw >> 16) | (yw & 0xffff0000u);
                }
            }
        };
        f4v_t acc[NDB];
#pragma unroll
        for (int db = 0; db < NDB; db++) acc[db] = f4v_t{0.f, 0.f, 0.f, 0.f};
        float m_run = -INFINITY, l_run = 0.f;   // per head bn; l_run is this lane's share
        // The V^T tile is private to its wave and LDS executes a wave's
        // accesses in order; the compiler barriers keep that order in the code.
        if (wave < nblk) v_stage(wave, vr);
        asm volatile("" ::: "memory");
        // One block's scores, softmax update and O^T accumulation (K in kr, V^T in
        // the wave's LDS tile).
        auto block = [&](int blk) {
            const int b0 = blk * 32;
            f4v_t st[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                if (b0 + 16 * h + bn == own) {
#pragma unroll
                    for (int c = 0; c < KC; c++) kr[h][c] = *reinterpret_cast<const u4_t*>(&L.kq[bj * (HD / 4) + 8 * c]);
                }
                st[h] = f4v_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < KC; c++) {
                    if constexpr (F16) {
                        st[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v_t, kr[h][c]), qb[c], st[h], 0, 0, 0);
                    } else {
                        const b8v_t kb = __builtin_bit_cast(b8v_t, kr[h][c]);
                        st[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qbh[c], st[h], 0, 0, 0);
                        st[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qbl[c], st[h], 0, 0, 0);
                    }
                }
            }
            // positions b0 + 16h + 4bj + i; those past the split are masked
            float bm = -INFINITY;
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (b0 + 16 * h + 4 * bj + i >= n) st[h][i] = -INFINITY;
                    bm = fmaxf(bm, st[h][i]);
                }
            bm = xor32_max(xor16_max(bm));
            const float m_new = fmaxf(m_run, bm);   // finite: every block holds a position
            const float alpha = exp2f(m_run - m_new);
            m_run = m_new;
            float ps[8];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int i = 0; i < 4; i++) ps[4 * h + i] = exp2f(st[h][i] - m_new);
            float lsum = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) lsum += ps[e];
            l_run = l_run * alpha + lsum;
            h8v_t pb;
            b8v_t pbh, pbl;
            if constexpr (F16) {
                pb = h8v_t{(_Float16)ps[0], (_Float16)ps[1], (_Float16)ps[2], (_Float16)ps[3],
                           (_Float16)ps[4], (_Float16)ps[5], (_Float16)ps[6], (_Float16)ps[7]};
            } else {
                split_bf16(ps, pbh, pbl);
            }
            const uint16_t* vrow = &L.vts[wave][0][0];
#pragma unroll
            for (int db = 0; db < NDB; db++) {
                const uint16_t* r = vrow + (16 * db + bn) * kVtLd;
                const uint2 lo = *reinterpret_cast<const uint2*>(r + 4 * bj);
                const uint2 hi = *reinterpret_cast<const uint2*>(r + 16 + 4 * bj);
                const u4_t va{lo.x, lo.y, hi.x, hi.y};
                acc[db] *= alpha;
                if constexpr (F16) {
                    acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v_t, va), pb, acc[db], 0, 0, 0);
                } else {
                    acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8v_t, va), pbh, acc[db], 0, 0, 0);
                    acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8v_t, va), pbl, acc[db], 0, 0, 0);
                }
            }
        };
        // Blocks with a successor in this wave prefetch it; the wave's last block
        // issues no load, so nothing is left in flight behind its use.
        int blk = wave;
        for (; blk + kWaves < nblk; blk += kWaves) {   // wave-uniform
            u4_t kn[2][KC], vn[VIT][2];
            kv_load(blk + kWaves, kn, vn);
            block(blk);
            asm volatile("" ::: "memory");
            v_stage(blk + kWaves, vn);   // after this block's reads
            asm volatile("" ::: "memory");
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int c = 0; c < KC; c++) kr[h][c] = kn[h][c];
        }
        if (blk < nblk) block(blk);
        // -- merge the waves: per-head statistics, then O^T rows
        l_run = xor32_sum(xor16_sum(l_run));
        if (bj == 0 && bn < G) {
            L.wst[wave][0][bn] = m_run;
            L.wst[wave][1][bn] = l_run;
        }
        if (bn < G) {
#pragma unroll
            for (int db = 0; db < NDB; db++)
                *reinterpret_cast<float4*>(&red[wave][bn * HD + 16 * db + 4 * bj]) =
                    float4{acc[db][0], acc[db][1], acc[db][2], acc[db][3]};
        }
        __syncthreads();
        if (tid < G) {
            float mx = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; w++) mx = fmaxf(mx, L.wst[w][0][tid]);
            float lt = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                const float wgt = L.wst[w][0][tid] == -INFINITY ? 0.f : exp2f(L.wst[w][0][tid] - mx);
                L.wst[w][0][tid] = wgt;
                lt += wgt * L.wst[w][1][tid];
            }
            stat[0][tid] = mx;
            stat[1][tid] = lt;
        }
        __syncthreads();
    }
    sync.phase(6);
    const bool direct = a.n_splits == 1;
    float* rec = a.part + ((size_t)kvh * a.n_splits + split) * REC;
    if (a.defer == 1 && !direct) {
        // records left for merge_parts hold the unnormalized output in binary16
        // (pairs of values per word in the record's first G*HD/2 words): half the
        // bytes for every workgroup of the projection that reads them all
        uint32_t* rh = reinterpret_cast<uint32_t*>(rec);
        for (int i2 = tid; i2 < G * HD / 2; i2 += kThreads) {
            const int idx = 2 * i2, g = idx / HD;
            float o0 = 0.f, o1 = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                o0 = fmaf(L.wst[w][0][g], red[w][idx], o0);
                o1 = fmaf(L.wst[w][0][g], red[w][idx + 1], o1);
            }
            const _Float16 h0 = (_Float16)o0, h1 = (_Float16)o1;
            st_agent(rh + i2, (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16));
        }
    } else {
        for (int idx = tid; idx < G * HD; idx += kThreads) {
            const int g = idx / HD;
            float o = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; w++) o = fmaf(L.wst[w][0][g], red[w][idx], o);
            if (direct) st_agent(a.out + (size_t)kvh * G * HD + idx, o / stat[1][g]);
            else st_agent(rec + idx, o);
        }
    }
    if (direct) return true;
    if (tid < G) {
        st_agent(rec + G * HD + tid, n > 0 ? stat[0][tid] : -INFINITY);
        st_agent(rec + G * HD + G + tid, n > 0 ? stat[1][tid] : 0.f);
    }
    if (a.defer) return true;   // a later launch merges the records (merge_parts, attention_merge_kernel)
    sync.phase(7);
    if (!arrive_last(a.counters + kvh, a.n_splits)) return true;
    sync.phase(8);

    // -- merge the splits of this KV head (log-sum-exp in base 2). The split
    //    statistics and the first batch of every output element's partials are
    //    all in flight at once: one round trip for up to SB splits.
    constexpr int NE = (G * HD + kThreads - 1) / kThreads;   // output elements per thread
    constexpr int SB = NE <= 2 ? 16 : 8;                      // splits per batch
    constexpr int GPW = (G + kWaves - 1) / kWaves;   // heads per wave in the statistics
    constexpr int SPL = kMaxSplits / 64;               // splits per lane
    const float* base = a.part + (size_t)kvh * a.n_splits * REC;
    float* swt = L.swt;                                // [G][n_splits] weights
    float mv[GPW][SPL], lv[GPW][SPL];
#pragma unroll
    for (int gi = 0; gi < GPW; gi++)
#pragma unroll
        for (int si = 0; si < SPL; si++) {
            const int g = wave + gi * kWaves, sp = lane + si * 64;
            const bool ok = g < G && sp < a.n_splits;
            mv[gi][si] = ok ? ld_agent(base + (size_t)sp * REC + G * HD + g) : -INFINITY;
            lv[gi][si] = ok ? ld_agent(base + (size_t)sp * REC + G * HD + G + g) : 0.f;
        }
    float pv[NE][SB];
    auto load_batch = [&](int sp0) {
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const int idx = e * kThreads + tid;
#pragma unroll
            for (int j = 0; j < SB; j++)
                pv[e][j] = idx < G * HD && sp0 + j < a.n_splits ? ld_agent(base + (size_t)(sp0 + j) * REC + idx) : 0.f;
        }
    };
    load_batch(0);
    // one wave per head: lanes hold the splits
#pragma unroll
    for (int gi = 0; gi < GPW; gi++) {
        const int g = wave + gi * kWaves;
        if (g < G) {   // wave-uniform
            float mx = -INFINITY;
#pragma unroll
            for (int si = 0; si < SPL; si++) mx = fmaxf(mx, mv[gi][si]);
            mx = wave_max(mx);
            float lt = 0.f;
#pragma unroll
            for (int si = 0; si < SPL; si++) {
                const int sp = lane + si * 64;
                const float wgt = mv[gi][si] == -INFINITY ? 0.f : exp2f(mv[gi][si] - mx);
                lt += lv[gi][si] * wgt;
                if (sp < a.n_splits) swt[g * a.n_splits + sp] = wgt;
            }
            lt = wave_sum(lt);
            if (lane == 0) stat[1][g] = lt;
        }
    }
    __syncthreads();
    float acc[NE];
#pragma unroll
    for (int e = 0; e < NE; e++) acc[e] = 0.f;
    for (int sp0 = 0; sp0 < a.n_splits; sp0 += SB) {
        if (sp0 > 0) load_batch(sp0);
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const int idx = e * kThreads + tid;
            const float* w8 = swt + (idx < G * HD ? idx / HD : 0) * a.n_splits;
#pragma unroll
            for (int j = 0; j < SB; j++)
                if (sp0 + j < a.n_splits) acc[e] = fmaf(pv[e][j], w8[sp0 + j], acc[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < NE; e++) {
        const int idx = e * kThreads + tid;
        if (idx < G * HD) st_agent(a.out + (size_t)kvh * G * HD + idx, acc[e] / stat[1][idx / HD]);
    }
    sync.phase(9);
    return true;
}

}  // namespace
}  // namespace ribn
