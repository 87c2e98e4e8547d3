// Integer-dot projections: the reference's experimental GemvMode::IntegerDot
// (crates/nvidia/src/decode.rs:298-312, 1409-1553), lossy by design.
//
//   q8_1 packing      quantize_q8_1 (nvidia/src/activation.cu:1-28): per 32
//                     values d = max|x| / 127, q = round-half-away(x / d), the
//                     header word half(d) | half(sum) << 16 (round to nearest
//                     even) and 8 words of signed bytes. The sum follows the
//                     32-lane xor butterfly (offsets 16, 8, 4, 2, 1), so the
//                     packed words are bit-identical to the reference's. The
//                     rows form fuses the RMSNorm that precedes a projection.
//   intdot matvec     q*_q8_1_gemv[_batch] (kernels/quantized/q4_k_q8_1.cu:40,
//                     86, q6_k_q8_1.cu:37, q8_0_q8_1.cu:27): every weight unit
//                     is read from HBM once and dotted (v_dot4_i32_i8, exact in
//                     int32) against up to kIdMaxMembers packed inputs.
//
// MI355X layout. A launch runs one 8-wave workgroup per compute unit. Each
// workgroup first issues the first load groups of its weight rows, then copies
// the members' packed inputs from L2 into LDS planes laid out like the weight
// units (lane i of a wave reads the i-th 16 bytes of a plane: no bank
// conflicts), with per-unit float4 factors. The weight walk is the register
// ring of the float matvec (16-byte loads of D load groups in flight); each
// unit's scales are decoded once and applied to every member:
//   Q4_K unit (16 values of sub-blocks 2p and 2p+1):
//       acc += (d sc_a) da_a t_a + (d sc_b) da_b t_b - (dmin m_a) S_a - (dmin m_b) S_b
//     with S (the Q8_1 block sum) counted once per 32-value sub-block (the
//     unit holding its first half);
//   Q6_K unit (16 values of sub-blocks s and s + 2, each with its own scale):
//       acc += (d sc_lo) da_lo (t_lo - 32 A_lo) + (d sc_hi) da_hi (t_hi - 32 A_hi)
//     with A the sum of the unit's 16 packed bytes (the -32 offset of the quants);
//   Q8_0 unit (16 values): acc += d da t.
#include <algorithm>

#include "device.h"

namespace ribn {
namespace {

constexpr int kIdWaves = 8;
constexpr int kIdThreads = kIdWaves * 64;

// ---------------------------------------------------------------------------
// Q8_1 packing of one 32-value block by 32 lanes (lane l holds value l). All
// lanes of the wave take part; `valid` only masks the stores.
__device__ __forceinline__ void pack_block(float v, uint32_t* blk, bool valid) {
    const int l = threadIdx.x & 31;
    float mx = fabsf(v), s = v;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off));
        s = s + __shfl_xor(s, off);
    }
    const float d = __fdiv_rn(mx, 127.0f);
    const int q = mx == 0.0f ? 0 : (int)roundf(__fdiv_rn(v, d));
    uint32_t word = (uint32_t)q & 0xffu;
    word |= ((uint32_t)__shfl_down((int)word, 1) & 0xffu) << 8;
    word |= ((uint32_t)__shfl_down((int)word, 2) & 0xffffu) << 16;
    if (!valid) return;
    if ((l & 3) == 0) blk[1 + (l >> 2)] = word;
    if (l == 0)
        blk[0] = (uint32_t)__half_as_ushort(__float2half_rn(d)) |
                 ((uint32_t)__half_as_ushort(__float2half_rn(s)) << 16);
}

// Workgroup (x, r): blocks 8x .. 8x + 7 of row r, one per half-wave. With a
// norm (rms_norm, model_ops.rs:108: x * inv * w with inv = 1 / sqrt(sum / n +
// eps)) every workgroup of the row sums the row's squares itself (the row is
// a few KB in L2), so the packing needs no second launch.
__global__ __launch_bounds__(256) void q8_1_rows_kernel(const float* x, int ldx, int k, const float* norm_w, float eps,
                                                        uint32_t* out) {
    __shared__ float red[4];
    const int r = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* xr = x + (size_t)r * ldx;
    const int nb = k / 32;
    const int b = blockIdx.x * 8 + (tid >> 5);
    const bool valid = b < nb;
    const int i = valid ? b * 32 + (tid & 31) : 0;
    float v = xr[i];
    float inv = 1.0f;
    if (norm_w) {
        const float w = norm_w[i];
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
        int j = tid;
        for (; j + 768 < k; j += 1024) {
            const float a0 = xr[j], a1 = xr[j + 256], a2 = xr[j + 512], a3 = xr[j + 768];
            s0 += a0 * a0; s1 += a1 * a1; s2 += a2 * a2; s3 += a3 * a3;
        }
        for (; j < k; j += 256) s0 += xr[j] * xr[j];
        float ss = wave_sum((s0 + s1) + (s2 + s3));
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        ss = red[0] + red[1] + red[2] + red[3];
        inv = 1.0f / sqrtf(ss / (float)k + eps);
        v = v * inv * w;
    }
    pack_block(v, out + ((size_t)r * nb + (valid ? b : 0)) * 9, valid);
}

__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float* x, size_t nb, uint32_t* out) {
    const size_t b = (size_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const bool valid = b < nb;
    const float v = valid ? x[b * 32 + (threadIdx.x & 31)] : 0.f;
    pack_block(v, out + (valid ? b : 0) * 9, valid);
}

// ---------------------------------------------------------------------------
// LDS planes of the packed inputs, per member: [planes][units] 16-byte entries,
// then one factor entry per unit (float4 for Q4_K / Q6_K, float for Q8_0).
template <int T>
struct Q8Plane {
    static constexpr int kPlanes = T == 8 ? 1 : 2;
    static constexpr int kFactor = T == 8 ? 4 : 16;
    static __host__ __device__ int units(int k) { return T == 8 ? k / 16 : k / 32; }
    static __host__ __device__ size_t member_bytes(int k) { return (size_t)units(k) * (16 * kPlanes + kFactor); }
};

__device__ __forceinline__ float f16_lo(uint32_t w) { return __half2float(__ushort_as_half((unsigned short)(w & 0xffffu))); }

// Copy the members' packed inputs into the planes of type T. A thread takes
// whole 32-value blocks, two at a time: all of a batch's loads are issued
// before any is used, so a batch costs one L2 round trip.
template <int T>
__device__ __forceinline__ void stage_q8(const uint32_t* xq, int k, int members, uint8_t* region) {
    const int nb = k / 32, U = Q8Plane<T>::units(k);
    const size_t mstride = Q8Plane<T>::member_bytes(k);
    const int total = members * nb;
    for (int base = 0; base < total; base += 2 * kIdThreads) {
        uint32_t w[2][9];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int it = base + i * kIdThreads + (int)threadIdx.x;
            const uint32_t* src = xq + (size_t)(it < total ? it : 0) * 9;
#pragma unroll
            for (int j = 0; j < 9; j++) w[i][j] = src[j];
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int it = base + i * kIdThreads + (int)threadIdx.x;
            if (it >= total) continue;
            const int m = it / nb, jb = it - m * nb;
            uint8_t* mr = region + (size_t)m * mstride;
            u4_t* planes = reinterpret_cast<u4_t*>(mr);
            const float da = f16_lo(w[i][0]);
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const u4_t q = u4_t{w[i][1 + 4 * hf], w[i][2 + 4 * hf], w[i][3 + 4 * hf], w[i][4 + 4 * hf]};
                if constexpr (T == 8) {
                    const int u = 2 * jb + hf;
                    planes[u] = q;
                    reinterpret_cast<float*>(mr + (size_t)U * 16)[u] = da;
                } else {
                    const int blk = jb >> 3, g = jb & 7;
                    int u, plane;
                    if constexpr (T == 12) {
                        u = blk * 8 + (g >> 1) * 2 + hf;
                        plane = g & 1;
                    } else {
                        const int v = g & 3;
                        u = blk * 8 + 4 * (g >> 2) + 2 * (v & 1) + hf;
                        plane = v >> 1;
                    }
                    planes[plane * U + u] = q;
                    float* f = reinterpret_cast<float*>(mr + (size_t)U * 32) + (size_t)u * 4;
                    f[plane] = da;
                    if constexpr (T == 12) {
                        // the block sum S enters once per sub-block: with the unit of its first half
                        f[2 + plane] = hf == 0 ? f16_lo(w[i][0] >> 16) : 0.0f;
                    } else {
                        int a = __builtin_amdgcn_sdot4((int)q.x, 0x01010101, 0, false);
                        a = __builtin_amdgcn_sdot4((int)q.y, 0x01010101, a, false);
                        a = __builtin_amdgcn_sdot4((int)q.z, 0x01010101, a, false);
                        a = __builtin_amdgcn_sdot4((int)q.w, 0x01010101, a, false);
                        f[2 + plane] = (float)(32 * a);
                    }
                }
            }
        }
    }
}

__device__ __forceinline__ int dot16(uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3, const u4_t& x) {
    int t = __builtin_amdgcn_sdot4((int)q0, (int)x.x, 0, false);
    t = __builtin_amdgcn_sdot4((int)q1, (int)x.y, t, false);
    t = __builtin_amdgcn_sdot4((int)q2, (int)x.z, t, false);
    return __builtin_amdgcn_sdot4((int)q3, (int)x.w, t, false);
}

// One weight unit against every member's planes.
template <int T, int MB>
struct IdApply;

template <int MB>
struct IdApply<12, MB> {
    static __device__ __forceinline__ void run(const typename Unit<12>::Raw& r, int u, const uint8_t* reg, int U,
                                               size_t ms, int members, float (&acc)[MB]) {
        const float d = h2f(r.dd), dmin = h2f(r.dd >> 16);
        const float ds_a = d * (float)(r.s & 0xffu), ds_b = d * (float)((r.s >> 8) & 0xffu);
        const float dm_a = dmin * (float)((r.s >> 16) & 0xffu), dm_b = dmin * (float)(r.s >> 24);
        const uint32_t m4 = 0x0f0f0f0fu;
        const uint32_t a0 = r.q.x & m4, a1 = r.q.y & m4, a2 = r.q.z & m4, a3 = r.q.w & m4;
        const uint32_t b0 = (r.q.x >> 4) & m4, b1 = (r.q.y >> 4) & m4, b2 = (r.q.z >> 4) & m4, b3 = (r.q.w >> 4) & m4;
#pragma unroll
        for (int m = 0; m < MB; m++) {
            if (m < members) {
                const uint8_t* base = reg + (size_t)m * ms;
                const u4_t* pl = reinterpret_cast<const u4_t*>(base);
                const float4 F = reinterpret_cast<const float4*>(base + (size_t)U * 32)[u];
                const int ta = dot16(a0, a1, a2, a3, pl[u]);
                const int tb = dot16(b0, b1, b2, b3, pl[U + u]);
                float a = fmaf(ds_a * F.x, (float)ta, acc[m]);
                a = fmaf(ds_b * F.y, (float)tb, a);
                a = fmaf(-dm_a, F.z, a);
                acc[m] = fmaf(-dm_b, F.w, a);
            }
        }
    }
};

template <int MB>
struct IdApply<14, MB> {
    static __device__ __forceinline__ void run(const typename Unit<14>::Raw& r, int u, const uint8_t* reg, int U,
                                               size_t ms, int members, float (&acc)[MB]) {
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
        const float dl = d * (float)(int8_t)(r.sc & 0xffu), dh = d * (float)(int8_t)(r.sc >> 8);
#pragma unroll
        for (int m = 0; m < MB; m++) {
            if (m < members) {
                const uint8_t* base = reg + (size_t)m * ms;
                const u4_t* pl = reinterpret_cast<const u4_t*>(base);
                const float4 F = reinterpret_cast<const float4*>(base + (size_t)U * 32)[u];
                const int tl = dot16(lo[0], lo[1], lo[2], lo[3], pl[u]);
                const int th = dot16(hi[0], hi[1], hi[2], hi[3], pl[U + u]);
                const float a = fmaf(dl * F.x, (float)tl - F.z, acc[m]);
                acc[m] = fmaf(dh * F.y, (float)th - F.w, a);
            }
        }
    }
};

template <int MB>
struct IdApply<8, MB> {
    static __device__ __forceinline__ void run(const typename Unit<8>::Raw& r, int u, const uint8_t* reg, int U,
                                               size_t ms, int members, float (&acc)[MB]) {
        const float d = h2f(r.d);
#pragma unroll
        for (int m = 0; m < MB; m++) {
            if (m < members) {
                const uint8_t* base = reg + (size_t)m * ms;
                const float f = reinterpret_cast<const float*>(base + (size_t)U * 16)[u];
                const int t = dot16(r.q.x, r.q.y, r.q.z, r.q.w, reinterpret_cast<const u4_t*>(base)[u]);
                acc[m] = fmaf(d * f, (float)t, acc[m]);
            }
        }
    }
};

template <int T, int MB>
__device__ __forceinline__ void id_group(const Group<T>& g, const WaveWork& w, const Cursor& c, const uint8_t* reg,
                                         int U, size_t ms, int members, float (&a)[MB], float (&b)[MB]) {
    const int u0 = c.gi * 128 + (threadIdx.x & 63), u1 = u0 + 64;
    if (u0 < w.n_units) {
        IdApply<T, MB>::run(g.a0, u0, reg, U, ms, members, a);
        IdApply<T, MB>::run(g.b0, u0, reg, U, ms, members, b);
    }
    if (u1 < w.n_units) {
        IdApply<T, MB>::run(g.a1, u1, reg, U, ms, members, a);
        IdApply<T, MB>::run(g.b1, u1, reg, U, ms, members, b);
    }
}

// After an item's last group: the wave sums of both rows for every member,
// then lane m writes member m's outputs.
template <int MODE, int MB>
__device__ __forceinline__ void id_finish(const IdArgs& p, const MvSeg& sg, const WaveWork& w, const Cursor& c,
                                          float (&a)[MB], float (&b)[MB]) {
    if (c.gi != w.ngr - 1) return;
    const int lane = threadIdx.x & 63;
    float va = 0.f, vb = 0.f;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        if (m < p.members) {
            // {a[l], a[l + 32]} in lanes 0-31 and {b[l - 32], b[l]} in lanes 32-63, then sums within each half
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[m]), __float_as_uint(b[m]), false, false);
            float v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
            v = xor16_sum(group_sum<16>(v));
            const float ya = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
            const float yb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
            if (lane == m) { va = ya; vb = yb; }
            a[m] = b[m] = 0.f;
        }
    }
    const int item = w.first_item + c.it * w.stride;
    const int ra = w.pair ? item : 2 * item;
    const int rb = w.pair ? item : ra + 1;
    const bool has_b = !w.pair && rb < w.n_rows;
    if (lane < p.members) {
        float* o = sg.out + (size_t)lane * p.ld;
        if constexpr (MODE == MV_ADD) {
            const float* rs = sg.res + (size_t)lane * p.ld;
            o[ra] = rs[ra] + va;
            if (has_b) o[rb] = rs[rb] + vb;
        } else if constexpr (MODE == MV_SILU) {
            o[ra] = va / (1.0f + expf(-va)) * vb;
        } else {
            o[ra] = sg.bias ? va + sg.bias[ra] : va;
            if (has_b) o[rb] = sg.bias ? vb + sg.bias[rb] : vb;
        }
    }
}

template <int TA, int TB>
__device__ __forceinline__ void id_stage_all(const IdArgs& p, uint8_t* lds) {
    stage_q8<TA>(p.xq, p.k, p.members, lds);
    if constexpr (TB != TA)
        if (p.nseg > 2) stage_q8<TB>(p.xq, p.k, p.members, lds + (size_t)p.members * Q8Plane<TA>::member_bytes(p.k));
}

// The ring of D load groups of the float matvec: the wave issues its first D
// groups, the workgroup stages the packed inputs (their loads queue behind the
// weight loads), and each group is refilled with the one D positions ahead
// right after it is used.
template <int T, int TA, int TB, int MODE, int MB, int D>
__device__ __forceinline__ void id_ring(const IdArgs& p, const MvSeg& sg, const WaveWork& w, uint8_t* lds,
                                        const uint8_t* reg) {
    const int total = w.n_items * w.ngr;
    Group<T> ring[D];
    Cursor ld{0, 0};
#pragma unroll
    for (int j = 0; j < D; j++) {
        load_group<T>(ring[j], w, ld.it, ld.gi);
        ld.next(w.ngr);
    }
    int ldq = D;
    id_stage_all<TA, TB>(p, lds);
    __syncthreads();
    const int U = Q8Plane<T>::units(p.k);
    const size_t ms = Q8Plane<T>::member_bytes(p.k);
    float a[MB], b[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) a[m] = b[m] = 0.f;
    Cursor c{0, 0};
    int q0 = 0;
    for (; q0 + D < total; q0 += D) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            id_group<T, MB>(ring[j], w, c, reg, U, ms, p.members, a, b);
            load_group<T>(ring[j], w, ld.it, ld.gi);
            if (ldq + 1 < total) {
                ld.next(w.ngr);
                ++ldq;
            }
            id_finish<MODE, MB>(p, sg, w, c, a, b);
            c.next(w.ngr);
        }
    }
#pragma unroll
    for (int j = 0; j < D; j++) {
        if (q0 + j < total) {
            id_group<T, MB>(ring[j], w, c, reg, U, ms, p.members, a, b);
            id_finish<MODE, MB>(p, sg, w, c, a, b);
            c.next(w.ngr);
        }
    }
}

// Ring depth 2 (as the float matvec's Q4_K ring; deeper rings spill with the
// member accumulators), 1 for a wave with a single group.
template <int T, int TA, int TB, int MODE, int MB>
__device__ __forceinline__ void id_run(const IdArgs& p, const MvSeg& sg, WaveWork& w, uint8_t* lds, const uint8_t* reg) {
    w.n_units = (int)sg.w.nb * Unit<T>::kPerBlock;
    w.ngr = (w.n_units + 127) / 128;
    const int total = w.n_items * w.ngr;
    if (total >= 2) {
        id_ring<T, TA, TB, MODE, MB, 2>(p, sg, w, lds, reg);
    } else if (total >= 1) {
        id_ring<T, TA, TB, MODE, MB, 1>(p, sg, w, lds, reg);
    } else {
        id_stage_all<TA, TB>(p, lds);   // no rows: take part in the staging and the barrier
        __syncthreads();
    }
}

// Workgroup wg of the launch: its segment, its waves' items (two rows, or one
// gate/up pair, per item), items strided by the wave count.
template <int TA, int TB, int MODE, int MB>
__global__ __launch_bounds__(kIdThreads) void intdot_kernel(IdArgs p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int wg = blockIdx.x;
    int si = 0;
    if (p.nseg > 1 && wg >= p.seg[1].wg_begin) si = 1;
    if (p.nseg > 2 && wg >= p.seg[2].wg_begin) si = 2;
    const MvSeg sg = p.seg[si];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr bool pair = MODE == MV_SILU;
    WaveWork w;
    w.wa = sg.w;
    w.wb = pair ? sg.w2 : sg.w;
    w.pair = pair;
    w.n_rows = (int)sg.w.rows;
    w.stride = kIdWaves;
    w.first_item = (wg - sg.wg_begin) * sg.ipw * kIdWaves + wave;
    const int n_item_total = pair ? w.n_rows : (w.n_rows + 1) / 2;
    w.n_items = max(0, min(sg.ipw, (n_item_total - w.first_item + kIdWaves - 1) / kIdWaves));
    if constexpr (TB != TA) {
        if (si == 2) {
            const uint8_t* reg = lds + (size_t)p.members * Q8Plane<TA>::member_bytes(p.k);
            id_run<TB, TA, TB, MODE, MB>(p, sg, w, lds, reg);
            return;
        }
    }
    id_run<TA, TA, TB, MODE, MB>(p, sg, w, lds, lds);
}

size_t intdot_lds(const IdArgs& p) {
    const uint32_t tb = p.nseg > 2 ? p.type_b : p.type_a;
    auto bytes = [&](uint32_t t) {
        return t == 8 ? Q8Plane<8>::member_bytes(p.k) : t == 12 ? Q8Plane<12>::member_bytes(p.k) : Q8Plane<14>::member_bytes(p.k);
    };
    size_t b = bytes(p.type_a) * (size_t)p.members;
    if (tb != p.type_a) b += bytes(tb) * (size_t)p.members;
    return b;
}

template <int TA, int TB, int MODE, int MB>
hipError_t id_launch(const IdArgs& p, int n_wg, size_t lds, hipStream_t st) {
    if (lds > 65536) {   // per device, so on every launch that needs it
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&intdot_kernel<TA, TB, MODE, MB>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    intdot_kernel<TA, TB, MODE, MB><<<n_wg, kIdThreads, lds, st>>>(p);
    return hipGetLastError();
}

template <int TA, int TB, int MODE>
hipError_t id_members(const IdArgs& p, int n_wg, size_t lds, hipStream_t st) {
    if (p.members <= 1) return id_launch<TA, TB, MODE, 1>(p, n_wg, lds, st);
    if (p.members <= 2) return id_launch<TA, TB, MODE, 2>(p, n_wg, lds, st);
    if (p.members <= 4) return id_launch<TA, TB, MODE, 4>(p, n_wg, lds, st);
    return id_launch<TA, TB, MODE, 8>(p, n_wg, lds, st);
}

template <int MODE>
hipError_t id_types(const IdArgs& p, int n_wg, size_t lds, hipStream_t st) {
    const uint32_t ta = p.type_a, tb = p.nseg > 2 ? p.type_b : p.type_a;
    if (ta != tb) {
        if constexpr (MODE == MV_STORE)
            if (ta == 12 && tb == 14) return id_members<12, 14, MODE>(p, n_wg, lds, st);
        return hipErrorInvalidValue;
    }
    if (ta == 12) return id_members<12, 12, MODE>(p, n_wg, lds, st);
    if (ta == 14) return id_members<14, 14, MODE>(p, n_wg, lds, st);
    if (ta == 8) return id_members<8, 8, MODE>(p, n_wg, lds, st);
    return hipErrorInvalidValue;
}

}  // namespace

int intdot_layout(IdArgs& a, int n_cu) {
    const bool pair = a.mode == MV_SILU;
    int items = 0;
    for (int i = 0; i < a.nseg; i++) items += pair ? (int)a.seg[i].w.rows : ((int)a.seg[i].w.rows + 1) / 2;
    const int per = kIdWaves * std::max(n_cu, 1);
    const int ipw = std::max(1, (items + per - 1) / per);
    a.items_per_wave = ipw;
    int wg = 0;
    for (int i = 0; i < a.nseg; i++) {
        const int it = pair ? (int)a.seg[i].w.rows : ((int)a.seg[i].w.rows + 1) / 2;
        a.seg[i].ipw = ipw;
        a.seg[i].wg_begin = wg;
        if (!a.seg[i].res) a.seg[i].res = a.seg[i].out;
        wg += (it + kIdWaves * ipw - 1) / (kIdWaves * ipw);
    }
    return wg;
}

hipError_t launch_intdot(const IdArgs& a, int n_wg, hipStream_t st) {
    if (n_wg <= 0 || a.k <= 0 || a.members < 1 || a.members > kIdMaxMembers || a.nseg < 1 || a.nseg > 3)
        return hipErrorInvalidValue;
    for (int i = 0; i < a.nseg; i++) {
        const QMat& w = a.seg[i].w;
        const uint32_t t = i == 2 ? a.type_b : a.type_a;
        if (w.type != t || (int)w.k != a.k) return hipErrorInvalidValue;
        if (a.k % (t == 8 ? 32 : 256)) return hipErrorInvalidValue;
        if (a.mode == MV_SILU && (a.seg[i].w2.rows != w.rows || a.seg[i].w2.type != t)) return hipErrorInvalidValue;
    }
    const size_t lds = intdot_lds(a);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    switch (a.mode) {
    case MV_STORE: return id_types<MV_STORE>(a, n_wg, lds, st);
    case MV_ADD: return id_types<MV_ADD>(a, n_wg, lds, st);
    case MV_SILU: return id_types<MV_SILU>(a, n_wg, lds, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_q8_1_rows(const float* x, int ldx, int rows, int k, const float* norm_w, float eps, uint32_t* out,
                            hipStream_t st) {
    if (rows <= 0 || k <= 0 || k % 32) return hipErrorInvalidValue;
    q8_1_rows_kernel<<<dim3((unsigned)(k / 32 + 7) / 8, (unsigned)rows), 256, 0, st>>>(x, ldx, k, norm_w, eps, out);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_1(const float* x, size_t n, uint32_t* out, hipStream_t st) {
    if (n == 0 || n % 32) return hipErrorInvalidValue;
    const size_t nb = n / 32;
    quantize_q8_1_kernel<<<(unsigned)((nb + 7) / 8), 256, 0, st>>>(x, nb, out);
    return hipGetLastError();
}

}  // namespace ribn
