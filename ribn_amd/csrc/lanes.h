// Cross-lane helpers for wave64 on gfx950, shared by the decode and prefill kernels.
#pragma once
#include <hip/hip_runtime.h>

namespace ribn {

// Cross-lane reductions without LDS traffic: DPP within rows of 16 lanes
// (quad permutes, then half-row and row mirrors, each of which pairs lanes that
// already hold equal partial results) and the gfx950 permlane swaps across rows.
// They need every lane of the wave active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
// v + (v of lane ^ 16), v + (v of lane ^ 32): the swap returns the pair {own, partner}
__device__ __forceinline__ float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// sum / maximum over aligned groups of W lanes (W = 4, 8, 16, 32 or 64), result in every lane
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (W >= 8) v += dpp_f<0x141>(v);   // row_half_mirror
    if constexpr (W >= 16) v += dpp_f<0x140>(v);  // row_mirror
    if constexpr (W >= 32) v = xor16_sum(v);
    if constexpr (W >= 64) v = xor32_sum(v);
    return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    if constexpr (W >= 8) v = fmaxf(v, dpp_f<0x141>(v));
    if constexpr (W >= 16) v = fmaxf(v, dpp_f<0x140>(v));
    if constexpr (W >= 32) v = xor16_max(v);
    if constexpr (W >= 64) v = xor32_max(v);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }

}  // namespace ribn
