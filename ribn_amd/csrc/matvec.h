// The standalone matvec kernel and its launch by value types (shared by
// kernels.hip, one input row, and matvec_rows.hip, several).
#pragma once
#include "device.h"

namespace ribn {
namespace {

// Ring depth (load groups in flight per wave) of the standalone matvec, per type.
// Under the one-workgroup-per-CU layout, the Q4_K gate/up launch measured 12.7 us
// at depth 2, 13.3 us at depth 3 and 16.0 us at depth 6; the Q6_K down launch
// 10.7 us at depth 2 against 11.7 us at depth 3 (two early input passes).
#ifndef RIBN_RING_SA_Q4
#define RIBN_RING_SA_Q4 2
#endif
#ifndef RIBN_RING_SA_Q6
#define RIBN_RING_SA_Q6 2
#endif
#ifndef RIBN_RING_SA_Q8
#define RIBN_RING_SA_Q8 3
#endif
template <int T>
constexpr int ring_standalone() {
    return T == 12 ? RIBN_RING_SA_Q4 : T == 14 ? RIBN_RING_SA_Q6 : RIBN_RING_SA_Q8;
}

// Fused dequant-matvec (gguf_gemv qwen_reference.rs:31-40; q*_gemv_warp
// kernels/quantized/q4_k.cu:103, q6_k.cu:45, q8_0.cu:27). Each wave computes
// two rows per item (or a gate/up pair); the first weight loads are issued
// before the input is staged, so HBM streaming overlaps the prologue.
template <int TA, int TB, int MODE, int R = 1>
__global__ __launch_bounds__(kMaxMvThreads) void matvec_kernel(MvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint64_t best = 0ull;
    mv_wg<TA, TB, MODE, ring_standalone<TA>(), ring_standalone<TB>(), R>(a, blockIdx.x, lds, best, NoSync{});
    if constexpr (MODE == MV_HEAD) head_finish(a, best, blockIdx.x, gridDim.x);
}

// matvec_kernel with its first workgroup start and last workgroup end folded
// into clk (timing only; kept apart so the product kernel carries no clock code).
template <int TA, int TB, int MODE>
__global__ __launch_bounds__(kMaxMvThreads) void matvec_clocked_kernel(MvArgs a, unsigned long long* clk) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint64_t best = 0ull;
    if (threadIdx.x == 0) atomicMin(&clk[0], (unsigned long long)wall_clock64());
    mv_wg<TA, TB, MODE, ring_standalone<TA>(), ring_standalone<TB>(), 1>(a, blockIdx.x, lds, best, NoSync{});
    __syncthreads();
    if (threadIdx.x == 0) atomicMax(&clk[1], (unsigned long long)wall_clock64());
}

inline int mv_waves(const MvArgs& a) { return a.waves ? a.waves : kWaves; }

template <int MODE, int R = 1>
hipError_t matvec_dispatch(const MvArgs& a, int n_wg, hipStream_t st) {
    const size_t lds = matvec_lds_bytes(a.k, R);
    const uint32_t ta = a.type_a, tb = a.nseg > 2 ? a.type_b : a.type_a;
#define RIBN_MV(A, B)                                                                              \
    if (ta == A && tb == B) {                                                                      \
        if (lds > 65536) {                                                                         \
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&matvec_kernel<A, B, MODE, R>), \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); \
            if (e != hipSuccess) return e;                                                         \
        }                                                                                          \
        matvec_kernel<A, B, MODE, R><<<n_wg, mv_waves(a) * 64, lds, st>>>(a);                      \
        return hipGetLastError();                                                                  \
    }
    if constexpr (MODE == MV_STORE) {
        RIBN_MV(12, 14) RIBN_MV(14, 12) RIBN_MV(12, 8) RIBN_MV(8, 12) RIBN_MV(14, 8) RIBN_MV(8, 14)
    }
    RIBN_MV(12, 12) RIBN_MV(14, 14) RIBN_MV(8, 8)
#undef RIBN_MV
    return hipErrorInvalidValue;
}


}  // namespace
}  // namespace ribn
