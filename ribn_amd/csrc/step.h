// Persistent decode step kernel template (instantiated per model profile in
// step_*.hip; registry and launcher in step.hip).
#pragma once
#include "device.h"

namespace ribn {
namespace {

// ---------------------------------------------------------------------------
// Persistent decode step. One launch of n_wg co-resident workgroups (two per CU)
// runs embedding -> L x [QKV, attention, O, gate/up, down] -> head, with a grid
// barrier in front of every stage that reads what the previous stage wrote.
// Each matvec stage issues its first load groups before it waits at its
// barrier, and each attention work item its first K/V tile, so the HBM stream
// continues through the dependency wait. Stage outputs are written through to
// memory with agent-scope stores into buffers that nothing in this launch has
// read before (a per-layer arena), so readers may use ordinary cached loads.

// Grid barrier, two levels. Workgroup w runs on XCD w % 8 (the dispatcher's
// round-robin placement), and the workgroups of one XCD form a group: each
// counts into its group's counter; the group's last arrival counts into the top
// counter; the last of those bumps every group's generation word, which the
// group's workgroups poll. Each counter and generation word has its own 256-byte
// line, so at most n/8 workgroups contend on one address (one flat counter for
// 512 workgroups measured 7-10 us per barrier, this 3 us). Every wait is
// bounded: past the deadline (or once another workgroup has flagged an error)
// the flag is set and the barrier reports failure, so every workgroup leaves
// the kernel and the grid drains. Layout of `bar` (uint32 words): [0] top
// count, [64] error flag, [64 (2 + g)] group g count, [64 (10 + g)] group g
// generation. Counts return to zero after every barrier.
static_assert(64 * 17 < kStepBarWords, "barrier words outside kStepBarWords");

__device__ __forceinline__ bool grid_sync(uint32_t* bar, uint32_t n, uint64_t deadline) {
    __shared__ int ok;
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        int good = 1;
        uint32_t* const flag = bar + 64;
        const uint32_t grp = blockIdx.x & 7, ng = (n - grp + 7) / 8;
        uint32_t* const gcnt = bar + 64 * (2 + grp);
        uint32_t* const ggen = bar + 64 * (10 + grp);
        const uint32_t groups = n < 8 ? n : 8;
        const uint32_t g = ld_agent(ggen);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (atomicAdd(gcnt, 1u) == ng - 1) {
            __hip_atomic_exchange(gcnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            if (atomicAdd(bar, 1u) == groups - 1) {
                __hip_atomic_exchange(bar, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                for (uint32_t i = 0; i < groups; i++) st_agent(bar + 64 * (10 + i), g + 1);
            }
        }
        for (uint32_t it = 0; ld_agent(ggen) == g; it++) {
            if ((it & 15) == 15) {
                if (ld_agent(flag) != 0u) { good = 0; break; }
                if ((uint64_t)wall_clock64() > deadline) {
                    st_agent(flag, 1u);
                    good = 0;
                    break;
                }
            }
            __builtin_amdgcn_s_sleep(2);
        }
        ok = good;
    }
    __syncthreads();
    return ok != 0;
}

struct GridSync {
    static constexpr bool kEarlyX = false;   // the input is written by the previous stage
    uint32_t* bar;
    uint32_t n;
    uint64_t deadline;
    uint64_t* stamp;      // profiling (workgroup 0, thread 0 only): wall clock at marks
    int* ns;
    __device__ __forceinline__ void mark() const {
        if (stamp && threadIdx.x == 0) stamp[(*ns)++] = wall_clock64();
    }
    __device__ __forceinline__ void phase(int) const {}
    __device__ __forceinline__ bool operator()() const {
        mark();
        const bool ok = grid_sync(bar, n, deadline);
        mark();
        return ok;
    }
};
// The barrier of the first work item only (later items of the same workgroup
// run after it).
struct OnceSync {
    const GridSync& g;
    bool done;
    static constexpr bool kEarlyX = false;
    __device__ __forceinline__ void phase(int) const {}
    __device__ __forceinline__ bool operator()() {
        if (done) return true;
        done = true;
        return g();
    }
};

template <int HD, int G, bool F16>
__device__ __forceinline__ bool attn_items(const AttnArgs& a, int wg, int n_wg, int pos, const int32_t* pages,
                                           uint8_t* lds, const GridSync& sync) {
    const int total = a.n_splits * a.hkv;
    if (wg >= total) return sync();
    OnceSync once{sync, false};
    for (int w = wg; w < total; w += n_wg) {
        const int kvh = w / a.n_splits, split = w % a.n_splits;
        if (!attention_item<HD, G, F16, true>(a, split, kvh, pos, pages, lds, once)) return false;
    }
    return true;
}

// Ring depth (load groups per wave) in the step kernel: its register budget is
// set by the attention stage, so the matvec stages can hold more groups in
// flight than the standalone kernel (a Q6_K group takes 40 VGPRs, a Q4_K 24).
#ifndef RIBN_RING_Q6
#define RIBN_RING_Q6 3
#endif
#ifndef RIBN_RING_Q4
#define RIBN_RING_Q4 4
#endif
template <int T>
constexpr int step_ring() { return T == 14 ? RIBN_RING_Q6 : RIBN_RING_Q4; }

// Value types of one model's matrices: QKV (q/k, v), attn_output, gate/up,
// down, head. The step kernel is compiled per profile, head dimension, query
// heads per KV head and KV element type, so each launch holds one matvec
// instantiation per stage (register pressure and code size stay those of a
// single stage).
template <int QA, int QB, int O, int GU, int DN, int HT>
struct Profile {
    static constexpr int qa = QA, qb = QB, o = O, gu = GU, dn = DN, ht = HT;
};

template <typename PR, int HD, int G, bool F16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void step_kernel(StepArgs s) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int wg = blockIdx.x, n_wg = gridDim.x;
    int ns = 0;
    const GridSync sync{s.bar, (uint32_t)n_wg, (uint64_t)wall_clock64() + s.timeout_ticks,
                        wg == 0 ? s.stamps : nullptr, &ns};
    const SeqState* seq = s.ctl->seq;
    const int pos = seq->pos;
    const int32_t* pages = seq->pages;
    {   // token embedding row and the step's rotary table (embed_kernel)
        const EmbedArgs& e = s.embed;
        const uint32_t tok = seq->tokens[pos];
        for (int i = wg * kThreads + threadIdx.x; i < e.hidden; i += n_wg * kThreads)
            st_agent(e.h + i, deq_elem(e.w, tok, (uint32_t)i));
        if (wg == n_wg - 1 && (int)threadIdx.x < e.half_rot) {
            const float theta = (float)pos * e.inv_freq[threadIdx.x];
            st_agent(e.rope + threadIdx.x, cosf(theta));
            st_agent(e.rope + e.half_rot + threadIdx.x, sinf(theta));
        }
    }
    uint64_t best = 0ull;
    const int n_splits = splits_for_ctx(pos + 1);
    sync.mark();
    for (int l = 0; l < s.n_layers; l++) {
        const LayerDev& L = s.layers[l];
        if (!mv_wg<PR::qa, PR::qb, MV_STORE, step_ring<PR::qa>(), step_ring<PR::qb>()>(L.qkv, wg, lds, best, sync)) return;
        sync.mark();
        AttnArgs at = L.attn;
        at.n_splits = n_splits;
        if (!attn_items<HD, G, F16>(at, wg, n_wg, pos, pages, lds, sync)) return;
        sync.mark();
        if (!mv_wg<PR::o, PR::o, MV_ADD, step_ring<PR::o>(), step_ring<PR::o>()>(L.o, wg, lds, best, sync)) return;
        sync.mark();
        if (!mv_wg<PR::gu, PR::gu, MV_SILU, step_ring<PR::gu>(), step_ring<PR::gu>()>(L.gu, wg, lds, best, sync)) return;
        sync.mark();
        if (!mv_wg<PR::dn, PR::dn, MV_ADD, step_ring<PR::dn>(), step_ring<PR::dn>()>(L.down, wg, lds, best, sync)) return;
        sync.mark();
    }
    if (s.head) {
        if (!mv_wg<PR::ht, PR::ht, MV_HEAD, step_ring<PR::ht>(), step_ring<PR::ht>()>(s.head_mv, wg, lds, best, sync)) return;
        sync.mark();
        head_finish(s.head_mv, best, wg, n_wg);
    } else if (wg == 0 && threadIdx.x == 0) {
        // every workgroup read the position before the first barrier
        s.ctl->seq->pos = pos + 1;
    }
}

}  // namespace

// One compiled configuration of the step kernel.
struct StepEntry {
    StepKey key;
    const void* fn;
    size_t attn_lds;
};

}  // namespace ribn

// Registers step_kernel<Profile<QA..HT>, HD, G, F16> in a StepEntry list.
#define RIBN_STEP_ENTRY(QA, QB, O, GU, DN, HT, HD, G, F16)                                                         \
    ::ribn::StepEntry{::ribn::StepKey{QA, QB, O, GU, DN, HT, HD, G, F16},                                          \
                      reinterpret_cast<const void*>(                                                               \
                          &::ribn::step_kernel<::ribn::Profile<QA, QB, O, GU, DN, HT>, HD, G, (F16) != 0>),        \
                      sizeof(::ribn::AttnLds<HD, G>)}
