// Persistent decode step: registry of the compiled configurations, occupancy
// query and launcher.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "kernels.h"
#include "step.h"

namespace ribn {

void step_entries_q4km(std::vector<StepEntry>& out);
void step_entries_q8(std::vector<StepEntry>& out);

namespace {
const StepEntry* find_entry(const StepKey& k) {
    static const std::vector<StepEntry> table = [] {
        std::vector<StepEntry> t;
        step_entries_q4km(t);
        step_entries_q8(t);
        return t;
    }();
    for (const StepEntry& e : table)
        if (e.key.qa == k.qa && e.key.qb == k.qb && e.key.o == k.o && e.key.gu == k.gu && e.key.dn == k.dn &&
            e.key.ht == k.ht && e.key.hd == k.hd && e.key.g == k.g && e.key.kv_f16 == k.kv_f16)
            return &e;
    return nullptr;
}
}  // namespace

int step_grid(const StepKey& k, int max_k, int device, size_t* lds) {
    const StepEntry* e = find_entry(k);
    if (!e || max_k % 16) return 0;
    const size_t need = std::max(e->attn_lds, matvec_lds_bytes(max_k));
    *lds = need;
    if (hipFuncSetAttribute(e->fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)need) != hipSuccess) return 0;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, e->fn, 256, need) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
    per_cu = std::min(per_cu, 2);
    return per_cu * cus;
}

hipError_t launch_step(const StepArgs& a, const StepKey& k, int n_wg, size_t lds, hipStream_t st) {
    const StepEntry* e = find_entry(k);
    if (!e || n_wg < 1) return hipErrorInvalidValue;
    StepArgs args = a;
    void* params[] = {&args};
    return hipLaunchKernel(e->fn, dim3(n_wg), dim3(256), params, lds, st);
}

}  // namespace ribn
