// Step kernels for Q4_K_M models (Q4_K q/k/o/gate/up, Q6_K v/down, Q6_K or tied Q4_K head).
#include <vector>

#include "step.h"

namespace ribn {
void step_entries_q4km(std::vector<StepEntry>& out) {
    out.push_back(RIBN_STEP_ENTRY(12, 14, 12, 12, 14, 14, 128, 4, 1));   // Qwen3-8B shape
    out.push_back(RIBN_STEP_ENTRY(12, 14, 12, 12, 14, 14, 128, 4, 0));
    out.push_back(RIBN_STEP_ENTRY(12, 14, 12, 12, 14, 14, 128, 8, 1));   // Qwen3-32B shape
    out.push_back(RIBN_STEP_ENTRY(12, 14, 12, 12, 14, 14, 64, 2, 1));
    out.push_back(RIBN_STEP_ENTRY(12, 14, 12, 12, 14, 14, 64, 2, 0));
    out.push_back(RIBN_STEP_ENTRY(12, 14, 12, 12, 14, 12, 64, 8, 1));    // tied Q4_K head
}
}  // namespace ribn
