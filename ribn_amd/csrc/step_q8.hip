// Step kernels for all-Q8_0 models (Qwen2.5-0.5B shape: 14 q / 2 KV heads x 64).
#include <vector>

#include "step.h"

namespace ribn {
void step_entries_q8(std::vector<StepEntry>& out) {
    out.push_back(RIBN_STEP_ENTRY(8, 8, 8, 8, 8, 8, 64, 7, 1));
    out.push_back(RIBN_STEP_ENTRY(8, 8, 8, 8, 8, 8, 64, 7, 0));
}
}  // namespace ribn
