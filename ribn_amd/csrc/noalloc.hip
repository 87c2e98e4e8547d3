// Allocation-free greedy argmax over device-resident logits, for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc). Same kernel and result as
// ribn_rocm_argmax; the cross-workgroup partials and the arrival counter live
// in a file-scope device array instead of per-call allocations.
#include <mutex>
#include <string>

#include "../../include/ribn_rocm.h"
#include "common.h"
#include "kernels.h"

namespace ribn {
namespace {

// Scratch: kArgmaxBlocks per-workgroup (key, index) maxima, then the arrival
// counter. Every GPU the library runs on holds its own copy until the process
// ends. Calls that overlap on one GPU share it and race.
constexpr int kArgmaxBlocks = 1024;   // launch_argmax's workgroup cap
constexpr size_t kScratchWords = kArgmaxBlocks + 32;
__device__ __align__(256) uint64_t scratch[kScratchWords];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint64_t* g_scratch[kMaxDevices] = {};   // device address of `scratch`, per device

__global__ void clear_words(uint32_t* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Device address of this device's scratch array (looked up once per device,
// with that device current).
hipError_t scratch_for(int dev, uint64_t** out) {
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch[dev] = static_cast<uint64_t*>(ptr);
    }
    *out = g_scratch[dev];
    return hipSuccess;
}

int error(char* err, size_t err_len, const std::string& msg, int code) {
    set_err(err, err_len, msg);
    return code;
}

std::string hip_text(const char* what, hipError_t e) {
    return std::string(what) + ": " + hipGetErrorString(e);
}

}  // namespace
}  // namespace ribn

using namespace ribn;

extern "C" int ribn_rocm_argmax_noalloc(const float* d_logits, uint64_t n, uint32_t* d_out, void* stream, char* err,
                                        size_t err_len) {
    if (!d_logits || !d_out) return error(err, err_len, "null argument", RIBN_ERR_INVALID);
    if (n == 0 || n > RIBN_ARGMAX_NOALLOC_MAX)
        return error(err, err_len,
                     "argmax length " + std::to_string(n) + " outside 1.." + std::to_string(RIBN_ARGMAX_NOALLOC_MAX),
                     RIBN_ERR_INVALID);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    uint64_t* s = nullptr;
    if (e == hipSuccess) e = scratch_for(dev, &s);
    if (e != hipSuccess) return error(err, err_len, hip_text("argmax_noalloc scratch", e), RIBN_ERR_DEVICE);
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* counter = reinterpret_cast<uint32_t*>(s + kArgmaxBlocks);
    // the counter starts at zero (a fill kernel, not a memset node: graph-capture safe)
    clear_words<<<1, 64, 0, st>>>(counter, 2);
    e = hipGetLastError();
    if (e == hipSuccess) e = launch_argmax(d_logits, (uint32_t)n, s, counter, d_out, st);
    if (e != hipSuccess) return error(err, err_len, hip_text("argmax_noalloc", e), RIBN_ERR_DEVICE);
    return RIBN_OK;
}
