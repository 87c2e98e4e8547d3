// Kernels of the qwen35 hybrid decode step (the reference's own architecture):
// the Gated-DeltaNet recurrent block between its input projection (one
// segmented matvec: q|k|v mix, z gate, beta|alpha) and its output projection
// (ssm_out, a residual matvec), and the sigmoid output gate of the gated
// full-attention block.
//
//   gdn_prep_kernel   one workgroup per head-sized channel block (q heads, k
//                     heads, v heads): the depth-KC causal convolution over the
//                     sequence's history and the new mix, SiLU, and for the q/k
//                     blocks the l2 normalization (gdn_conv_step and
//                     l2_normalize, crates/nvidia/src/qwen_reference.rs:44-49,
//                     105-134; kernels model_ops.rs gdn_conv_silu,
//                     l2_norm_heads). The history shifts in place: each thread
//                     owns one channel's history.
//   gdn_state_kernel  one workgroup per V head, one thread per state column:
//                     beta = sigmoid, decay = exp(softplus(alpha + dt) * a), the
//                     delta-rule update S = decay S + k ((v - S^T k) beta)^T and
//                     the read o = S^T q / sqrt(d) (gdn_state_step,
//                     qwen_reference.rs:61-103), then the gated norm
//                     rms(o) * ssm_norm * silu(z) (qwen_reference.rs:254-266).
//                     The column lives in registers: the state is read and
//                     written once per token, coalesced across the columns.
//   gate_mul_kernel   attn *= sigmoid(gate) (qwen_reference.rs:464-474).
//
// The recurrent state of the active sequence is reached through the step
// control block (StepCtl::rec), so the captured step graphs serve every
// sequence. All arithmetic is FP32.
#include "kernels.h"

namespace ribn {
namespace {

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();   // `red` may still be read by a previous reduction
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

__global__ __launch_bounds__(256) void gdn_prep_kernel(GdnArgs a) {
    __shared__ float red[4];
    const int blk = blockIdx.x, d = a.d, t = threadIdx.x;
    const int ch = blk * d + t;
    const int hist_n = a.conv_k - 1;
    float* hist = a.ctl->rec + a.conv_off + (size_t)ch * hist_n;
    const float* w = a.conv_w + (size_t)ch * a.conv_k;   // element (tap, channel) at tap + channel * conv_k
    const float x = a.mixed[ch];
    float s = 0.f;
    for (int tap = 0; tap < hist_n; tap++) s = s + hist[tap] * w[tap];
    s = s + x * w[hist_n];
    for (int tap = 0; tap + 1 < hist_n; tap++) hist[tap] = hist[tap + 1];
    hist[hist_n - 1] = x;
    float y = s * sigmoid(s);
    if (blk < 2 * a.hk) {   // q and k heads: l2 normalization, 1 / max(|x|, eps)
        const float nrm = sqrtf(block_sum(y * y, red));
        y = y * (1.0f / fmaxf(nrm, a.eps));
    }
    a.act[ch] = y;
}

template <int D>
__global__ __launch_bounds__(D) void gdn_state_kernel(GdnArgs a) {
    __shared__ float qs[D], ks[D], red[4];
    const int j = blockIdx.x, c = threadIdx.x, kh = j % a.hk;
    qs[c] = a.act[(size_t)kh * D + c];
    ks[c] = a.act[(size_t)(a.hk + kh) * D + c];
    const float v = a.act[(size_t)(2 * a.hk + j) * D + c];
    const float beta = sigmoid(a.ba[j]);
    const float ar = a.ba[a.hv + j] + a.dt_bias[j];
    const float sp = ar > 20.0f ? ar : logf(1.0f + expf(ar));
    const float decay = expf(sp * a.ssm_a[j]);
    float* S = a.ctl->rec + a.state_off + (size_t)j * D * D;
    float col[D];
#pragma unroll
    for (int r = 0; r < D; r++) col[r] = S[(size_t)r * D + c] * decay;
    __syncthreads();
    float sk = 0.f;
#pragma unroll
    for (int r = 0; r < D; r++) sk = fmaf(col[r], ks[r], sk);
    const float dlt = (v - sk) * beta;
    float o = 0.f;
#pragma unroll
    for (int r = 0; r < D; r++) {
        col[r] = fmaf(ks[r], dlt, col[r]);
        o = fmaf(col[r], qs[r], o);
        S[(size_t)r * D + c] = col[r];
    }
    o *= 1.0f / sqrtf((float)D);
    const float inv = 1.0f / sqrtf(block_sum(o * o, red) / (float)D + a.eps);
    const float z = a.z[(size_t)j * D + c];
    a.gated[(size_t)j * D + c] = o * inv * a.ssm_norm[c] * (z * sigmoid(z));
}

__global__ __launch_bounds__(256) void gate_mul_kernel(float* x, const float* gate, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = x[i] * sigmoid(gate[i]);
}

}  // namespace

hipError_t launch_gdn(const GdnArgs& a, hipStream_t st) {
    if (a.d != 64 && a.d != 128) return hipErrorInvalidValue;
    if (a.hk <= 0 || a.hv % a.hk || a.conv_k < 2) return hipErrorInvalidValue;
    gdn_prep_kernel<<<2 * a.hk + a.hv, a.d, 0, st>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (a.d == 64) gdn_state_kernel<64><<<a.hv, 64, 0, st>>>(a);
    else gdn_state_kernel<128><<<a.hv, 128, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_gate_mul(float* x, const float* gate, int n, hipStream_t st) {
    gate_mul_kernel<<<(n + 255) / 256, 256, 0, st>>>(x, gate, n);
    return hipGetLastError();
}

}  // namespace ribn
