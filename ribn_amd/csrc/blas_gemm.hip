// Plain binary16 GEMM on hipBLASLt, for the resident-weight mode: the layer's
// matrices are dequantized once at load (exactly, then rounded to binary16 —
// the same operand values the dequant GEMM builds in registers) and chunked
// prefill / batched decode run library GEMMs on them (gemv_batch,
// nvidia/src/decode.rs:1591-1633, as dense contractions).
//
// Row-major y[m][ldy] = x[m][k] w[n][k]^T is, in hipBLASLt's column-major
// terms, D (n x m, ld ldy) = op(A) B with A = w (k x n, ld k) transposed and
// B = x (k x m, ld k). beta = 1 with C = D adds the residual in place; the
// bias epilogue adds a per-row (n) vector. One algorithm per shape is chosen by
// the library heuristic and cached.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <dlfcn.h>

#include <map>
#include <tuple>

#include "kernels.h"

namespace ribn {

struct BlasGemm {
    hipblasLtHandle_t handle = nullptr;
    void* workspace = nullptr;
    size_t ws_bytes = 0;
    struct Plan {
        hipblasLtMatmulDesc_t desc = nullptr;
        hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
        hipblasLtMatmulAlgo_t algo{};
    };
    // key: m, n, k, ldy, add, bias
    std::map<std::tuple<int, int, int, int, bool, bool>, Plan> plans;
};

namespace {

// hipBLASLt is opened on first use (dlopen), so the library does not depend on
// it unless the resident-weight mode runs.
struct LtApi {
    decltype(&::hipblasLtCreate) Create = nullptr;
    decltype(&::hipblasLtDestroy) Destroy = nullptr;
    decltype(&::hipblasLtMatmul) Matmul = nullptr;
    decltype(&::hipblasLtMatmulAlgoGetHeuristic) MatmulAlgoGetHeuristic = nullptr;
    decltype(&::hipblasLtMatmulDescCreate) MatmulDescCreate = nullptr;
    decltype(&::hipblasLtMatmulDescDestroy) MatmulDescDestroy = nullptr;
    decltype(&::hipblasLtMatmulDescSetAttribute) MatmulDescSetAttribute = nullptr;
    decltype(&::hipblasLtMatmulPreferenceCreate) MatmulPreferenceCreate = nullptr;
    decltype(&::hipblasLtMatmulPreferenceDestroy) MatmulPreferenceDestroy = nullptr;
    decltype(&::hipblasLtMatmulPreferenceSetAttribute) MatmulPreferenceSetAttribute = nullptr;
    decltype(&::hipblasLtMatrixLayoutCreate) MatrixLayoutCreate = nullptr;
    decltype(&::hipblasLtMatrixLayoutDestroy) MatrixLayoutDestroy = nullptr;
};

const LtApi* lt_api() {
    static const LtApi* api = [] {
        void* h = dlopen("libhipblaslt.so", RTLD_NOW | RTLD_LOCAL);
        if (!h) h = dlopen("/opt/rocm/lib/libhipblaslt.so", RTLD_NOW | RTLD_LOCAL);
        if (!h) return static_cast<const LtApi*>(nullptr);
        static LtApi a;
        bool ok = true;
        ok = ok && (a.Create = reinterpret_cast<decltype(&::hipblasLtCreate)>(dlsym(h, "hipblasLtCreate")));
        ok = ok && (a.Destroy = reinterpret_cast<decltype(&::hipblasLtDestroy)>(dlsym(h, "hipblasLtDestroy")));
        ok = ok && (a.Matmul = reinterpret_cast<decltype(&::hipblasLtMatmul)>(dlsym(h, "hipblasLtMatmul")));
        ok = ok && (a.MatmulAlgoGetHeuristic = reinterpret_cast<decltype(&::hipblasLtMatmulAlgoGetHeuristic)>(dlsym(h, "hipblasLtMatmulAlgoGetHeuristic")));
        ok = ok && (a.MatmulDescCreate = reinterpret_cast<decltype(&::hipblasLtMatmulDescCreate)>(dlsym(h, "hipblasLtMatmulDescCreate")));
        ok = ok && (a.MatmulDescDestroy = reinterpret_cast<decltype(&::hipblasLtMatmulDescDestroy)>(dlsym(h, "hipblasLtMatmulDescDestroy")));
        ok = ok && (a.MatmulDescSetAttribute = reinterpret_cast<decltype(&::hipblasLtMatmulDescSetAttribute)>(dlsym(h, "hipblasLtMatmulDescSetAttribute")));
        ok = ok && (a.MatmulPreferenceCreate = reinterpret_cast<decltype(&::hipblasLtMatmulPreferenceCreate)>(dlsym(h, "hipblasLtMatmulPreferenceCreate")));
        ok = ok && (a.MatmulPreferenceDestroy = reinterpret_cast<decltype(&::hipblasLtMatmulPreferenceDestroy)>(dlsym(h, "hipblasLtMatmulPreferenceDestroy")));
        ok = ok && (a.MatmulPreferenceSetAttribute = reinterpret_cast<decltype(&::hipblasLtMatmulPreferenceSetAttribute)>(dlsym(h, "hipblasLtMatmulPreferenceSetAttribute")));
        ok = ok && (a.MatrixLayoutCreate = reinterpret_cast<decltype(&::hipblasLtMatrixLayoutCreate)>(dlsym(h, "hipblasLtMatrixLayoutCreate")));
        ok = ok && (a.MatrixLayoutDestroy = reinterpret_cast<decltype(&::hipblasLtMatrixLayoutDestroy)>(dlsym(h, "hipblasLtMatrixLayoutDestroy")));
        return ok ? static_cast<const LtApi*>(&a) : nullptr;
    }();
    return api;
}

constexpr size_t kWorkspaceBytes = 64ull << 20;

hipError_t to_hip(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorUnknown; }

void destroy_plan(BlasGemm::Plan& p) {
    if (p.a) lt_api()->MatrixLayoutDestroy(p.a);
    if (p.b) lt_api()->MatrixLayoutDestroy(p.b);
    if (p.c) lt_api()->MatrixLayoutDestroy(p.c);
    if (p.desc) lt_api()->MatmulDescDestroy(p.desc);
    p = BlasGemm::Plan{};
}

hipError_t make_plan(BlasGemm* g, int m, int n, int k, int ldy, bool add, bool bias, BlasGemm::Plan* out) {
    BlasGemm::Plan p;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    hipblasStatus_t s = lt_api()->MatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = lt_api()->MatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = lt_api()->MatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
    if (s == HIPBLAS_STATUS_SUCCESS && bias) {
        const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
        const hipDataType bt = HIP_R_32F;
        s = lt_api()->MatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep));
        if (s == HIPBLAS_STATUS_SUCCESS)
            s = lt_api()->MatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt));
    }
    if (s == HIPBLAS_STATUS_SUCCESS) s = lt_api()->MatrixLayoutCreate(&p.a, HIP_R_16F, k, n, k);
    if (s == HIPBLAS_STATUS_SUCCESS) s = lt_api()->MatrixLayoutCreate(&p.b, HIP_R_16F, k, m, k);
    if (s == HIPBLAS_STATUS_SUCCESS) s = lt_api()->MatrixLayoutCreate(&p.c, HIP_R_32F, n, m, ldy);
    hipblasLtMatmulPreference_t pref = nullptr;
    if (s == HIPBLAS_STATUS_SUCCESS) s = lt_api()->MatmulPreferenceCreate(&pref);
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = lt_api()->MatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &g->ws_bytes,
                                                  sizeof(g->ws_bytes));
    hipblasLtMatmulHeuristicResult_t res[1];
    int found = 0;
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = lt_api()->MatmulAlgoGetHeuristic(g->handle, p.desc, p.a, p.b, p.c, p.c, pref, 1, res, &found);
    if (pref) lt_api()->MatmulPreferenceDestroy(pref);
    if (s != HIPBLAS_STATUS_SUCCESS || found < 1) {
        destroy_plan(p);
        return hipErrorNotSupported;
    }
    p.algo = res[0].algo;
    (void)add;
    *out = p;
    return hipSuccess;
}

}  // namespace

hipError_t blas_create(BlasGemm** out, hipStream_t stream) {
    (void)stream;
    if (!lt_api()) return hipErrorSharedObjectInitFailed;   // libhipblaslt.so not loadable
    BlasGemm* g = new BlasGemm();
    hipError_t e = to_hip(lt_api()->Create(&g->handle));
    if (e == hipSuccess) e = hipMalloc(&g->workspace, kWorkspaceBytes);
    if (e != hipSuccess) {
        blas_destroy(g);
        return e;
    }
    g->ws_bytes = kWorkspaceBytes;
    *out = g;
    return hipSuccess;
}

void blas_destroy(BlasGemm* g) {
    if (!g) return;
    for (auto& kv : g->plans) destroy_plan(kv.second);
    if (g->workspace) (void)hipFree(g->workspace);
    if (g->handle) lt_api()->Destroy(g->handle);
    delete g;
}

hipError_t blas_gemm(BlasGemm* g, const uint16_t* x, int m, int k, const uint16_t* w16, int n, float* y, int ldy,
                     bool add, const float* bias, hipStream_t stream) {
    if (!g || m <= 0 || n <= 0 || k <= 0 || ldy < n) return hipErrorInvalidValue;
    const auto key = std::make_tuple(m, n, k, ldy, add, bias != nullptr);
    auto it = g->plans.find(key);
    if (it == g->plans.end()) {
        BlasGemm::Plan p;
        const hipError_t e = make_plan(g, m, n, k, ldy, add, bias != nullptr, &p);
        if (e != hipSuccess) return e;
        it = g->plans.emplace(key, p).first;
    }
    BlasGemm::Plan& p = it->second;
    if (bias) {
        const hipblasStatus_t s =
            lt_api()->MatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
        if (s != HIPBLAS_STATUS_SUCCESS) return hipErrorUnknown;
    }
    const float alpha = 1.0f, beta = add ? 1.0f : 0.0f;
    return to_hip(lt_api()->Matmul(g->handle, p.desc, &alpha, w16, p.a, x, p.b, &beta, y, p.c, y, p.c, &p.algo,
                                  g->workspace, g->ws_bytes, stream));
}

}  // namespace ribn
