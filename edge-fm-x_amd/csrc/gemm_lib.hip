// Plain prefill projections through hipBLASLt (the vendor's tuned GEMM library), for the
// GEMMs that are nothing but C = A . W^T (+ bias): the reference runs the same calls
// through cuBLASLt with the BIAS epilogue (src/layers/linear.cu:41-58, 1387-1461).
//
// Row-major C[M, N] = A[M, K] . W[N, K]^T is the column-major product
// C^T[N, M] = op_T(W)[N, K] . A^T[K, M] with W seen as a K x N column-major matrix
// (ld K), A as K x M (ld K) and C as N x M (ld N); the bias epilogue adds bias[n] to
// every element of row n of C^T, i.e. to output feature n, in fp32 before the bf16
// rounding, as this library's own MFMA kernels do.
//
// One library handle per device; the algorithm for a shape is hipBLASLt's heuristic
// first choice under the workspace the caller provides (capped at kLibMaxWorkspace),
// cached per (device, M, N, K, bias, workspace cap), so a shape always runs the same
// algorithm for the same workspace and the results are reproducible. A shape the
// library has no algorithm for falls back to this library's MFMA kernels.
#include "common.hpp"

#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <tuple>

namespace efm {

constexpr size_t kLibMaxWorkspace = 64ull << 20;
constexpr size_t kLibMaxPlans = 4096;   // cached (shape, workspace) plans before the cache restarts

static std::atomic<int> g_gemm_backend{EFM_GEMM_BACKEND_AUTO};

int gemm_backend() { return g_gemm_backend.load(std::memory_order_relaxed); }

namespace {

struct LibPlan {
    bool ok = false;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
};

typedef std::tuple<int, int64_t, int64_t, int64_t, bool, size_t> PlanKey;

struct LibState {
    std::mutex mu;
    std::map<int, hipblasLtHandle_t> handles;
    std::map<PlanKey, LibPlan> plans;
};

LibState& lib_state() {
    static LibState* s = new LibState();   // never destroyed: handles outlive static teardown
    return *s;
}

// Descriptors of one call (host objects, created per call: the bias pointer is part of
// the matmul descriptor).
struct LibDescs {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t w = nullptr, a = nullptr, c = nullptr;
    bool ok = false;
    LibDescs(int64_t M, int64_t N, int64_t K, const void* bias) {
        if (hipblasLtMatmulDescCreate(&op, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return;
        const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
        if (hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) != HIPBLAS_STATUS_SUCCESS ||
            hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) != HIPBLAS_STATUS_SUCCESS)
            return;
        if (bias != nullptr) {
            const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
            const hipDataType bt = HIP_R_16BF;
            if (hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep)) !=
                    HIPBLAS_STATUS_SUCCESS ||
                hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) !=
                    HIPBLAS_STATUS_SUCCESS ||
                hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)) !=
                    HIPBLAS_STATUS_SUCCESS)
                return;
        }
        if (hipblasLtMatrixLayoutCreate(&w, HIP_R_16BF, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
            hipblasLtMatrixLayoutCreate(&a, HIP_R_16BF, K, M, K) != HIPBLAS_STATUS_SUCCESS ||
            hipblasLtMatrixLayoutCreate(&c, HIP_R_16BF, N, M, N) != HIPBLAS_STATUS_SUCCESS)
            return;
        ok = true;
    }
    ~LibDescs() {
        if (c) hipblasLtMatrixLayoutDestroy(c);
        if (a) hipblasLtMatrixLayoutDestroy(a);
        if (w) hipblasLtMatrixLayoutDestroy(w);
        if (op) hipblasLtMatmulDescDestroy(op);
    }
};

// Handle of the current device and the plan of a shape (both created on first use).
bool lib_plan(int64_t M, int64_t N, int64_t K, bool has_bias, size_t ws_cap, hipblasLtHandle_t* h, LibPlan* plan) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    LibState& s = lib_state();
    std::lock_guard<std::mutex> lock(s.mu);
    auto hit = s.handles.find(dev);
    if (hit == s.handles.end()) {
        hipblasLtHandle_t nh = nullptr;
        if (hipblasLtCreate(&nh) != HIPBLAS_STATUS_SUCCESS) return false;
        hit = s.handles.emplace(dev, nh).first;
    }
    *h = hit->second;
    const PlanKey key(dev, M, N, K, has_bias, ws_cap);
    auto pit = s.plans.find(key);
    if (pit == s.plans.end()) {
        LibPlan p;
        // any non-null bias pointer selects the same epilogue and algorithm
        static const uint16_t kDummyBias = 0;
        LibDescs d(M, N, K, has_bias ? &kDummyBias : nullptr);
        hipblasLtMatmulPreference_t pref = nullptr;
        if (d.ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS) {
            const uint64_t cap = ws_cap;
            hipblasLtMatmulHeuristicResult_t res{};
            int n = 0;
            if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &cap,
                                                      sizeof(cap)) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatmulAlgoGetHeuristic(*h, d.op, d.w, d.a, d.c, d.c, pref, 1, &res, &n) ==
                    HIPBLAS_STATUS_SUCCESS &&
                n > 0 && res.state == HIPBLAS_STATUS_SUCCESS && res.workspaceSize <= ws_cap) {
                p.ok = true;
                p.algo = res.algo;
                p.ws = res.workspaceSize;
            }
            hipblasLtMatmulPreferenceDestroy(pref);
        }
        if (s.plans.size() >= kLibMaxPlans) s.plans.clear();   // bounded: one entry per distinct M
        pit = s.plans.emplace(key, p).first;
    }
    *plan = pit->second;
    return plan->ok;
}

}  // namespace

bool gemm_lib_applies(int32_t out_dtype) {
    return gemm_backend() == EFM_GEMM_BACKEND_AUTO && out_dtype == EFM_DTYPE_BF16;
}

size_t gemm_lib_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    hipblasLtHandle_t h;
    LibPlan p;
    return lib_plan(M, N, K, false, kLibMaxWorkspace, &h, &p) ? p.ws : 0;
}

// C[M, N] (bf16, row-major) = A . W^T (+ bias). Returns EFM_OK, or EFM_ERR_UNSUPPORTED when
// the library has no algorithm for the shape (the caller then runs its own kernels).
int gemm_lib(int64_t M, int64_t N, int64_t K, const void* A, const void* W, const void* bias, void* C,
             void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (((reinterpret_cast<uintptr_t>(C) | reinterpret_cast<uintptr_t>(bias) |
          reinterpret_cast<uintptr_t>(workspace)) & 15u) != 0)
        return EFM_ERR_UNSUPPORTED;
    // Under stream capture the library is not used (its first call per shape creates
    // handles and plans, and an algorithm may record memory fills into the graph): the
    // MFMA kernels run instead.
    hipStreamCaptureStatus cap_status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap_status) != hipSuccess || cap_status != hipStreamCaptureStatusNone)
        return EFM_ERR_UNSUPPORTED;
    const size_t cap = (workspace == nullptr) ? 0 : std::min(workspace_bytes, kLibMaxWorkspace);
    hipblasLtHandle_t h;
    LibPlan p;
    if (!lib_plan(M, N, K, bias != nullptr, cap, &h, &p)) return EFM_ERR_UNSUPPORTED;
    LibDescs d(M, N, K, bias);
    if (!d.ok) return set_error(EFM_ERR_DEVICE, "gemm (hipBLASLt): descriptor setup failed");
    const float alpha = 1.f, beta = 0.f;
    const hipblasStatus_t st = hipblasLtMatmul(h, d.op, &alpha, W, d.w, A, d.a, &beta, C, d.c, C, d.c, &p.algo,
                                               p.ws > 0 ? workspace : nullptr, p.ws, stream);
    if (st != HIPBLAS_STATUS_SUCCESS)
        return set_error(EFM_ERR_DEVICE, "gemm (hipBLASLt): matmul failed (status %d) for %lld x %lld x %lld", (int)st,
                         (long long)M, (long long)N, (long long)K);
    return check_launch("gemm (hipBLASLt)");
}

}  // namespace efm

extern "C" int efm_set_gemm_backend(int32_t backend) {
    if (backend != EFM_GEMM_BACKEND_AUTO && backend != EFM_GEMM_BACKEND_OWN)
        return efm::set_error(EFM_ERR_INVALID_ARGUMENT, "set_gemm_backend: unknown backend %d", backend);
    efm::g_gemm_backend.store(backend, std::memory_order_relaxed);
    return EFM_OK;
}

extern "C" int32_t efm_get_gemm_backend(void) { return efm::gemm_backend(); }
