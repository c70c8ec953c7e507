// C-ABI glue: error reporting and the entry points that dispatch between the decode
// GEMV (m == 1) and the prefill MFMA GEMM (m > 1).
#include "common.hpp"

#include <atomic>
#include <cstdarg>
#include <cstdio>

namespace efm {

static std::atomic<int> g_knobs[EFM_KNOB_COUNT];

int kernel_knob(int knob) {
    return (knob >= 0 && knob < EFM_KNOB_COUNT) ? g_knobs[knob].load(std::memory_order_relaxed) : 0;
}

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(EFM_ERR_DEVICE, "%s: launch failed: %s", what, hipGetErrorString(e));
    return EFM_OK;
}

int gemv_plain(int64_t K, int64_t N, const void* x, const void* W, const void* bias, void* y, int32_t out_dtype,
               hipStream_t stream);
int gemv_swiglu(int64_t K, int64_t inter, const void* x, const void* W, void* y, hipStream_t stream);
int gemm_bf16(int64_t M, int64_t N, int64_t K, const void* A, const void* B, const void* bias, void* C,
              int32_t out_dtype, hipStream_t stream);
int gemm_swiglu(int64_t M, int64_t inter, int64_t K, const void* A, const void* W, void* out, hipStream_t stream);
size_t gemm_swiglu_workspace_bytes(int64_t M, int64_t inter, int64_t K);
int gemm_swiglu_ws(int64_t M, int64_t inter, int64_t K, const void* A, const void* W, void* out, void* workspace,
                   size_t workspace_bytes, hipStream_t stream);
size_t gemm_bf16_workspace_bytes(int64_t M, int64_t N, int64_t K);
int gemm_bf16_ws(int64_t M, int64_t N, int64_t K, const void* A, const void* B, const void* bias, void* C,
                 int32_t out_dtype, void* workspace, size_t workspace_bytes, hipStream_t stream);

}  // namespace efm

using namespace efm;

extern "C" const char* efm_last_error(void) { return g_last_error; }

extern "C" const char* efm_version(void) { return "edgefm-hip 0.2.0 gfx950"; }

extern "C" int efm_testing_set_kernel_path(int32_t knob, int32_t value) {
    if (knob < 0 || knob >= EFM_KNOB_COUNT)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "testing_set_kernel_path: unknown knob %d", knob);
    const bool ok = (knob == EFM_KNOB_PREFILL_SHAPE) ? (value == 0 || value == 2 || value == 4 || value == 8)
                    : (knob == EFM_KNOB_GEMM_TILE)   ? (value >= 0 && value <= 3)
                                                     : (value == 0 || value == 1);
    if (!ok) return set_error(EFM_ERR_INVALID_ARGUMENT, "testing_set_kernel_path: bad value %d for knob %d", value, knob);
    g_knobs[knob].store(value, std::memory_order_relaxed);
    return EFM_OK;
}

extern "C" int efm_linear(int64_t m, int64_t in_features, int64_t out_features, const void* x, const void* w,
                          const void* bias, void* y, int32_t out_dtype, hipStream_t stream) {
    if (m < 0 || in_features <= 0 || out_features <= 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "linear: bad shape m=%lld in=%lld out=%lld", (long long)m,
                         (long long)in_features, (long long)out_features);
    if (m == 0) return EFM_OK;
    if (m == 1) return gemv_plain(in_features, out_features, x, w, bias, y, out_dtype, stream);
    return gemm_bf16(m, out_features, in_features, x, w, bias, y, out_dtype, stream);
}

extern "C" size_t efm_linear_workspace_bytes(int64_t m, int64_t in_features, int64_t out_features) {
    if (m <= 1 || in_features <= 0 || out_features <= 0) return 0;
    return gemm_bf16_workspace_bytes(m, out_features, in_features);
}

extern "C" int efm_linear_ws(int64_t m, int64_t in_features, int64_t out_features, const void* x, const void* w,
                             const void* bias, void* y, int32_t out_dtype, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
    if (m < 0 || in_features <= 0 || out_features <= 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "linear: bad shape m=%lld in=%lld out=%lld", (long long)m,
                         (long long)in_features, (long long)out_features);
    if (m == 0) return EFM_OK;
    if (m == 1) return gemv_plain(in_features, out_features, x, w, bias, y, out_dtype, stream);
    return gemm_bf16_ws(m, out_features, in_features, x, w, bias, y, out_dtype, workspace, workspace_bytes, stream);
}

extern "C" int efm_fused_gate_up_swiglu(int64_t m, int64_t hidden, int64_t inter, const void* x,
                                        const void* w_up_gate, void* out, hipStream_t stream) {
    if (m < 0 || hidden <= 0 || inter <= 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "fused_gate_up_swiglu: bad shape");
    if (m == 0) return EFM_OK;
    if (m == 1) return gemv_swiglu(hidden, inter, x, w_up_gate, out, stream);
    return gemm_swiglu(m, inter, hidden, x, w_up_gate, out, stream);
}

extern "C" size_t efm_fused_gate_up_swiglu_workspace_bytes(int64_t m, int64_t hidden, int64_t inter) {
    if (m <= 1 || hidden <= 0 || inter <= 0) return 0;
    return gemm_swiglu_workspace_bytes(m, inter, hidden);
}

extern "C" int efm_fused_gate_up_swiglu_ws(int64_t m, int64_t hidden, int64_t inter, const void* x,
                                           const void* w_up_gate, void* out, void* workspace, size_t workspace_bytes,
                                           hipStream_t stream) {
    if (m < 0 || hidden <= 0 || inter <= 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "fused_gate_up_swiglu: bad shape");
    if (m == 0) return EFM_OK;
    if (m == 1) return gemv_swiglu(hidden, inter, x, w_up_gate, out, stream);
    return gemm_swiglu_ws(m, inter, hidden, x, w_up_gate, out, workspace, workspace_bytes, stream);
}
