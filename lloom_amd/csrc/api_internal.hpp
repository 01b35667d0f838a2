// api_internal.hpp -- the context and the qmatmul plan shared by the C-ABI
// sources (api.hip and the entry points built on it).
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "../../include/lloom_hip.h"
#include "kernels.hpp"

struct lloom_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    void* ws = nullptr;  // grow-only workspace
    size_t ws_bytes = 0;
    // Workspaces outgrown by a larger call.  They are not freed before the
    // context is destroyed: launches still queued, and graphs captured
    // earlier, keep reading them, so growth needs no device synchronization.
    // Growth at least doubles, so they hold less than the current one.
    std::vector<void*> retired;
    int* flags = nullptr;  // [0] sticky expert-id error
    int mv_rows_max = 16;
    int prefill_mma = lloom::GEMM_AUTO;
    std::mutex mu;
};

// Records the message of a failure for lloom_hip_last_error; returns code.
int fail(int code, const char* fmt, ...);

#define HIP_OK(expr)                                                                         \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess) return fail(LLOOM_HIP_EHIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

struct QmmPlan {
    bool decode;
    size_t path_bytes;  // the kernels' own workspace
    size_t x32_off, y32_off, total;
};

QmmPlan qmm_plan(int mv_rows_max, int prefill_mma, int ggml_type, int64_t n, int64_t k, int64_t m, int x_dtype,
                 int y_dtype);
// Argument checks of a qmatmul call (0 or the refusal's code).
int qmatmul_check(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k, const void* x_dev,
                  int x_dtype, int64_t m, void* y_dev, int y_dtype, int epi);
// The call's launches on workspace `ws` of `ws_cap` bytes (>= the plan's total).
int qmatmul_run(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k, const void* x_dev,
                int x_dtype, int64_t m, void* y_dev, int y_dtype, int epi, hipStream_t s, const QmmPlan& p, void* ws,
                size_t ws_cap);
