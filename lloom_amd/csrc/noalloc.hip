// noalloc.hip -- lloom_hip_qmatmul_noalloc: the quantized matmul for callers
// that cannot allocate device memory (code under graph capture, tight
// serving loops).  Its workspace is a fixed device array, `scratch`, one
// copy per GPU, held until the process ends.
//
// On the host, `scratch` names a stand-in for the device symbol, not a
// device address: host code never passes it to a kernel or a copy.  The
// address of each GPU's copy comes from hipGetSymbolAddress, called with
// that device current on every call (it allocates nothing and is cheap, and
// a module reloaded after hipDeviceReset may place the array elsewhere); the
// last address is kept per device for the record.
//
// Nothing in the workspace must start at zero: every kernel of the qmatmul
// routes writes what it later reads.  Calls on one GPU share the array, so
// calls that overlap on one GPU (other streams, other contexts) race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "api_internal.hpp"
#include "kq_common.hpp"

using namespace lloom;

namespace {

constexpr size_t SCRATCH_BYTES = (size_t)32 << 20;
__device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
void* g_scratch_ptr[MAX_DEVICES];
std::mutex g_scratch_mu;

// The device address of `device`'s copy of the scratch array; the device is
// current.  0 or the refusal's code.
int scratch_of(int device, void** out) {
    if (device < 0 || device >= MAX_DEVICES)
        return fail(LLOOM_HIP_EDEVICE, "qmatmul_noalloc: device %d is past the scratch table", device);
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(LLOOM_HIP_EHIP, "qmatmul_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", device,
                    hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    g_scratch_ptr[device] = ptr;
    *out = ptr;
    return LLOOM_HIP_OK;
}

}  // namespace

extern "C" int lloom_hip_qmatmul_noalloc(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k,
                                         const void* x_dev, int x_dtype, int64_t m, void* y_dev, int y_dtype,
                                         void* stream) {
    if (int rc = qmatmul_check(ctx, ggml_type, w_dev, n, k, x_dev, x_dtype, m, y_dev, y_dtype, EPI_STORE)) return rc;
    HIP_OK(hipSetDevice(ctx->device));
    void* ws = nullptr;
    if (int rc = scratch_of(ctx->device, &ws)) return rc;
    std::lock_guard<std::mutex> lock(ctx->mu);
    const QmmPlan p = qmm_plan(ctx->mv_rows_max, ctx->prefill_mma, ggml_type, n, k, m, x_dtype, y_dtype);
    if (p.total > SCRATCH_BYTES)
        return fail(LLOOM_HIP_ENOMEM,
                    "qmatmul_noalloc: the call needs %zu bytes of workspace and the static scratch holds %zu "
                    "(use lloom_hip_qmatmul, or fewer rows a call)",
                    p.total, SCRATCH_BYTES);
    return qmatmul_run(ctx, ggml_type, w_dev, n, k, x_dev, x_dtype, m, y_dev, y_dtype, EPI_STORE, (hipStream_t)stream,
                       p, ws, SCRATCH_BYTES);
}
