// gemm.hip -- prefill-shaped quantized matmul (m > 16 activation rows).
// Interim: tiles of 16 activation rows through the fused matvec kernel.
#include "kq_common.hpp"
#include "kernels.hpp"

namespace lloom {

size_t gemm_workspace_bytes(int type, int64_t k, int64_t m) {
    (void)m;
    return matvec_workspace_bytes(type, k, 16);
}

hipError_t launch_gemm(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                       void* qbuf, hipStream_t s) {
    (void)qbuf;
    for (int64_t r = 0; r < m; r += 16) {
        int64_t mm = m - r < 16 ? m - r : 16;
        hipError_t e = launch_matvec(type, w, x + r * k, y + r * n, n, k, mm, qbuf, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace lloom
