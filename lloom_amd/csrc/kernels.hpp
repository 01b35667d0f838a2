// kernels.hpp -- launchers of the gfx950 kernels (host side of each .hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lloom {

// quant.hip
hipError_t launch_quantize_act(int vec_dot_type, const float* x, void* out, int64_t elems, hipStream_t s);
hipError_t launch_quantize_weights(int type, const float* x, void* out, int64_t elems, hipStream_t s);
hipError_t launch_dequantize(int type, const void* w, void* y, int out_dtype, int64_t elems, hipStream_t s);
// F32 <-> F16 conversion of count elements (f32 -> f16 round-to-nearest-even);
// src and dst 16-byte aligned.
hipError_t launch_cast(int src_t, const void* src, int dst_t, void* dst, int64_t count, hipStream_t s);
// Rows ids[0 .. n_ids) of an [rows, hidden] weight, dequantized; a bad id
// gives a zero row and sets flag[0] and flag[1].
hipError_t launch_embedding(int type, const void* w, int64_t rows, int64_t hidden, const uint32_t* ids, int64_t n_ids,
                            void* y, int out_dtype, int* flag, hipStream_t s);

// quant.hip: Q8_K activations in the split layout the MFMA kernels read:
// qs int8 [m][k] then d f32 [k/256][mp] (m padded to mp, a multiple of 16),
// 256-byte aligned, then (when asked for) the sub-block sums as an MFMA
// operand, int8 [k/256][mp][16].
size_t split_q8k_bytes(int64_t k, int64_t m);
void split_q8k_ptrs(void* base, int64_t k, int64_t m, int8_t** qs, float** d, int8_t** bsp = nullptr);
hipError_t launch_quantize_split_q8k(const float* x, int64_t m, int64_t k, int8_t* qs, float* d, hipStream_t s,
                                     int8_t* bsp = nullptr, bool tiled = false);

// matvec.hip: m <= 16.  Rows up to MV_DOT_MAX_ROWS (Q4_K on a weight of at
// most 2048^2 elements: up to 4) take the fused dot4 kernel; more rows take
// the MFMA kernels on a workspace of matvec_workspace_bytes.
constexpr int MV_DOT_MAX_ROWS = 2;
size_t matvec_workspace_bytes(int type, int64_t n, int64_t k, int64_t m);
hipError_t launch_matvec(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                         void* ws, int epi, hipStream_t s);
// matvec.hip: Q4_K with up to MV_DMA_MA_MAX_ROWS rows and k <= 2048 on the
// DMA kernel with one to eight 16-row activation tiles (the decode path from
// 5 rows, the GEMM path from 17; the workspace is split_q8k_bytes: the split
// quantizer in its tiled layout, then one launch).
constexpr int MV_DMA_MA_MAX_ROWS = 128;
bool mv_dma_ma_fits(int type, int64_t k, int64_t m);
hipError_t launch_mv_dma_ma(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                            void* ws, int epi, hipStream_t s);
// stream.hip: Q4_K with 2..16 rows on weights of at least
// LLOOM_HIP_STREAM_MIN_MB (default 24) MB, k = 4096, 6144 or 8192 (and
// k = 2048 with 2..4 rows):
// the persistent pipelined MFMA decode kernel (the split quantizer in its
// tiled layout, then one launch; workspace split_q8k_bytes).
// CUs of the current device (asked once per device).
int cu_count();
bool mv_stream_fits(int type, int64_t n, int64_t k, int64_t m);
hipError_t launch_mv_stream(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                            void* ws, int epi, hipStream_t s);
// matvec.hip: Q4_K / Q6_K with any number of rows on the MFMA decode kernel,
// 64 activation rows per workgroup layer (the weights are re-read per
// layer): the workspace quantizer, then one launch.
hipError_t launch_mq(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* ws,
                     int epi, hipStream_t s);

// gemm.hip: m > 16 rows.  Q4_K on MFMA (mode: GEMM_F16, exact integer
// operands on fp16 MFMA, or GEMM_INT8, two int8 scale planes), the
// other types through decode tiles; qbuf is workspace for the prepared x.
constexpr int GEMM_F16 = 0, GEMM_INT8 = 1, GEMM_AUTO = 2;
// GEMM_AUTO's choice: the fp16 route to 320 rows (m = 256 on [8192, 2048]:
// 27.2 against 32.2 us), the int8 planes past (fp16 / int8: m = 352 33.8 /
// 33.5, 512 36.8 / 35.5, 768 52.1 / 50.4, 1024 56.1 / 54.9, 2048 108.8 /
// 102.4)
constexpr int64_t GEMM_AUTO_INT8_ROWS = 320;
inline int gemm_mode(int mode, int64_t m) {
    return mode == GEMM_AUTO ? (m > GEMM_AUTO_INT8_ROWS ? GEMM_INT8 : GEMM_F16) : mode;
}
// LLOOM_HIP_PREFILL_MMA: "int8", "f16", anything else or unset: auto
inline int gemm_mode_env(const char* e) {
    if (!e) return GEMM_AUTO;
    if (e[0] == 'i' && e[1] == 'n' && e[2] == 't' && e[3] == '8' && !e[4]) return GEMM_INT8;
    if (e[0] == 'f' && e[1] == '1' && e[2] == '6' && !e[3]) return GEMM_F16;
    return GEMM_AUTO;
}
hipError_t launch_gemm(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m,
                       void* qbuf, size_t ws_cap, int mode, int epi, hipStream_t s);
size_t gemm_workspace_bytes(int type, int64_t n, int64_t k, int64_t m, int mode);
// gemm_i8.hip: Q4_K prefill on int8 MFMA (two scale planes, f16-MFMA min
// term), 128 x 256 tiles; its activation and weight-record prep (one
// launch) runs in the same call.
bool gemm_i8_fits(int64_t n, int64_t k, int64_t m);
size_t gemm_i8_workspace_bytes(int64_t n, int64_t m, int64_t k);
hipError_t launch_gemm_i8(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* ws,
                          int epi, hipStream_t s);
// gemm_q6.hip: Q6_K from Q6_GEMM_MIN_ROWS rows (below, k_mv_mfma with 64
// activation rows a layer: m = 32 22.6 / 17.0 us against 21.7 for the GEMM
// on [2048, 8192] / [8192, 2048]; m = 64 31.2 / 23.3 against 22.3 / 23.2).
constexpr int Q6_GEMM_MIN_ROWS = 48;
bool q6_gemm_fits(int64_t n, int64_t k, int64_t m);
size_t q6_gemm_workspace_bytes(int64_t n, int64_t k, int64_t m);
hipError_t launch_q6_gemm(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* qbuf,
                          size_t ws_cap, int epi, hipStream_t s);
// gemm_q8.hip: Q8_0 from Q8_GEMM_MIN_ROWS rows (K in 256-element steps).
constexpr int Q8_GEMM_MIN_ROWS = 5;
bool q8_gemm_fits(int64_t n, int64_t k, int64_t m);
size_t q8_gemm_workspace_bytes(int64_t m, int64_t k);
hipError_t launch_q8_gemm(const void* w, const float* x, float* y, int64_t n, int64_t k, int64_t m, void* qbuf,
                          size_t ws_cap, int epi, hipStream_t s);

// moe.hip
// The router keeps two ints per expert in LDS.
constexpr int MOE_MAX_EXPERTS = 4096;
size_t moe_workspace_ints(int64_t n_experts, int64_t planes);
// mode MOE_ONE: y = W . x; MOE_PAIR: y = W . x and y2 = W2 . x in one
// launch; MOE_GLU: y = silu(W . x) * (W2 . x).  The workspace holds the
// routing ints (and, for a GLU over rows too long to stage, the up planes).
constexpr int MOE_ONE = 0, MOE_PAIR = 1, MOE_GLU = 2;
size_t moe_workspace_bytes(int64_t n_experts, int64_t planes, int64_t n, int64_t k, int mode);
bool moe_stages(int64_t k);
hipError_t launch_moe(int type, const void* w, int64_t n_experts, int64_t n, int64_t k, const float* x,
                      int64_t batch, int64_t in_dim1, const uint32_t* ids, int64_t topk, float* y, int* ws,
                      int* sticky, int mode, const void* w2, float* y2, hipStream_t s);

}  // namespace lloom
