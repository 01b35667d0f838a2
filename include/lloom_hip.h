/*
 * lloom_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul path.
 *
 * This is the drop-in boundary a `QStorage::Hip` arm of lloom-tensor binds
 * through a thin `lloom-hip-sys` crate (extern "C" declarations of exactly
 * these functions).  Plain pointers and sizes only: every buffer argument
 * named `*_dev` is device memory owned by the caller; `stream` is the
 * hipStream_t every launch of the call is queued on, used as given (NULL is
 * HIP's null stream; lloom_hip_ctx_stream() returns the context's own).
 *
 * Type ids are GGUF's (GgmlDType::to_u32, lloom-tensor/src/quantized/mod.rs
 * :539-568): F32 = 0, F16 = 1, Q8_0 = 8, Q4K = 12, Q6K = 14, Q8K = 15.
 * Weights are stored exactly as GGUF lays them out, [n, k] row-major rows of
 * blocks (mod.rs:1915 "self is transposed so n is first then k"), with a tail
 * pad (lloom_hip_weight_bytes) so vector loads past the last block stay in
 * bounds, as the CUDA arm pads (quantized/cuda.rs:29-38).
 *
 * Every function returns 0 on success or a LLOOM_HIP_E* code; the message of
 * the last failure on the calling thread is lloom_hip_last_error().  Bad
 * arguments are refused by name, never downgraded (quantized/route.rs:1-10).
 *
 * Threading: one context serves one stream at a time (the reference issues
 * every forward from one scheduler thread, lloom-engine/src/batch.rs:3-6).
 * The context's workspace is reused by consecutive calls in stream order.
 */
#ifndef LLOOM_HIP_H
#define LLOOM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    LLOOM_HIP_OK = 0,
    LLOOM_HIP_EINVAL = 1,      /* null pointer, negative or zero size        */
    LLOOM_HIP_EDTYPE = 2,      /* dtype not supported by this entry point   */
    LLOOM_HIP_ESHAPE = 3,      /* k not a multiple of the block, mismatch   */
    LLOOM_HIP_EEXPERT = 4,     /* an expert id >= n_experts                  */
    LLOOM_HIP_EHIP = 5,        /* a HIP runtime call failed                 */
    LLOOM_HIP_ENOMEM = 6,      /* device allocation failed                  */
    LLOOM_HIP_EDEVICE = 7      /* no gfx950 device at that ordinal          */
};

enum {
    LLOOM_HIP_F32 = 0,
    LLOOM_HIP_F16 = 1,
    LLOOM_HIP_Q8_0 = 8,
    LLOOM_HIP_Q4K = 12,
    LLOOM_HIP_Q6K = 14,
    LLOOM_HIP_Q8K = 15
};

typedef struct lloom_hip_ctx lloom_hip_ctx;

/* Message of the last failure on this thread ("" if none). */
const char* lloom_hip_last_error(void);

/* Library version string. */
const char* lloom_hip_version(void);

/* --------------------------------------------------------------- context --
 * Replaces CudaDevice::new (lloom-tensor/src/cuda_backend/device.rs:59-68)
 * for the quantized arm: binds a device ordinal, creates the context stream
 * and the grow-only workspace (quantized/fast_mmvq.rs:49-80). */
int lloom_hip_ctx_create(int device, lloom_hip_ctx** out);
int lloom_hip_ctx_destroy(lloom_hip_ctx* ctx);
/* The context stream (hipStream_t), for callers that share it. */
void* lloom_hip_ctx_stream(lloom_hip_ctx* ctx);
/* Decode/GEMM route knob: rows <= mv_rows_max take the fused matvec,
 * more rows the MFMA GEMM (default 16, range 1..16).  The reference's knobs
 * are MMVQ_MAX_BATCH (fast_mmvq.rs:38) and qmv.mm_from (tuning.rs:1413). */
int lloom_hip_ctx_set_mv_rows_max(lloom_hip_ctx* ctx, int rows);
/* Matrix-core family of the Q4_K prefill GEMM (m > mv_rows_max).  Both
 * compute the CPU arm's integer sums exactly (Q8_K activations, per-sub-block
 * integer scales) and combine them in f32 once per superblock:
 * LLOOM_HIP_MMA_F16: the integer operands x8 and sc * q, both exact in
 *   fp16, on v_mfma_f32_32x32x16_f16 (f32 accumulation of exact products),
 *   the min term as one more MFMA;
 * LLOOM_HIP_MMA_INT8: v_mfma_i32_32x32x32_i8 with the weights split into
 *   two int8 planes (sc = 8 sc_hi + sc_lo);
 * LLOOM_HIP_MMA_AUTO (default): F16 up to 320 rows, INT8 past (each the
 *   faster there).
 * LLOOM_HIP_PREFILL_MMA=f16|int8|auto sets the default of new contexts.
 * No counterpart in the reference (its CUDA arm has one MMQ kernel). */
enum { LLOOM_HIP_MMA_F16 = 0, LLOOM_HIP_MMA_INT8 = 1, LLOOM_HIP_MMA_AUTO = 2 };
int lloom_hip_ctx_set_prefill_mma(lloom_hip_ctx* ctx, int mode);

/* Wait for the device; report a device-side error (an out-of-range expert
 * id seen by a routed matmul, or an out-of-range embedding id) recorded
 * since the last check, and clear it. */
int lloom_hip_ctx_sync(lloom_hip_ctx* ctx);

/* ---------------------------------------------------------------- memory --
 * Device buffers for callers without a tensor runtime (the Rust HipStorage).
 * QCudaStorage::zeros / load_quantized (quantized/cuda.rs:624-637, 1005-1024). */
int lloom_hip_alloc(lloom_hip_ctx* ctx, size_t bytes, void** out_dev);
int lloom_hip_free(lloom_hip_ctx* ctx, void* dev);
int lloom_hip_memcpy_h2d(lloom_hip_ctx* ctx, void* dst_dev, const void* src, size_t bytes,
                         void* stream);
int lloom_hip_memcpy_d2h(lloom_hip_ctx* ctx, void* dst, const void* src_dev, size_t bytes,
                         void* stream);

/* Bytes of the packed blocks of an [n, k] weight (no pad), and the bytes to
 * allocate for it (with the tail pad).  k must be a multiple of the block. */
int lloom_hip_weight_bytes(int ggml_type, int64_t n, int64_t k, size_t* packed_bytes,
                           size_t* alloc_bytes);

/* -------------------------------------------------------------- quantize --
 * QTensor::quantize (mod.rs:919-938) -> QStorage::quantize (:257-267) for a
 * device f32 source: BlockQ8_0/Q4K/Q6K/Q8K::from_float (k_quants.rs:738-767,
 * 1622-1680, 2174-2244, 2400-2438), bit for bit, on the GPU.  elems must be
 * a multiple of the block size. */
int lloom_hip_quantize(lloom_hip_ctx* ctx, int ggml_type, const float* src_dev, int64_t elems,
                       void* dst_dev, void* stream);

/* Activation quantization of an [m, k] f32 matrix to the weight's VecDotType
 * (Q8_0 for Q8_0 weights, Q8K for Q4K/Q6K), as k_quants::matmul does before
 * its dots (k_quants.rs:2477-2508).  Bit-exact with from_float.  The CUDA arm
 * quantizes to Q8_1 instead (quantized/cuda.rs:48-103). */
int lloom_hip_quantize_act(lloom_hip_ctx* ctx, int vec_dot_type, const float* x_dev, int64_t m,
                           int64_t k, void* out_dev, void* stream);

/* ------------------------------------------------------------ dequantize --
 * QTensor::dequantize / dequantize_f16 (mod.rs:1065-1086), to_float of
 * k_quants.rs:720-736, 1747-1774, 2327-2358, 2440-2451; out_dtype F32 or F16
 * (f16 = RNE of the f32 value, as Tensor::to_dtype does).  Bit-exact. */
int lloom_hip_dequantize(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t elems,
                         void* y_dev, int out_dtype, void* stream);

/* ---------------------------------------------------------------- matmul --
 * QMatMul::forward -> CustomOp1 for QTensor (mod.rs:1901-2020, 2022-2025):
 * y[m, n] = x[m, k] . W[n, k]^T with W packed (ggml_type Q8_0/Q4K/Q6K) and
 * x f32.  Replaces QCudaStorage::fwd (quantized/cuda.rs:862-894).  Each call
 * quantizes x to the VecDotType exactly as the CPU arm does; the dots then
 * run in integer arithmetic with f32 scales, within 1e-3 * max|y row| of the
 * CPU result.  x_dtype / y_dtype: F32 or F16 each.  F16 activations are
 * the CPU arm's matmul_t_f16 (mod.rs:722,761; k_quants.rs:2802-2835): x
 * widened to f32 exactly, then the f32 path; an F16 y is each f32 sum
 * rounded to nearest-even.  The conversions run in the workspace. */
int lloom_hip_qmatmul(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k,
                      const void* x_dev, int x_dtype, int64_t m, void* y_dev, int y_dtype,
                      void* stream);

/* Store epilogues of the matmul: QMatMul::forward_silu and forward_mul_into
 * (mod.rs:2102-2156), the MvStore::{Silu, MulInto} blocks of the reference's
 * Metal matvec store (mod.rs:1667-1696, kernels/metal_src/
 * quantized_store.metal): the product is formed as in lloom_hip_qmatmul and
 * then stored as
 *   LLOOM_HIP_STORE_PLAIN     y = v
 *   LLOOM_HIP_STORE_SILU      y = v / (1 + exp(-v))
 *   LLOOM_HIP_STORE_MUL_INTO  y = y * v  (y is read: the SwiGLU gate's own
 *                             buffer holding silu(g), which then holds
 *                             silu(g) * u; y must have no other reader)
 * in the same launch, on every row count (decode and prefill); the
 * reference serves these on Metal only and returns None elsewhere. */
enum { LLOOM_HIP_STORE_PLAIN = 0, LLOOM_HIP_STORE_SILU = 1, LLOOM_HIP_STORE_MUL_INTO = 2 };
int lloom_hip_qmatmul_store(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k,
                            const void* x_dev, int x_dtype, int64_t m, void* y_dev, int y_dtype, int store,
                            void* stream);

/* Workspace a lloom_hip_qmatmul call of this shape needs on ctx (NULL: a
 * new context's defaults), so a caller can reserve it before capturing the
 * call into a graph.  The reference's counterpart is the CUDA arm's
 * grow-only workspace (quantized/fast_mmvq.rs:49-80), sized on first use. */
int lloom_hip_qmatmul_workspace_bytes(lloom_hip_ctx* ctx, int ggml_type, int64_t n, int64_t k, int64_t m,
                                      int x_dtype, int y_dtype, size_t* bytes);
/* Grow the context workspace to at least `bytes` now.  A call that would
 * grow it while its stream is being captured fails with LLOOM_HIP_ENOMEM
 * instead; outgrown workspaces stay allocated until lloom_hip_ctx_destroy
 * (graphs captured earlier keep using theirs). */
int lloom_hip_ctx_reserve(lloom_hip_ctx* ctx, size_t bytes);
/* Bytes the context workspace holds now. */
int lloom_hip_ctx_workspace_bytes(lloom_hip_ctx* ctx, size_t* bytes);

/* Tensor::to_dtype between F32 and F16 on the device (f32 -> f16 round to
 * nearest even, as half::f16::from_f32), for the casts the reference makes
 * around this path: indexed_moe_forward_as casting x to `act`
 * (mod.rs:1567-1571).  src and dst 16-byte aligned. */
int lloom_hip_cast(lloom_hip_ctx* ctx, const void* src_dev, int src_dtype, void* dst_dev, int dst_dtype,
                   int64_t count, void* stream);

/* lloom_hip_qmatmul without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workspace is a static device array of 32 MiB per GPU, held until the
 * process ends (its address is looked up on the first call on each device);
 * a call that needs more fails with LLOOM_HIP_ENOMEM
 * (lloom_hip_qmatmul_workspace_bytes tells ahead).  Every call on one GPU
 * shares that array: calls that overlap on one GPU (other streams, other
 * contexts) race.  Same arguments, results and refusals as
 * lloom_hip_qmatmul. */
int lloom_hip_qmatmul_noalloc(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k,
                              const void* x_dev, int x_dtype, int64_t m, void* y_dev, int y_dtype, void* stream);

/* ------------------------------------------------------- routed experts --
 * QTensor::indexed_moe_forward{,_with,_as} (mod.rs:1560-1645), CPU arm
 * matmul_t_indexed (mod.rs:766-810): W [n_experts, n, k] packed, x f32
 * [batch, in_dim1, k] with in_dim1 in {1, topk}, ids u32 [batch, topk],
 * y f32 [batch, topk, n]; plane (b, t) = x[b, t or 0] . W[ids[b, t]]^T.
 * The dots take the f32 activations as they are (no activation
 * quantization, as on the CPU arm) against the exactly dequantized weights,
 * factored per 16-element run: scale * sum(q * x) - min * sum(x), the CPU
 * arm's dot of a dequantized row in another rounding order.  n_experts is at
 * most 4096 (LLOOM_HIP_ESHAPE beyond).  An id >= n_experts yields a zero plane
 * and LLOOM_HIP_EEXPERT from this call (it synchronizes the stream to read
 * the device flag) unless strict is 0, in which case the next
 * lloom_hip_ctx_sync reports it. */
int lloom_hip_moe_matmul(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n_experts,
                         int64_t n, int64_t k, const float* x_dev, int64_t batch, int64_t in_dim1,
                         const uint32_t* ids_dev, int64_t topk, float* y_dev, int strict,
                         void* stream);

/* Gate and up of one routed layer in one launch: QTensor::
 * indexed_moe_forward_pair (mod.rs:1365-1455; one Metal launch,
 * kernel_mul_mv_id2, on the reference).  Both stacks have the same type and
 * shape [n_experts, n, k]; y_gate and y_up are each what
 * lloom_hip_moe_matmul computes for its weight, bit for bit. */
int lloom_hip_moe_matmul_pair(lloom_hip_ctx* ctx, int ggml_type, const void* w_gate_dev,
                              const void* w_up_dev, int64_t n_experts, int64_t n, int64_t k,
                              const float* x_dev, int64_t batch, int64_t in_dim1,
                              const uint32_t* ids_dev, int64_t topk, float* y_gate_dev,
                              float* y_up_dev, int strict, void* stream);

/* silu(gate) * up of the pair in one launch, y [batch, topk, n]: QTensor::
 * indexed_moe_forward_glu_as (mod.rs:1457-1531), silu_mul's element
 * (silu(g) = g / (1 + exp(-g)), then the product) over the two sums the
 * pair stores. */
int lloom_hip_moe_matmul_glu(lloom_hip_ctx* ctx, int ggml_type, const void* w_gate_dev,
                             const void* w_up_dev, int64_t n_experts, int64_t n, int64_t k,
                             const float* x_dev, int64_t batch, int64_t in_dim1,
                             const uint32_t* ids_dev, int64_t topk, float* y_dev, int strict,
                             void* stream);

/* ------------------------------------------------------------- embedding --
 * QTensor::embedding (mod.rs:1101-1137; CPU arm QuantizedType::embedding,
 * :812-838; CUDA quantized.cu get_rows): y[i, :] = to_float of weight row
 * ids[i] of a packed [rows, hidden] weight, bit-exact; out_dtype F32 or F16
 * (RNE of the f32 value).  hidden must be a multiple of the block.  An
 * id >= rows stores a zero row and fails the call with LLOOM_HIP_EEXPERT
 * ("embedding id ... is out of range"; the call synchronizes to read the
 * device flag) unless strict is 0, when the next lloom_hip_ctx_sync reports
 * it.  n_ids = 0 is a no-op. */
int lloom_hip_embedding(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t rows,
                        int64_t hidden, const uint32_t* ids_dev, int64_t n_ids, void* y_dev,
                        int out_dtype, int strict, void* stream);

/* ------------------------------------------------------- synthetic data --
 * The benchmark/test input generator (not part of the reference): SplitMix64
 * seeding xoshiro256**, Box-Muller normals N(mean, std) written as f32 into a
 * host buffer.  Deterministic for a seed on every host. */
int lloom_hip_synth_normal(uint64_t seed, float mean, float std, float* out, int64_t count);
int lloom_hip_synth_uniform(uint64_t seed, float lo, float hi, float* out, int64_t count);

#ifdef __cplusplus
}
#endif
#endif
