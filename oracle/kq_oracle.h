/*
 * kq_oracle.h -- CPU oracle for the quantized-matmul path (TEST INFRASTRUCTURE).
 *
 * This is a plain-C restatement of lloom-tensor's CPU arithmetic for GGUF
 * Q8_0 / Q4_K / Q6_K weights and the Q8_0 / Q8_K activation blocks:
 *   lloom-tensor/src/quantized/k_quants.rs  (block layouts, from_float,
 *                                           to_float, vec_dot_unopt, matmul)
 *   lloom-tensor/src/quantized/utils.rs     (nearest_int, get_scale_min_k4,
 *                                           make_qx_quants, make_qkx1_quants)
 *   lloom-tensor/src/quantized/mod.rs       (matmul_t_indexed, the MoE arm)
 *
 * It is the CHECKER, never the product: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it.  It is compiled with
 * -ffp-contract=off and no fast-math so every f32 operation rounds exactly as
 * the Rust source does (Rust never contracts a*b+c into an FMA).
 *
 * Parity pins (each function is checked by tests/test_oracle_pins.py):
 *   f16 conversion        : exhaustive f16->f32, random f32->f16 vs numpy (RNE)
 *   Q4K/Q6K/Q8K quantize  : literal dequant values of quantized_tests.rs
 *                           :880-888, :974-982, :1021-1029, elementwise
 *                           bounds, RMSE <= 0.002 (:527-568)
 *   Q8_0 quantize         : closed form (absmax int8) + RMSE/dot bounds
 *   vec_dot_unopt         : ggml error bounds (:1117-1153), brute-force f64
 *                           dot of the dequantized operands, AVX restatement
 *                           |opt-unopt|/len <= 1e-6 (:1183)
 *   matmul                : GEMM rows == per-row decode bit for bit
 *                           (:1769-1903), scalar f64 oracle <= 0.02
 *   matmul_indexed        : closed form (dequantized row, sequential f32 dot)
 *   quantize -> matmul    : the StdRng known answers of quantized_matmul_
 *                           q4k/q6k/q8k (:1441-1542), with the inputs drawn
 *                           by tests/stdrng.py (rand 0.9's ChaCha12 StdRng
 *                           and its f32 sampling, restated and pinned by the
 *                           same tests' literals)
 */
#ifndef KQ_ORACLE_H
#define KQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids, GgmlDType::to_u32 (mod.rs:539-568). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q4K = 12, ORC_Q6K = 14, ORC_Q8K = 15 };

#define ORC_QK_K 256
#define ORC_QK8_0 32

/* k_quants.rs:154-159 */
typedef struct {
    uint16_t d;
    int8_t qs[32];
} orc_block_q8_0;

/* k_quants.rs:216-223 */
typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[128];
} orc_block_q4k;

/* k_quants.rs:254-261 */
typedef struct {
    uint8_t ql[128];
    uint8_t qh[64];
    int8_t scales[16];
    uint16_t d;
} orc_block_q6k;

/* k_quants.rs:264-270 */
typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} orc_block_q8k;

uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);

/* bytes of one block and elements per block of a type id, 0 if unknown */
size_t orc_block_bytes(int type);
size_t orc_block_elems(int type);

/* from_float over n elements (n % block == 0). Returns 0 or -1. */
int orc_quantize(int type, const float* x, size_t n, void* out);
/* to_float over n elements. */
int orc_dequantize(int type, const void* blocks, size_t n, float* y);
/* dequantize then f32 -> f16 (RNE), QTensor::dequantize_f16 (mod.rs:1072-1086). */
int orc_dequantize_f16(int type, const void* blocks, size_t n, uint16_t* y);

/* vec_dot_unopt of a weight row (type) against activation blocks
 * (Q8_0 for Q8_0, Q8_K for Q4K / Q6K / Q8K). */
float orc_vec_dot_unopt(int type, size_t n, const void* w, const void* a);

/* k_quants::matmul (k_quants.rs:2455-2641) with vec_dot_unopt as the dot:
 * quantize each lhs row, then dst[r, c] = vec_dot(w row c, lhs row r). */
int orc_matmul(int type, size_t m, size_t k, size_t n, const float* lhs, const void* w,
               float* dst);

/* QuantizedType::matmul_t_indexed (mod.rs:766-810).  w: [n_experts, n, k]
 * blocks, x: [batch, in_dim1, k] f32, ids: [batch, topk], dst [batch, topk, n].
 * Returns -1 when k is not a multiple of the block or an id is out of range. */
int orc_matmul_indexed(int type, const void* w, size_t n_experts, size_t n, size_t k, const float* x,
                       size_t in_dim1, const uint32_t* ids, size_t batch, size_t topk,
                       float* dst);

#ifdef __cplusplus
}
#endif
#endif
