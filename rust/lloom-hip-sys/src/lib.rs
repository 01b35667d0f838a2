//! Raw bindings to `liblloom_hip.so`, the gfx950 arm of lloom's quantized
//! matmul (Q8_0, Q4_K, Q6_K weights; f32 / f16 activations).
//!
//! One `extern "C"` block, one line per function of `include/lloom_hip.h`,
//! in the header's order and with its parameter names.  A CPU test of the
//! repository parses both files and fails on any difference in name, arity
//! or type, so the two cannot drift apart.
//!
//! Conventions (from the header): every call returns `LLOOM_HIP_OK` or an
//! error code, with the message in `lloom_hip_last_error()` (per thread);
//! `*_dev` pointers are device addresses; `stream` is a `hipStream_t` passed
//! as `*mut c_void` (null = the context's own stream); dtypes are GGUF type
//! ids (`LLOOM_HIP_F32` .. `LLOOM_HIP_Q8K`).
#![allow(non_camel_case_types)]
#![no_std]

use core::ffi::{c_char, c_int, c_void};

/// Opaque per-device context: device ordinal, stream, grow-only workspace.
#[repr(C)]
pub struct lloom_hip_ctx {
    _opaque: [u8; 0],
    _pin: core::marker::PhantomData<(*mut u8, core::marker::PhantomPinned)>,
}

// Return codes.
pub const LLOOM_HIP_OK: c_int = 0;
pub const LLOOM_HIP_EINVAL: c_int = 1;
pub const LLOOM_HIP_EDTYPE: c_int = 2;
pub const LLOOM_HIP_ESHAPE: c_int = 3;
pub const LLOOM_HIP_EEXPERT: c_int = 4;
pub const LLOOM_HIP_EHIP: c_int = 5;
pub const LLOOM_HIP_ENOMEM: c_int = 6;
pub const LLOOM_HIP_EDEVICE: c_int = 7;

// Type ids (GgmlDType::to_u32, mod.rs:505-568).
pub const LLOOM_HIP_F32: c_int = 0;
pub const LLOOM_HIP_F16: c_int = 1;
pub const LLOOM_HIP_Q8_0: c_int = 8;
pub const LLOOM_HIP_Q4K: c_int = 12;
pub const LLOOM_HIP_Q6K: c_int = 14;
pub const LLOOM_HIP_Q8K: c_int = 15;

// Prefill operand mode (lloom_hip_ctx_set_prefill_mma).
pub const LLOOM_HIP_MMA_F16: c_int = 0;
pub const LLOOM_HIP_MMA_INT8: c_int = 1;
pub const LLOOM_HIP_MMA_AUTO: c_int = 2;

// Fused stores (MvStore: none / Silu / MulInto).
pub const LLOOM_HIP_STORE_PLAIN: c_int = 0;
pub const LLOOM_HIP_STORE_SILU: c_int = 1;
pub const LLOOM_HIP_STORE_MUL_INTO: c_int = 2;

#[link(name = "lloom_hip")]
extern "C" {
    pub fn lloom_hip_last_error() -> *const c_char;
    pub fn lloom_hip_version() -> *const c_char;

    // Context (the CudaDevice / per-device workspace of cuda.rs and fast_mmvq.rs:49-80).
    pub fn lloom_hip_ctx_create(device: c_int, out: *mut *mut lloom_hip_ctx) -> c_int;
    pub fn lloom_hip_ctx_destroy(ctx: *mut lloom_hip_ctx) -> c_int;
    pub fn lloom_hip_ctx_stream(ctx: *mut lloom_hip_ctx) -> *mut c_void;
    pub fn lloom_hip_ctx_set_mv_rows_max(ctx: *mut lloom_hip_ctx, rows: c_int) -> c_int;
    pub fn lloom_hip_ctx_set_prefill_mma(ctx: *mut lloom_hip_ctx, mode: c_int) -> c_int;
    pub fn lloom_hip_ctx_sync(ctx: *mut lloom_hip_ctx) -> c_int;

    // Device memory (Device::qzeros, load_quantized, QCudaStorage::data).
    pub fn lloom_hip_alloc(ctx: *mut lloom_hip_ctx, bytes: usize, out_dev: *mut *mut c_void) -> c_int;
    pub fn lloom_hip_free(ctx: *mut lloom_hip_ctx, dev: *mut c_void) -> c_int;
    pub fn lloom_hip_memcpy_h2d(
        ctx: *mut lloom_hip_ctx,
        dst_dev: *mut c_void,
        src: *const c_void,
        bytes: usize,
        stream: *mut c_void,
    ) -> c_int;
    pub fn lloom_hip_memcpy_d2h(
        ctx: *mut lloom_hip_ctx,
        dst: *mut c_void,
        src_dev: *const c_void,
        bytes: usize,
        stream: *mut c_void,
    ) -> c_int;

    // Geometry (the padded buffer of cuda.rs:29-38).
    pub fn lloom_hip_weight_bytes(
        ggml_type: c_int,
        n: i64,
        k: i64,
        packed_bytes: *mut usize,
        alloc_bytes: *mut usize,
    ) -> c_int;

    // QStorage::quantize / from_float on the device (k_quants.rs from_float).
    pub fn lloom_hip_quantize(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        src_dev: *const f32,
        elems: i64,
        dst_dev: *mut c_void,
        stream: *mut c_void,
    ) -> c_int;
    // The VecDotType quantizer of the activations (BlockQ8_0 / BlockQ8K from_float).
    pub fn lloom_hip_quantize_act(
        ctx: *mut lloom_hip_ctx,
        vec_dot_type: c_int,
        x_dev: *const f32,
        m: i64,
        k: i64,
        out_dev: *mut c_void,
        stream: *mut c_void,
    ) -> c_int;
    // QStorage::dequantize / QTensor::dequantize_f16.
    pub fn lloom_hip_dequantize(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        w_dev: *const c_void,
        elems: i64,
        y_dev: *mut c_void,
        out_dtype: c_int,
        stream: *mut c_void,
    ) -> c_int;

    // CustomOp1 for QTensor (mod.rs:1901-2020): y[m, n] = x[m, k] . W[n, k]^T.
    pub fn lloom_hip_qmatmul(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        w_dev: *const c_void,
        n: i64,
        k: i64,
        x_dev: *const c_void,
        x_dtype: c_int,
        m: i64,
        y_dev: *mut c_void,
        y_dtype: c_int,
        stream: *mut c_void,
    ) -> c_int;
    // QMatMul::forward_silu / forward_mul_into.
    pub fn lloom_hip_qmatmul_store(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        w_dev: *const c_void,
        n: i64,
        k: i64,
        x_dev: *const c_void,
        x_dtype: c_int,
        m: i64,
        y_dev: *mut c_void,
        y_dtype: c_int,
        store: c_int,
        stream: *mut c_void,
    ) -> c_int;
    pub fn lloom_hip_qmatmul_workspace_bytes(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        n: i64,
        k: i64,
        m: i64,
        x_dtype: c_int,
        y_dtype: c_int,
        bytes: *mut usize,
    ) -> c_int;
    pub fn lloom_hip_ctx_reserve(ctx: *mut lloom_hip_ctx, bytes: usize) -> c_int;
    pub fn lloom_hip_ctx_workspace_bytes(ctx: *mut lloom_hip_ctx, bytes: *mut usize) -> c_int;
    // Tensor::to_dtype between F32 and F16 (the `act` casts of indexed_moe_forward_as).
    pub fn lloom_hip_cast(
        ctx: *mut lloom_hip_ctx,
        src_dev: *const c_void,
        src_dtype: c_int,
        dst_dev: *mut c_void,
        dst_dtype: c_int,
        count: i64,
        stream: *mut c_void,
    ) -> c_int;
    // No counterpart in the reference: lloom_hip_qmatmul for callers that cannot
    // allocate (graph capture, serving loops); a static per-GPU scratch array.
    pub fn lloom_hip_qmatmul_noalloc(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        w_dev: *const c_void,
        n: i64,
        k: i64,
        x_dev: *const c_void,
        x_dtype: c_int,
        m: i64,
        y_dev: *mut c_void,
        y_dtype: c_int,
        stream: *mut c_void,
    ) -> c_int;

    // QTensor::indexed_moe_forward* (mod.rs:1370-1645).
    pub fn lloom_hip_moe_matmul(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        w_dev: *const c_void,
        n_experts: i64,
        n: i64,
        k: i64,
        x_dev: *const f32,
        batch: i64,
        in_dim1: i64,
        ids_dev: *const u32,
        topk: i64,
        y_dev: *mut f32,
        strict: c_int,
        stream: *mut c_void,
    ) -> c_int;
    pub fn lloom_hip_moe_matmul_pair(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        w_gate_dev: *const c_void,
        w_up_dev: *const c_void,
        n_experts: i64,
        n: i64,
        k: i64,
        x_dev: *const f32,
        batch: i64,
        in_dim1: i64,
        ids_dev: *const u32,
        topk: i64,
        y_gate_dev: *mut f32,
        y_up_dev: *mut f32,
        strict: c_int,
        stream: *mut c_void,
    ) -> c_int;
    pub fn lloom_hip_moe_matmul_glu(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        w_gate_dev: *const c_void,
        w_up_dev: *const c_void,
        n_experts: i64,
        n: i64,
        k: i64,
        x_dev: *const f32,
        batch: i64,
        in_dim1: i64,
        ids_dev: *const u32,
        topk: i64,
        y_dev: *mut f32,
        strict: c_int,
        stream: *mut c_void,
    ) -> c_int;

    // QTensor::embedding (mod.rs:1101-1137).
    pub fn lloom_hip_embedding(
        ctx: *mut lloom_hip_ctx,
        ggml_type: c_int,
        w_dev: *const c_void,
        rows: i64,
        hidden: i64,
        ids_dev: *const u32,
        n_ids: i64,
        y_dev: *mut c_void,
        out_dtype: c_int,
        strict: c_int,
        stream: *mut c_void,
    ) -> c_int;

    // Host-side synthetic inputs (StdRng-seeded normal / uniform), for benches.
    pub fn lloom_hip_synth_normal(seed: u64, mean: f32, std: f32, out: *mut f32, count: i64) -> c_int;
    pub fn lloom_hip_synth_uniform(seed: u64, lo: f32, hi: f32, out: *mut f32, count: i64) -> c_int;
}
