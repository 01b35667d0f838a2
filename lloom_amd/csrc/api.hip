// api.hip -- the C ABI (include/lloom_hip.h): argument checks, the context
// (device, stream, grow-only workspace) and dispatch to the kernels.
//
// The argument checks mirror the CPU arm's refusals, by name:
//   k not a multiple of the block     mod.rs:775-780, check_shape (mod.rs:900-907)
//   x last dim != weight k            CustomOp1::cpu_fwd (mod.rs:1920-1923)
//   MoE shapes                        indexed_moe_forward_as (mod.rs:1616-1623)
//   expert id out of range            matmul_t_indexed (mod.rs:796-798)
//   unsupported dtype                 QStorage::from_data (mod.rs:206-220)
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/lloom_hip.h"
#include "kernels.hpp"
#include "kq_common.hpp"
#include "api_internal.hpp"

using namespace lloom;

static thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}


// The caller's stream, verbatim: NULL is HIP's null stream (torch's default
// stream handle is 0), never silently another stream.
static hipStream_t pick_stream(lloom_hip_ctx* ctx, void* stream) {
    (void)ctx;
    return (hipStream_t)stream;
}

static bool is_weight_type(int t) { return t == T_Q8_0 || t == T_Q4K || t == T_Q6K; }

static const char* type_name(int t) {
    switch (t) {
        case T_F32: return "F32";
        case T_F16: return "F16";
        case T_Q8_0: return "Q8_0";
        case T_Q4K: return "Q4K";
        case T_Q6K: return "Q6K";
        case T_Q8K: return "Q8K";
    }
    return "unknown";
}

// Workspace of at least `bytes`, 256-byte aligned; grows, never shrinks
// (the CUDA arm's per-device workspace, quantized/fast_mmvq.rs:49-80).  A
// growth allocates a new buffer of at least twice the old size and retires
// the old one until the context is destroyed (see lloom_hip_ctx).  Growth is
// refused while `s` is being captured into a graph: an allocation there
// would not be part of the graph, so the caller reserves the workspace first
// (lloom_hip_ctx_reserve).
static int ensure_ws(lloom_hip_ctx* ctx, size_t bytes, hipStream_t s, void** out) {
    if (bytes > ctx->ws_bytes) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
            return fail(LLOOM_HIP_ENOMEM,
                        "the call needs a workspace of %zu bytes and the context holds %zu: it cannot grow while "
                        "the stream is being captured (reserve it first with lloom_hip_ctx_reserve)",
                        bytes, ctx->ws_bytes);
        size_t want = bytes > 2 * ctx->ws_bytes ? bytes : 2 * ctx->ws_bytes;
        want = (want + 0xFFFFF) & ~(size_t)0xFFFFF;
        void* fresh = nullptr;
        if (hipMalloc(&fresh, want) != hipSuccess)
            return fail(LLOOM_HIP_ENOMEM, "workspace allocation of %zu bytes failed", want);
        if (ctx->ws) ctx->retired.push_back(ctx->ws);
        ctx->ws = fresh;
        ctx->ws_bytes = want;
    }
    *out = ctx->ws;
    return LLOOM_HIP_OK;
}

extern "C" {

const char* lloom_hip_last_error(void) { return g_err.c_str(); }

const char* lloom_hip_version(void) { return "lloom-hip 0.1 (gfx950)"; }

int lloom_hip_ctx_create(int device, lloom_hip_ctx** out) {
    if (!out) return fail(LLOOM_HIP_EINVAL, "ctx_create: out is null");
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count)
        return fail(LLOOM_HIP_EDEVICE, "ctx_create: no HIP device %d (%d visible)", device, count);
    hipDeviceProp_t prop;
    HIP_OK(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(LLOOM_HIP_EDEVICE, "ctx_create: device %d is %s, this library is built for gfx950", device,
                    prop.gcnArchName);
    HIP_OK(hipSetDevice(device));
    lloom_hip_ctx* c = new lloom_hip_ctx();
    c->device = device;
    c->prefill_mma = gemm_mode_env(getenv("LLOOM_HIP_PREFILL_MMA"));
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return fail(LLOOM_HIP_EHIP, "ctx_create: stream creation failed");
    }
    if (hipMalloc(&c->flags, 256) != hipSuccess) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return fail(LLOOM_HIP_ENOMEM, "ctx_create: flag allocation failed");
    }
    (void)hipMemset(c->flags, 0, 256);
    (void)hipDeviceSynchronize();
    *out = c;
    return LLOOM_HIP_OK;
}

int lloom_hip_ctx_destroy(lloom_hip_ctx* ctx) {
    if (!ctx) return LLOOM_HIP_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();  // calls may have queued work on any stream
    if (ctx->ws) (void)hipFree(ctx->ws);
    for (void* p : ctx->retired) (void)hipFree(p);
    if (ctx->flags) (void)hipFree(ctx->flags);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return LLOOM_HIP_OK;
}

void* lloom_hip_ctx_stream(lloom_hip_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int lloom_hip_ctx_set_mv_rows_max(lloom_hip_ctx* ctx, int rows) {
    if (!ctx) return fail(LLOOM_HIP_EINVAL, "set_mv_rows_max: null context");
    if (rows < 1 || rows > 16) return fail(LLOOM_HIP_EINVAL, "set_mv_rows_max: %d is outside 1..16", rows);
    ctx->mv_rows_max = rows;
    return LLOOM_HIP_OK;
}

int lloom_hip_ctx_set_prefill_mma(lloom_hip_ctx* ctx, int mode) {
    if (!ctx) return fail(LLOOM_HIP_EINVAL, "set_prefill_mma: null context");
    if (mode != LLOOM_HIP_MMA_F16 && mode != LLOOM_HIP_MMA_INT8 && mode != LLOOM_HIP_MMA_AUTO)
        return fail(LLOOM_HIP_EINVAL, "set_prefill_mma: mode %d is none of F16 (0), INT8 (1), AUTO (2)", mode);
    ctx->prefill_mma = mode == LLOOM_HIP_MMA_INT8 ? GEMM_INT8 : mode == LLOOM_HIP_MMA_F16 ? GEMM_F16 : GEMM_AUTO;
    return LLOOM_HIP_OK;
}

int lloom_hip_ctx_sync(lloom_hip_ctx* ctx) {
    if (!ctx) return fail(LLOOM_HIP_EINVAL, "ctx_sync: null context");
    HIP_OK(hipSetDevice(ctx->device));
    HIP_OK(hipDeviceSynchronize());
    int flag = 0;
    HIP_OK(hipMemcpy(&flag, ctx->flags, sizeof(int), hipMemcpyDeviceToHost));
    if (flag) {
        int zero = 0;
        HIP_OK(hipMemcpy(ctx->flags, &zero, sizeof(int), hipMemcpyHostToDevice));
        return fail(LLOOM_HIP_EEXPERT, "a routed matmul or embedding saw an id out of range");
    }
    return LLOOM_HIP_OK;
}

int lloom_hip_alloc(lloom_hip_ctx* ctx, size_t bytes, void** out_dev) {
    if (!ctx || !out_dev) return fail(LLOOM_HIP_EINVAL, "alloc: null argument");
    HIP_OK(hipSetDevice(ctx->device));
    if (hipMalloc(out_dev, bytes ? bytes : 1) != hipSuccess)
        return fail(LLOOM_HIP_ENOMEM, "alloc: %zu bytes failed", bytes);
    return LLOOM_HIP_OK;
}

int lloom_hip_free(lloom_hip_ctx* ctx, void* dev) {
    if (!ctx) return fail(LLOOM_HIP_EINVAL, "free: null context");
    if (dev) HIP_OK(hipFree(dev));
    return LLOOM_HIP_OK;
}

int lloom_hip_memcpy_h2d(lloom_hip_ctx* ctx, void* dst_dev, const void* src, size_t bytes, void* stream) {
    if (!ctx || (!dst_dev && bytes) || (!src && bytes)) return fail(LLOOM_HIP_EINVAL, "memcpy_h2d: null argument");
    hipStream_t s = pick_stream(ctx, stream);
    HIP_OK(hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, s));
    HIP_OK(hipStreamSynchronize(s));
    return LLOOM_HIP_OK;
}

int lloom_hip_memcpy_d2h(lloom_hip_ctx* ctx, void* dst, const void* src_dev, size_t bytes, void* stream) {
    if (!ctx || (!dst && bytes) || (!src_dev && bytes)) return fail(LLOOM_HIP_EINVAL, "memcpy_d2h: null argument");
    hipStream_t s = pick_stream(ctx, stream);
    HIP_OK(hipMemcpyAsync(dst, src_dev, bytes, hipMemcpyDeviceToHost, s));
    HIP_OK(hipStreamSynchronize(s));
    return LLOOM_HIP_OK;
}

int lloom_hip_weight_bytes(int ggml_type, int64_t n, int64_t k, size_t* packed_bytes, size_t* alloc_bytes) {
    int be = block_elems(ggml_type);
    if (!be) return fail(LLOOM_HIP_EDTYPE, "weight_bytes: dtype %s (%d) is not a block type", type_name(ggml_type), ggml_type);
    if (n < 0 || k < 0) return fail(LLOOM_HIP_EINVAL, "weight_bytes: negative shape");
    if (k % be) return fail(LLOOM_HIP_ESHAPE, "weight_bytes: k %lld is not divisible by block size %d", (long long)k, be);
    size_t b = (size_t)n * (size_t)(k / be) * (size_t)block_bytes(ggml_type);
    if (packed_bytes) *packed_bytes = b;
    if (alloc_bytes) *alloc_bytes = b + WEIGHT_TAIL_PAD;
    return LLOOM_HIP_OK;
}

int lloom_hip_quantize(lloom_hip_ctx* ctx, int ggml_type, const float* src_dev, int64_t elems, void* dst_dev,
                       void* stream) {
    if (!ctx || !src_dev || !dst_dev) return fail(LLOOM_HIP_EINVAL, "quantize: null argument");
    int be = block_elems(ggml_type);
    if (!be) return fail(LLOOM_HIP_EDTYPE, "quantize: %s (%d) is not supported on the HIP quantized path", type_name(ggml_type), ggml_type);
    if (elems <= 0 || elems % be)
        return fail(LLOOM_HIP_ESHAPE, "quantize: tensor size %lld is not divisible by block size %d", (long long)elems, be);
    if ((uintptr_t)src_dev % 16 || (uintptr_t)dst_dev % 4)
        return fail(LLOOM_HIP_EINVAL, "quantize: src must be 16-byte and dst 4-byte aligned");
    HIP_OK(hipSetDevice(ctx->device));
    HIP_OK(launch_quantize_weights(ggml_type, src_dev, dst_dev, elems, pick_stream(ctx, stream)));
    return LLOOM_HIP_OK;
}

int lloom_hip_quantize_act(lloom_hip_ctx* ctx, int vec_dot_type, const float* x_dev, int64_t m, int64_t k,
                           void* out_dev, void* stream) {
    if (!ctx || !x_dev || !out_dev) return fail(LLOOM_HIP_EINVAL, "quantize_act: null argument");
    if (vec_dot_type != T_Q8_0 && vec_dot_type != T_Q8K)
        return fail(LLOOM_HIP_EDTYPE, "quantize_act: %s (%d) is not a vec-dot type (Q8_0 or Q8K)", type_name(vec_dot_type), vec_dot_type);
    int be = block_elems(vec_dot_type);
    if (m <= 0 || k <= 0) return fail(LLOOM_HIP_EINVAL, "quantize_act: empty shape (%lld, %lld)", (long long)m, (long long)k);
    if (k % be) return fail(LLOOM_HIP_ESHAPE, "quantize_act: k %lld is not divisible by block size %d", (long long)k, be);
    if ((uintptr_t)x_dev % 16 || (uintptr_t)out_dev % 4)
        return fail(LLOOM_HIP_EINVAL, "quantize_act: x must be 16-byte and out 4-byte aligned");
    HIP_OK(hipSetDevice(ctx->device));
    HIP_OK(launch_quantize_act(vec_dot_type, x_dev, out_dev, m * k, pick_stream(ctx, stream)));
    return LLOOM_HIP_OK;
}

int lloom_hip_dequantize(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t elems, void* y_dev,
                         int out_dtype, void* stream) {
    if (!ctx || !w_dev || !y_dev) return fail(LLOOM_HIP_EINVAL, "dequantize: null argument");
    int be = block_elems(ggml_type);
    if (!be) return fail(LLOOM_HIP_EDTYPE, "dequantize: %s (%d) is not supported on the HIP quantized path", type_name(ggml_type), ggml_type);
    if (out_dtype != T_F32 && out_dtype != T_F16)
        return fail(LLOOM_HIP_EDTYPE, "dequantize: output dtype %s (%d) must be F32 or F16", type_name(out_dtype), out_dtype);
    if (elems <= 0 || elems % be)
        return fail(LLOOM_HIP_ESHAPE, "dequantize: %lld elements is not divisible by block size %d", (long long)elems, be);
    if ((uintptr_t)w_dev % 4) return fail(LLOOM_HIP_EINVAL, "dequantize: weight must be 4-byte aligned");
    HIP_OK(hipSetDevice(ctx->device));
    HIP_OK(launch_dequantize(ggml_type, w_dev, y_dev, out_dtype, elems, pick_stream(ctx, stream)));
    return LLOOM_HIP_OK;
}

}  // extern "C"

// The route a qmatmul call takes and the workspace it needs.  Activations
// in F16 (matmul_t_f16, k_quants.rs:2802-2835: the f16 lhs converted to f32,
// quantized to the VecDotType and dotted exactly as the f32 path; each f32
// sum rounded to f16) are converted into the workspace first, and F16
// outputs are formed in f32 in the workspace and rounded at the end.

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

QmmPlan qmm_plan(int mv_rows_max, int prefill_mma, int ggml_type, int64_t n, int64_t k, int64_t m,
                        int x_dtype, int y_dtype) {
    QmmPlan p;
    // Q8_0 from 5 rows takes the GEMM (the decode kernel's time grows with
    // the rows, 10.6 us at m = 4 and 22.1 at m = 8 on [8192, 2048]; the
    // split-K GEMM with its activation prep is 11.1 us from m = 3 to 9)
    p.decode = m <= mv_rows_max && !(ggml_type == T_Q8_0 && m >= Q8_GEMM_MIN_ROWS && q8_gemm_fits(n, k, m));
    p.path_bytes = p.decode ? matvec_workspace_bytes(ggml_type, n, k, m)
                            : gemm_workspace_bytes(ggml_type, n, k, m, prefill_mma);
    p.x32_off = align256(p.path_bytes);
    p.y32_off = p.x32_off + (x_dtype == T_F16 ? align256((size_t)m * k * sizeof(float)) : 0);
    p.total = p.y32_off + (y_dtype == T_F16 ? align256((size_t)m * n * sizeof(float)) : 0);
    return p;
}

int qmatmul_check(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k,
                         const void* x_dev, int x_dtype, int64_t m, void* y_dev, int y_dtype, int epi) {
    if (!ctx || !w_dev || !x_dev || !y_dev) return fail(LLOOM_HIP_EINVAL, "qmatmul: null argument");
    if (!is_weight_type(ggml_type))
        return fail(LLOOM_HIP_EDTYPE, "qmatmul: weight dtype %s (%d) is not supported on the HIP quantized path (Q8_0, Q4K, Q6K)", type_name(ggml_type), ggml_type);
    if ((x_dtype != T_F32 && x_dtype != T_F16) || (y_dtype != T_F32 && y_dtype != T_F16))
        return fail(LLOOM_HIP_EDTYPE, "qmatmul: activation dtypes %s -> %s: x and y must each be F32 or F16", type_name(x_dtype), type_name(y_dtype));
    (void)epi;
    int be = block_elems(ggml_type);
    if (n <= 0 || k <= 0 || m <= 0)
        return fail(LLOOM_HIP_EINVAL, "qmatmul: empty shape m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
    if (k % be) return fail(LLOOM_HIP_ESHAPE, "qmatmul: k %lld is not divisible by block size %d", (long long)k, be);
    if (n > INT32_MAX || k > INT32_MAX || m > INT32_MAX) return fail(LLOOM_HIP_ESHAPE, "qmatmul: dimension exceeds 2^31");
    if ((uintptr_t)w_dev % (ggml_type == T_Q4K ? 16 : 4))
        return fail(LLOOM_HIP_EINVAL, "qmatmul: weight pointer is not %d-byte aligned", ggml_type == T_Q4K ? 16 : 4);
    if ((uintptr_t)x_dev % 16) return fail(LLOOM_HIP_EINVAL, "qmatmul: x must be 16-byte aligned");
    if (y_dtype == T_F16 && (uintptr_t)y_dev % 16) return fail(LLOOM_HIP_EINVAL, "qmatmul: an F16 y must be 16-byte aligned");
    return LLOOM_HIP_OK;
}

// The call on a workspace `ws` of `ws_cap` bytes (the plan's total fits).
int qmatmul_run(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k, const void* x_dev,
                       int x_dtype, int64_t m, void* y_dev, int y_dtype, int epi, hipStream_t s, const QmmPlan& p,
                       void* ws, size_t ws_cap) {
    const float* x = (const float*)x_dev;
    float* y = (float*)y_dev;
    if (x_dtype == T_F16) {
        float* x32 = (float*)((uint8_t*)ws + p.x32_off);
        HIP_OK(launch_cast(T_F16, x_dev, T_F32, x32, m * k, s));
        x = x32;
    }
    if (y_dtype == T_F16) {
        y = (float*)((uint8_t*)ws + p.y32_off);
        // the multiply-into store reads y: its f16 values, widened exactly
        if (epi == EPI_MUL_INTO) HIP_OK(launch_cast(T_F16, y_dev, T_F32, y, m * n, s));
    }
    if (p.decode)
        HIP_OK(launch_matvec(ggml_type, w_dev, x, y, n, k, m, ws, epi, s));
    else
        HIP_OK(launch_gemm(ggml_type, w_dev, x, y, n, k, m, ws, p.total > p.x32_off ? p.x32_off : ws_cap,
                           ctx->prefill_mma, epi, s));
    if (y_dtype == T_F16) HIP_OK(launch_cast(T_F32, y, T_F16, y_dev, m * n, s));
    return LLOOM_HIP_OK;
}

static int qmatmul_impl(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k,
                        const void* x_dev, int x_dtype, int64_t m, void* y_dev, int y_dtype, int epi, void* stream) {
    if (int rc = qmatmul_check(ctx, ggml_type, w_dev, n, k, x_dev, x_dtype, m, y_dev, y_dtype, epi)) return rc;
    HIP_OK(hipSetDevice(ctx->device));
    hipStream_t s = pick_stream(ctx, stream);
    std::lock_guard<std::mutex> lock(ctx->mu);
    const QmmPlan p = qmm_plan(ctx->mv_rows_max, ctx->prefill_mma, ggml_type, n, k, m, x_dtype, y_dtype);
    void* ws = nullptr;
    if (p.total) {
        if (int rc = ensure_ws(ctx, p.total, s, &ws)) return rc;
    }
    return qmatmul_run(ctx, ggml_type, w_dev, n, k, x_dev, x_dtype, m, y_dev, y_dtype, epi, s, p, ws, ctx->ws_bytes);
}

static int moe_impl(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, const void* w2_dev, int64_t n_experts,
                    int64_t n, int64_t k, const float* x_dev, int64_t batch, int64_t in_dim1,
                    const uint32_t* ids_dev, int64_t topk, float* y_dev, float* y2_dev, int mode, int strict,
                    void* stream);

extern "C" {

int lloom_hip_qmatmul(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k,
                      const void* x_dev, int x_dtype, int64_t m, void* y_dev, int y_dtype, void* stream) {
    return qmatmul_impl(ctx, ggml_type, w_dev, n, k, x_dev, x_dtype, m, y_dev, y_dtype, EPI_STORE, stream);
}

int lloom_hip_qmatmul_store(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n, int64_t k,
                            const void* x_dev, int x_dtype, int64_t m, void* y_dev, int y_dtype, int store,
                            void* stream) {
    if (store != LLOOM_HIP_STORE_PLAIN && store != LLOOM_HIP_STORE_SILU && store != LLOOM_HIP_STORE_MUL_INTO)
        return fail(LLOOM_HIP_EINVAL, "qmatmul_store: store %d is not PLAIN (0), SILU (1) or MUL_INTO (2)", store);
    const int epi = store == LLOOM_HIP_STORE_SILU ? EPI_SILU : store == LLOOM_HIP_STORE_MUL_INTO ? EPI_MUL_INTO : EPI_STORE;
    return qmatmul_impl(ctx, ggml_type, w_dev, n, k, x_dev, x_dtype, m, y_dev, y_dtype, epi, stream);
}

int lloom_hip_qmatmul_workspace_bytes(lloom_hip_ctx* ctx, int ggml_type, int64_t n, int64_t k, int64_t m, int x_dtype,
                                      int y_dtype, size_t* bytes) {
    if (!bytes) return fail(LLOOM_HIP_EINVAL, "qmatmul_workspace_bytes: null output");
    if (!is_weight_type(ggml_type))
        return fail(LLOOM_HIP_EDTYPE, "qmatmul_workspace_bytes: weight dtype %s (%d) is not supported", type_name(ggml_type), ggml_type);
    if ((x_dtype != T_F32 && x_dtype != T_F16) || (y_dtype != T_F32 && y_dtype != T_F16))
        return fail(LLOOM_HIP_EDTYPE, "qmatmul_workspace_bytes: x and y must each be F32 or F16");
    if (n <= 0 || k <= 0 || m <= 0 || k % block_elems(ggml_type))
        return fail(LLOOM_HIP_ESHAPE, "qmatmul_workspace_bytes: bad shape m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
    const int rows_max = ctx ? ctx->mv_rows_max : 16;
    const int mma = ctx ? ctx->prefill_mma : gemm_mode_env(getenv("LLOOM_HIP_PREFILL_MMA"));
    *bytes = qmm_plan(rows_max, mma, ggml_type, n, k, m, x_dtype, y_dtype).total;
    return LLOOM_HIP_OK;
}

int lloom_hip_ctx_reserve(lloom_hip_ctx* ctx, size_t bytes) {
    if (!ctx) return fail(LLOOM_HIP_EINVAL, "ctx_reserve: null context");
    HIP_OK(hipSetDevice(ctx->device));
    std::lock_guard<std::mutex> lock(ctx->mu);
    void* ws = nullptr;
    return bytes ? ensure_ws(ctx, bytes, nullptr, &ws) : LLOOM_HIP_OK;
}

int lloom_hip_ctx_workspace_bytes(lloom_hip_ctx* ctx, size_t* bytes) {
    if (!ctx || !bytes) return fail(LLOOM_HIP_EINVAL, "ctx_workspace_bytes: null argument");
    std::lock_guard<std::mutex> lock(ctx->mu);
    *bytes = ctx->ws_bytes;
    return LLOOM_HIP_OK;
}

int lloom_hip_cast(lloom_hip_ctx* ctx, const void* src_dev, int src_dtype, void* dst_dev, int dst_dtype, int64_t count,
                   void* stream) {
    if (!ctx || (count && (!src_dev || !dst_dev))) return fail(LLOOM_HIP_EINVAL, "cast: null argument");
    if (!((src_dtype == T_F32 && dst_dtype == T_F16) || (src_dtype == T_F16 && dst_dtype == T_F32)))
        return fail(LLOOM_HIP_EDTYPE, "cast: %s -> %s is not F32 <-> F16", type_name(src_dtype), type_name(dst_dtype));
    if (count < 0) return fail(LLOOM_HIP_EINVAL, "cast: negative count");
    if ((uintptr_t)src_dev % 16 || (uintptr_t)dst_dev % 16) return fail(LLOOM_HIP_EINVAL, "cast: src and dst must be 16-byte aligned");
    if (count == 0) return LLOOM_HIP_OK;
    HIP_OK(hipSetDevice(ctx->device));
    HIP_OK(launch_cast(src_dtype, src_dev, dst_dtype, dst_dev, count, pick_stream(ctx, stream)));
    return LLOOM_HIP_OK;
}

}  // extern "C"

static int moe_impl(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, const void* w2_dev, int64_t n_experts,
                    int64_t n, int64_t k, const float* x_dev, int64_t batch, int64_t in_dim1,
                    const uint32_t* ids_dev, int64_t topk, float* y_dev, float* y2_dev, int mode, int strict,
                    void* stream) {
    if (!ctx || !w_dev || !x_dev || !ids_dev || !y_dev) return fail(LLOOM_HIP_EINVAL, "moe_matmul: null argument");
    if (mode != MOE_ONE && !w2_dev) return fail(LLOOM_HIP_EINVAL, "moe_matmul: null up weight");
    if (mode == MOE_PAIR && !y2_dev) return fail(LLOOM_HIP_EINVAL, "moe_matmul: null up output");
    if (!is_weight_type(ggml_type))
        return fail(LLOOM_HIP_EDTYPE, "moe_matmul: weight dtype %s (%d) is not supported on the HIP quantized path", type_name(ggml_type), ggml_type);
    int be = block_elems(ggml_type);
    if (n_experts <= 0 || n <= 0 || k <= 0 || batch <= 0 || topk <= 0)
        return fail(LLOOM_HIP_EINVAL, "moe_matmul: empty shape");
    if (k % be) return fail(LLOOM_HIP_ESHAPE, "routed matmul k %lld is not divisible by block size %d", (long long)k, be);
    if (in_dim1 != 1 && in_dim1 != topk)
        return fail(LLOOM_HIP_ESHAPE, "indexed_moe_forward: x dim 1 (%lld) must be 1 or topk (%lld)", (long long)in_dim1, (long long)topk);
    if (batch * topk > (1 << 24) || n > INT32_MAX || k > INT32_MAX)
        return fail(LLOOM_HIP_ESHAPE, "moe_matmul: shape too large");
    if (n_experts > MOE_MAX_EXPERTS)
        return fail(LLOOM_HIP_ESHAPE, "moe_matmul: %lld experts, at most %d are routed on the device",
                    (long long)n_experts, MOE_MAX_EXPERTS);
    if ((uintptr_t)w_dev % (ggml_type == T_Q4K ? 16 : 4) || (uintptr_t)x_dev % 16 ||
        (w2_dev && (uintptr_t)w2_dev % (ggml_type == T_Q4K ? 16 : 4)))
        return fail(LLOOM_HIP_EINVAL, "moe_matmul: misaligned weight or x pointer");
    HIP_OK(hipSetDevice(ctx->device));
    hipStream_t s = pick_stream(ctx, stream);
    std::lock_guard<std::mutex> lock(ctx->mu);
    void* ws = nullptr;
    int rc = ensure_ws(ctx, moe_workspace_bytes(n_experts, batch * topk, n, k, mode), s, &ws);
    if (rc) return rc;
    HIP_OK(launch_moe(ggml_type, w_dev, n_experts, n, k, x_dev, batch, in_dim1, ids_dev, topk, y_dev, (int*)ws,
                      ctx->flags, mode, w2_dev, y2_dev, s));
    if (strict) {
        int flag = 0;
        HIP_OK(hipMemcpyAsync(&flag, ws, sizeof(int), hipMemcpyDeviceToHost, s));
        HIP_OK(hipStreamSynchronize(s));
        if (flag) {
            int zero = 0;
            HIP_OK(hipMemcpy(ctx->flags, &zero, sizeof(int), hipMemcpyHostToDevice));
            return fail(LLOOM_HIP_EEXPERT, "expert id is out of range for %lld experts", (long long)n_experts);
        }
    }
    return LLOOM_HIP_OK;
}

extern "C" {

int lloom_hip_moe_matmul(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t n_experts, int64_t n,
                         int64_t k, const float* x_dev, int64_t batch, int64_t in_dim1, const uint32_t* ids_dev,
                         int64_t topk, float* y_dev, int strict, void* stream) {
    return moe_impl(ctx, ggml_type, w_dev, nullptr, n_experts, n, k, x_dev, batch, in_dim1, ids_dev, topk, y_dev,
                    nullptr, MOE_ONE, strict, stream);
}

int lloom_hip_moe_matmul_pair(lloom_hip_ctx* ctx, int ggml_type, const void* w_gate_dev, const void* w_up_dev,
                              int64_t n_experts, int64_t n, int64_t k, const float* x_dev, int64_t batch,
                              int64_t in_dim1, const uint32_t* ids_dev, int64_t topk, float* y_gate_dev,
                              float* y_up_dev, int strict, void* stream) {
    return moe_impl(ctx, ggml_type, w_gate_dev, w_up_dev, n_experts, n, k, x_dev, batch, in_dim1, ids_dev, topk,
                    y_gate_dev, y_up_dev, MOE_PAIR, strict, stream);
}

int lloom_hip_moe_matmul_glu(lloom_hip_ctx* ctx, int ggml_type, const void* w_gate_dev, const void* w_up_dev,
                             int64_t n_experts, int64_t n, int64_t k, const float* x_dev, int64_t batch,
                             int64_t in_dim1, const uint32_t* ids_dev, int64_t topk, float* y_dev, int strict,
                             void* stream) {
    return moe_impl(ctx, ggml_type, w_gate_dev, w_up_dev, n_experts, n, k, x_dev, batch, in_dim1, ids_dev, topk,
                    y_dev, nullptr, MOE_GLU, strict, stream);
}

int lloom_hip_embedding(lloom_hip_ctx* ctx, int ggml_type, const void* w_dev, int64_t rows, int64_t hidden,
                        const uint32_t* ids_dev, int64_t n_ids, void* y_dev, int out_dtype, int strict,
                        void* stream) {
    if (!ctx || !w_dev || (n_ids && (!ids_dev || !y_dev))) return fail(LLOOM_HIP_EINVAL, "embedding: null argument");
    if (!is_weight_type(ggml_type))
        return fail(LLOOM_HIP_EDTYPE, "embedding: %s (%d) is not supported on the HIP quantized path", type_name(ggml_type), ggml_type);
    if (out_dtype != T_F32 && out_dtype != T_F16)
        return fail(LLOOM_HIP_EDTYPE, "embedding: output dtype %s (%d) must be F32 or F16", type_name(out_dtype), out_dtype);
    const int be = block_elems(ggml_type);
    if (rows <= 0 || hidden <= 0 || n_ids < 0) return fail(LLOOM_HIP_EINVAL, "embedding: empty or negative shape");
    if (hidden % be)
        return fail(LLOOM_HIP_ESHAPE, "quantized embedding hidden size %lld is not divisible by block size %d", (long long)hidden, be);
    if ((uintptr_t)w_dev % 4) return fail(LLOOM_HIP_EINVAL, "embedding: weight must be 4-byte aligned");
    if (n_ids == 0) return LLOOM_HIP_OK;
    HIP_OK(hipSetDevice(ctx->device));
    hipStream_t s = pick_stream(ctx, stream);
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (strict) HIP_OK(hipMemsetAsync(ctx->flags + 1, 0, sizeof(int), s));
    HIP_OK(launch_embedding(ggml_type, w_dev, rows, hidden, ids_dev, n_ids, y_dev, out_dtype, ctx->flags, s));
    if (strict) {
        int flag = 0;
        HIP_OK(hipMemcpyAsync(&flag, ctx->flags + 1, sizeof(int), hipMemcpyDeviceToHost, s));
        HIP_OK(hipStreamSynchronize(s));
        if (flag) {
            int zero = 0;
            HIP_OK(hipMemcpy(ctx->flags, &zero, sizeof(int), hipMemcpyHostToDevice));
            return fail(LLOOM_HIP_EEXPERT, "embedding id is out of range for %lld rows", (long long)rows);
        }
    }
    return LLOOM_HIP_OK;
}

}  // extern "C"
