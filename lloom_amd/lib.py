"""ctypes binding of liblloom_hip.so (the C ABI of include/lloom_hip.h)."""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
_lock = threading.Lock()
_lib = None

ERRORS = {
    1: "EINVAL", 2: "EDTYPE", 3: "ESHAPE", 4: "EEXPERT", 5: "EHIP", 6: "ENOMEM", 7: "EDEVICE",
}


class LloomHipError(RuntimeError):
    """A refused call: ``code`` is the LLOOM_HIP_E* value, the message names the cause."""

    def __init__(self, code, msg):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code
        self.name = ERRORS.get(code, str(code))


def lib_path():
    return os.path.join(_HERE, "liblloom_hip.so")


def lib():
    """The loaded library.  Raises if it has not been built (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not os.path.exists(path):
                raise RuntimeError(
                    f"{path} is missing: build it with __graft_entry__.build() "
                    "(there is no CPU fallback for the quantized HIP path)")
            L = ctypes.CDLL(path)
            vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
            sigs = {
                "lloom_hip_last_error": ([], ctypes.c_char_p),
                "lloom_hip_version": ([], ctypes.c_char_p),
                "lloom_hip_ctx_create": ([i32, ctypes.POINTER(vp)], i32),
                "lloom_hip_ctx_destroy": ([vp], i32),
                "lloom_hip_ctx_stream": ([vp], vp),
                "lloom_hip_ctx_set_mv_rows_max": ([vp, i32], i32),
                "lloom_hip_ctx_sync": ([vp], i32),
                "lloom_hip_ctx_set_prefill_mma": ([vp, i32], i32),
                "lloom_hip_alloc": ([vp, sz, ctypes.POINTER(vp)], i32),
                "lloom_hip_free": ([vp, vp], i32),
                "lloom_hip_memcpy_h2d": ([vp, vp, vp, sz, vp], i32),
                "lloom_hip_memcpy_d2h": ([vp, vp, vp, sz, vp], i32),
                "lloom_hip_weight_bytes": ([i32, i64, i64, ctypes.POINTER(sz), ctypes.POINTER(sz)], i32),
                "lloom_hip_quantize": ([vp, i32, vp, i64, vp, vp], i32),
                "lloom_hip_quantize_act": ([vp, i32, vp, i64, i64, vp, vp], i32),
                "lloom_hip_dequantize": ([vp, i32, vp, i64, vp, i32, vp], i32),
                "lloom_hip_qmatmul": ([vp, i32, vp, i64, i64, vp, i32, i64, vp, i32, vp], i32),
                "lloom_hip_qmatmul_store": ([vp, i32, vp, i64, i64, vp, i32, i64, vp, i32, i32, vp], i32),
                "lloom_hip_qmatmul_workspace_bytes": ([vp, i32, i64, i64, i64, i32, i32, ctypes.POINTER(sz)], i32),
                "lloom_hip_ctx_reserve": ([vp, sz], i32),
                "lloom_hip_ctx_workspace_bytes": ([vp, ctypes.POINTER(sz)], i32),
                "lloom_hip_cast": ([vp, vp, i32, vp, i32, i64, vp], i32),
                "lloom_hip_qmatmul_noalloc": ([vp, i32, vp, i64, i64, vp, i32, i64, vp, i32, vp], i32),
                "lloom_hip_moe_matmul": ([vp, i32, vp, i64, i64, i64, vp, i64, i64, vp, i64, vp, i32, vp], i32),
                "lloom_hip_moe_matmul_pair": ([vp, i32, vp, vp, i64, i64, i64, vp, i64, i64, vp, i64, vp, vp, i32,
                                               vp], i32),
                "lloom_hip_moe_matmul_glu": ([vp, i32, vp, vp, i64, i64, i64, vp, i64, i64, vp, i64, vp, i32, vp],
                                             i32),
                "lloom_hip_embedding": ([vp, i32, vp, i64, i64, vp, i64, vp, i32, i32, vp], i32),
                "lloom_hip_synth_normal": ([ctypes.c_uint64, ctypes.c_float, ctypes.c_float, vp, i64], i32),
                "lloom_hip_synth_uniform": ([ctypes.c_uint64, ctypes.c_float, ctypes.c_float, vp, i64], i32),
            }
            for name, (args, res) in sigs.items():
                f = getattr(L, name)
                f.argtypes = args
                f.restype = res
            _lib = L
    return _lib


def check(rc):
    if rc != 0:
        msg = lib().lloom_hip_last_error().decode(errors="replace")
        raise LloomHipError(rc, msg)
