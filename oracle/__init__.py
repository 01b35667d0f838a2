"""ctypes front of the CPU oracle (TEST INFRASTRUCTURE).

The oracle restates lloom-tensor's CPU arithmetic for the quantized matmul
path (``lloom-tensor/src/quantized/k_quants.rs``, ``utils.rs``,
``mod.rs:766-810``) in plain C, see ``kq_oracle.c``.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this package: it is the checker, never the thing measured or shipped.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))

F32, F16, Q8_0, Q4K, Q6K, Q8K = 0, 1, 8, 12, 14, 15
BLOCK_BYTES = {Q8_0: 34, Q4K: 144, Q6K: 210, Q8K: 292}
BLOCK_ELEMS = {Q8_0: 32, Q4K: 256, Q6K: 256, Q8K: 256}
VEC_DOT_TYPE = {Q8_0: Q8_0, Q4K: Q8K, Q6K: Q8K, Q8K: Q8K}

_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(_HERE, "libkq_oracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle not built: {path} (run __graft_entry__.build())")
        L = ctypes.CDLL(path)
        vp, sz, fp = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_quantize.argtypes = [ctypes.c_int, fp, sz, vp]
        L.orc_dequantize.argtypes = [ctypes.c_int, vp, sz, fp]
        L.orc_dequantize_f16.argtypes = [ctypes.c_int, vp, sz, vp]
        L.orc_vec_dot_unopt.restype = ctypes.c_float
        L.orc_vec_dot_unopt.argtypes = [ctypes.c_int, sz, vp, vp]
        L.orc_matmul.argtypes = [ctypes.c_int, sz, sz, sz, fp, vp, fp]
        L.orc_matmul_indexed.argtypes = [ctypes.c_int, vp, sz, sz, sz, fp, sz, vp, sz, sz, fp]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def quantize(dtype, x):
    """from_float of a flat f32 array -> uint8 bytes of the blocks."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    be = BLOCK_ELEMS[dtype]
    assert x.size % be == 0
    out = np.zeros(x.size // be * BLOCK_BYTES[dtype], dtype=np.uint8)
    assert lib().orc_quantize(dtype, _p(x), x.size, _p(out)) == 0
    return out


def dequantize(dtype, blocks, n):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty(n, dtype=np.float32)
    assert lib().orc_dequantize(dtype, _p(blocks), n, _p(y)) == 0
    return y


def dequantize_f16(dtype, blocks, n):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty(n, dtype=np.uint16)
    assert lib().orc_dequantize_f16(dtype, _p(blocks), n, _p(y)) == 0
    return y.view(np.float16)


def vec_dot_unopt(dtype, n, w_blocks, a_blocks):
    return lib().orc_vec_dot_unopt(dtype, n, _p(np.ascontiguousarray(w_blocks)),
                                   _p(np.ascontiguousarray(a_blocks)))


def matmul(dtype, x, w_blocks, n):
    """k_quants::matmul: x [m, k] f32, w [n, k] blocks -> [m, n] f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    dst = np.empty((m, n), dtype=np.float32)
    w_blocks = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    assert lib().orc_matmul(dtype, m, k, n, _p(x), _p(w_blocks), _p(dst)) == 0
    return dst


def matmul_indexed(dtype, w_blocks, n_experts, n, k, x, ids):
    """matmul_t_indexed: x [batch, in_dim1, k], ids [batch, topk] -> [batch, topk, n]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    batch, in_dim1, kk = x.shape
    assert kk == k
    topk = ids.shape[1]
    dst = np.empty((batch, topk, n), dtype=np.float32)
    rc = lib().orc_matmul_indexed(dtype, _p(np.ascontiguousarray(w_blocks, dtype=np.uint8)),
                                  n_experts, n, k, _p(x), in_dim1, _p(ids), batch, topk, _p(dst))
    if rc != 0:
        raise ValueError("matmul_indexed refused its inputs")
    return dst


def f32_to_f16_bits(f):
    return lib().orc_f32_to_f16(float(f))


def f16_bits_to_f32(h):
    return lib().orc_f16_to_f32(int(h))
