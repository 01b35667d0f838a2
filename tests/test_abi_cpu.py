"""CPU-side checks: the C-ABI library loads and exports every function
include/lloom_hip.h declares, the host-only entry points behave, and the
CPU-baseline restatement agrees with the oracle (no GPU needed)."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "lloom_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lloom_hip_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import lloom_amd

    L = lloom_amd.lib()
    names = declared_functions()
    assert len(names) >= 19
    for name in names:
        assert hasattr(L, name), name
    assert L.lloom_hip_version().startswith(b"lloom-hip")


def test_weight_bytes_and_refusals():
    import lloom_amd
    from lloom_amd.lib import lib

    packed, alloc = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib().lloom_hip_weight_bytes(12, 6144, 2048, ctypes.byref(packed), ctypes.byref(alloc)) == 0
    assert packed.value == 7077888 and alloc.value > packed.value  # W [6144, 2048] Q4_K: 6144 rows x 8 superblocks x 144 B
    assert lib().lloom_hip_weight_bytes(8, 8192, 2048, ctypes.byref(packed), ctypes.byref(alloc)) == 0
    assert packed.value == 17825792
    assert lib().lloom_hip_weight_bytes(14, 2048, 8192, ctypes.byref(packed), ctypes.byref(alloc)) == 0
    assert packed.value == 13762560
    assert lib().lloom_hip_weight_bytes(12, 4, 100, ctypes.byref(packed), ctypes.byref(alloc)) == 3
    assert b"divisible" in lib().lloom_hip_last_error()
    assert lib().lloom_hip_weight_bytes(99, 4, 256, ctypes.byref(packed), ctypes.byref(alloc)) == 2
    assert isinstance(lloom_amd.LloomHipError(3, "x"), RuntimeError)


def test_synth_is_deterministic_and_normal():
    import lloom_amd as L

    a = L.synth_normal(42, 1 << 18)
    b = L.synth_normal(42, 1 << 18)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    assert not np.array_equal(a, L.synth_normal(43, 1 << 18))
    # a prefix is independent of the total count (chunked streams)
    assert np.array_equal(L.synth_normal(42, 1000), a[:1000])
    u = L.synth_uniform(1, 100000, 0.0, 1.0)
    assert u.min() >= 0.0 and u.max() < 1.0 and abs(u.mean() - 0.5) < 0.01


@pytest.fixture(scope="module")
def cpb():
    path = os.path.join(ROOT, "oracle", "libkq_cpubase.so")
    if not os.path.exists(path):
        pytest.skip("cpu baseline not built")
    lib = ctypes.CDLL(path)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    lib.cpb_vec_dot.restype = ctypes.c_float
    lib.cpb_vec_dot.argtypes = [ctypes.c_int, sz, vp, vp]
    lib.cpb_matmul.argtypes = [ctypes.c_int, sz, sz, sz, vp, vp, vp]
    lib.cpb_pool_init.argtypes = [ctypes.c_int]
    lib.cpb_pool_init(4)
    return lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
def test_cpu_baseline_avx_matches_unopt(cpb, dt):
    """|opt - unopt| / len <= 1e-6 (quantized_tests.rs:1183)."""
    rng = np.random.default_rng(dt)
    for k in (256, 2048, 4096):
        w = (rng.standard_normal(k) * 0.5).astype(np.float32)
        x = rng.standard_normal(k).astype(np.float32)
        wq = O.quantize(dt, w)
        xq = O.quantize(O.VEC_DOT_TYPE[dt], x)
        opt = cpb.cpb_vec_dot(dt, k, _p(wq), _p(xq))
        unopt = O.vec_dot_unopt(dt, k, wq, xq)
        assert abs(opt - unopt) / k <= 1e-6


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
def test_cpu_baseline_gemm_equals_decode_rows(cpb, dt):
    """Prompt GEMM rows are bit-identical to per-row decode (:1769-1903)."""
    rng = np.random.default_rng(1)
    m, n, k = 17, 65, 768
    w = O.quantize(dt, (rng.standard_normal(n * k) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    full = np.empty((m, n), np.float32)
    assert cpb.cpb_matmul(dt, m, k, n, _p(x), _p(w), _p(full)) == 0
    for r in range(m):
        row = np.empty((1, n), np.float32)
        xr = np.ascontiguousarray(x[r:r + 1])
        assert cpb.cpb_matmul(dt, 1, k, n, _p(xr), _p(w), _p(row)) == 0
        assert np.array_equal(row[0].view(np.uint32), full[r].view(np.uint32))
    ref = O.matmul(dt, x, w, n)
    assert np.all(np.abs(full - ref) <= 1e-5 * np.abs(ref).max() + 1e-6)
