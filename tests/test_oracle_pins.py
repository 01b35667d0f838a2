"""Pins of the CPU oracle against what the reference's own tests fix.

Every check here is one that a plausible mistake in the restatement (a dropped
term, a wrong index or sign, a wrong rounding rule) fails.  Sources:
lloom-tensor/tests/quantized_tests.rs (line numbers below).
"""
import numpy as np
import pytest

import oracle as O
from tests.stdrng import StdRng

GGML_TEST_SIZE = 32 * 128  # quantized_tests.rs:12
GGML_MAX_QUANTIZATION_TOTAL_ERROR = 0.002  # :14
GGML_MAX_DOT_PRODUCT_ERROR = 0.02  # :17
# ggml_reference_matmul_error (:1117-1153)
GGML_REF_ERR = {O.Q4K: 0.002425, O.Q6K: 0.000952, O.Q8_0: 0.000092, O.Q8K: 0.00065}


def get_test_vector2(bound, size):  # :492-505
    v = (np.arange(size, dtype=np.float32) - np.float32(size / 2)) * np.float32(bound) / np.float32(size / 2)
    assert v[0] == -bound and v[size // 2] == 0.0
    return v.astype(np.float32)


def create_ggml_like_vector(offset):  # :527-532
    i = np.arange(GGML_TEST_SIZE, dtype=np.float32)
    return (np.float32(0.1) + np.float32(2.0) * np.cos(i + np.float32(offset))).astype(np.float32)


def rmse(a, b):  # :535-544 (sqrt of the sum, divided by the length)
    return float(np.sqrt(np.sum((a.astype(np.float32) - b.astype(np.float32)) ** 2, dtype=np.float32))) / len(a)


def round3(v):
    return [round(float(x) * 1000.0) / 1000.0 for x in v]


# ---------------------------------------------------------------- f16 ---

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_bits_to_f32(b) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10) ** rng.integers(-9, 6, 20000).astype(np.float32),
        # exact ties between two f16 values, subnormal range, overflow edge
        (np.arange(1, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24),
        np.array([65504.0, 65519.0, 65520.0, 1e9, -0.0, 0.0, 2.0 ** -25, 2.0 ** -26, 3 * 2.0 ** -26], dtype=np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16_bits(v) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


# ----------------------------------------------- quantize / dequantize ---

LITERAL = {  # quantized_tests.rs:880-888, :974-982, :1021-1029
    O.Q4K: ([-0.5, -0.373, -0.25, 0.0, 0.288, 0.498], 0.017, 4.5),
    O.Q6K: ([-0.497, -0.372, -0.25, -0.0, 0.284, 0.5], 0.008, 2.0),
    O.Q8K: ([-0.5, -0.374, -0.25, -0.0, 0.283, 0.499], 0.008, 0.6),
}


@pytest.mark.parametrize("dtype", [O.Q4K, O.Q6K, O.Q8K])
def test_quantize_kquant_literals(dtype):
    lit, tol, tol_big = LITERAL[dtype]
    src = get_test_vector2(0.5, 1024)
    q = O.quantize(dtype, src)
    dst = O.dequantize(dtype, q, 1024)
    # dequantize_f16 == f16(dequantize) exactly (:867-873)
    assert np.array_equal(O.dequantize_f16(dtype, q, 1024).view(np.uint16),
                          dst.astype(np.float16).view(np.uint16))
    assert np.all(np.abs(dst - src) < tol)
    idx = [0, 128, 256, 512, 800, 1023]
    assert np.array_equal(src[idx], np.array([-0.5, -0.375, -0.25, 0.0, 0.28125, 0.49902344], np.float32))
    assert round3(dst[idx]) == lit
    big = get_test_vector2(128.0, 1024)
    dbig = O.dequantize(dtype, O.quantize(dtype, big), 1024)
    assert np.all(np.abs(dbig - big) < tol_big)
    g = create_ggml_like_vector(0.0)
    assert rmse(g, O.dequantize(dtype, O.quantize(dtype, g), g.size)) <= GGML_MAX_QUANTIZATION_TOTAL_ERROR


def test_q8_0_closed_form():
    """BlockQ8_0::from_float is textbook absmax int8: d = amax/127 (stored f16),
    q = round_half_away(x * (1/d)) with the f32 d, not the f16 one (:738-767)."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(32 * 64) * 3).astype(np.float32)
    x[:32] = 0.0  # all-zero block: d = 0, id = 0, q = 0
    q = O.quantize(O.Q8_0, x).reshape(-1, 34)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1).astype(np.float32)
    d = (amax / np.float32(127)).astype(np.float32)
    idd = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
    prod = (xb * idd[:, None]).astype(np.float32)
    qq = (np.sign(prod) * np.floor(np.abs(prod) + np.float32(0.5))).astype(np.int8)
    assert np.array_equal(q[:, :2].copy().view(np.uint16).ravel(), d.astype(np.float16).view(np.uint16))
    assert np.array_equal(q[:, 2:].view(np.int8), qq)
    g = create_ggml_like_vector(0.0)
    assert rmse(g, O.dequantize(O.Q8_0, O.quantize(O.Q8_0, g), g.size)) <= GGML_MAX_QUANTIZATION_TOTAL_ERROR


def test_q8k_sign_of_max_and_bsums():
    """BlockQ8K::from_float: iscale = -127/max with max the signed value of the
    largest |x| (first wins on ties), bsums are 16-element sums (:2400-2438)."""
    x = np.zeros(512, dtype=np.float32)
    x[3], x[7] = -2.0, 2.0  # tie on |x|: the first (-2) is max -> iscale = +63.5
    x[10] = 1.0
    x[256:] = 0.0  # all-zero block
    q = O.quantize(O.Q8K, x).reshape(2, 292)
    d0 = q[0, :4].copy().view(np.float32)[0]
    qs0 = q[0, 4:260].view(np.int8)
    bs0 = q[0, 260:292].copy().view(np.int16)
    assert d0 == np.float32(1.0) / (np.float32(-127.0) / np.float32(-2.0))
    assert qs0[3] == -127 and qs0[7] == 127 and qs0[10] == 64  # round(63.5) = 64 (half away)
    assert np.array_equal(bs0, qs0.astype(np.int32).reshape(16, 16).sum(1).astype(np.int16))
    assert q[1, :4].copy().view(np.float32)[0] == 0.0 and not q[1, 4:].any()


# ------------------------------------------------------------ vec_dot ---

def _ggml_matmul_error(dtype, a, b, err_m):  # :1183-1222
    n = a.size
    aq = O.quantize(dtype, a)
    bq = O.quantize(O.VEC_DOT_TYPE[dtype], b)
    unopt = O.vec_dot_unopt(dtype, n, aq, bq)
    mm = O.matmul(dtype, b.reshape(1, n), aq, 1)[0, 0]
    assert abs(mm - unopt) / n <= 1e-6
    ref = np.float32(0)
    for x, y in zip(a, b):  # vec_dot_reference: sequential f32 sum
        ref = np.float32(ref + np.float32(x * y))
    err = abs(float(unopt) - float(ref)) / n
    assert np.isfinite(err) and err <= GGML_MAX_DOT_PRODUCT_ERROR
    assert err - 0.00001 <= GGML_REF_ERR[dtype] * err_m
    return unopt


@pytest.mark.parametrize("dtype", [O.Q8_0, O.Q4K, O.Q6K, O.Q8K])
def test_ggml_matmul_error(dtype):
    _ggml_matmul_error(dtype, create_ggml_like_vector(0.0), create_ggml_like_vector(1.0), 1.0)
    ramp = (np.arange(GGML_TEST_SIZE, dtype=np.float32) / np.float32(GGML_TEST_SIZE)).astype(np.float32)
    _ggml_matmul_error(dtype, ramp, ramp.copy(), 2.0)


@pytest.mark.parametrize("dtype", [O.Q8_0, O.Q4K, O.Q6K, O.Q8K])
def test_vec_dot_equals_f64_dot_of_dequantized(dtype):
    """The integer inner sums are exact, so vec_dot_unopt equals the f64 dot
    of the dequantized operands up to f32 rounding of the outer sums.  A
    dropped min term, scale or wrong nibble index fails by orders of magnitude."""
    rng = np.random.default_rng(7)
    k = 2048
    for trial in range(4):
        w = (rng.standard_normal(k) * 0.02).astype(np.float32)
        x = rng.standard_normal(k).astype(np.float32)
        wq = O.quantize(dtype, w)
        vt = O.VEC_DOT_TYPE[dtype]
        xq = O.quantize(vt, x)
        wd = O.dequantize(dtype, wq, k).astype(np.float64)
        xd = O.dequantize(vt, xq, k).astype(np.float64)
        ref = float(wd @ xd)
        got = O.vec_dot_unopt(dtype, k, wq, xq)
        scale = float(np.abs(wd * xd).sum())
        assert abs(got - ref) <= 2e-6 * scale, (trial, got, ref)


# ------------------------------------------------------------- matmul ---

@pytest.mark.parametrize("dtype", [O.Q8_0, O.Q4K, O.Q6K])
def test_prompt_gemm_bit_identical_to_decode_rows(dtype):
    """:1769-1903 on its closed-form inputs, plus the scalar f64 oracle <= 0.02."""
    for m in [2, 17]:
        for n in [1, 3, 4, 7]:
            for k in [256, 768]:
                lhs = ((np.arange(m * k) * 17 % 211).astype(np.float32) - np.float32(103)) / np.float32(73)
                wts = ((np.arange(n * k) * 31 % 173).astype(np.float32) - np.float32(87)) / np.float32(61)
                lhs = lhs.astype(np.float32).reshape(m, k)
                rhs = O.quantize(dtype, wts.astype(np.float32))
                got = O.matmul(dtype, lhs, rhs, n)
                rows = np.concatenate([O.matmul(dtype, lhs[r:r + 1], rhs, n) for r in range(m)])
                assert np.array_equal(got.view(np.uint32), rows.view(np.uint32))
                dense = O.dequantize(dtype, rhs, n * k).reshape(n, k).astype(np.float64)
                vt = O.VEC_DOT_TYPE[dtype]
                for r in range(m):
                    xd = O.dequantize(vt, O.quantize(vt, lhs[r]), k).astype(np.float64)
                    ref = dense @ xd
                    err = np.abs(got[r] - ref) / np.maximum(np.abs(ref), 1.0)
                    assert np.all(err <= GGML_MAX_DOT_PRODUCT_ERROR)


def _stdrng_tensors(m, k, n):  # get_random_tensors, :1267-1287
    rng = StdRng(314159265358979)
    lhs = (rng.random_f32(m * k) - np.float32(0.5)).astype(np.float32).reshape(m, k)
    rhs = (rng.random_f32(n * k) - np.float32(0.5)).astype(np.float32).reshape(n, k)
    return lhs, rhs


@pytest.fixture(scope="module")
def stdrng_11_512_21():
    return _stdrng_tensors(11, 512, 21)


def _pick(v, m, n):
    f = v.ravel()
    return round3([f[0], f[m * n // 3], f[m * n * 2 // 3], f[m * n - 1]])


def test_stdrng_restatement_matches_reference_f32_matmul(stdrng_11_512_21):
    """The literal f32 matmul values of quantized_matmul_q4k/q6k/q8k (:1451)
    pin the ChaCha12/PCG32 restatement that the next test relies on."""
    lhs, rhs = stdrng_11_512_21
    mm = lhs.astype(np.float64) @ rhs.astype(np.float64).T
    assert _pick(mm, 11, 21) == [1.262, 1.513, -0.208, 1.702]


@pytest.mark.parametrize("dtype,want", [
    (O.Q4K, [1.094, 1.442, -0.196, 1.587]),  # :1460
    (O.Q6K, [1.293, 1.497, -0.159, 1.737]),  # :1514
    (O.Q8K, [1.241, 1.52, -0.2, 1.7]),
])
def test_quantized_matmul_known_answers(stdrng_11_512_21, dtype, want):
    lhs, rhs = stdrng_11_512_21
    q = O.quantize(dtype, rhs.ravel())
    got = O.matmul(dtype, lhs, q, 21)
    assert _pick(got, 11, 21) == want


# ------------------------------------------------------------ indexed ---

def test_matmul_indexed_closed_form_and_refusals():
    rng = np.random.default_rng(3)
    E, n, k, batch, topk = 4, 5, 256, 3, 2
    w = (rng.standard_normal((E, n, k)) * 0.1).astype(np.float32)
    wq = O.quantize(O.Q4K, w.ravel())
    dense = O.dequantize(O.Q4K, wq, E * n * k).reshape(E, n, k)
    ids = np.array([[1, 1], [0, 3], [2, 1]], dtype=np.uint32)
    for in_dim1 in (1, topk):
        x = rng.standard_normal((batch, in_dim1, k)).astype(np.float32)
        got = O.matmul_indexed(O.Q4K, wq, E, n, k, x, ids)
        for b in range(batch):
            for t in range(topk):
                xr = x[b, 0 if in_dim1 == 1 else t].astype(np.float64)
                ref = dense[ids[b, t]].astype(np.float64) @ xr
                assert np.allclose(got[b, t], ref, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        O.matmul_indexed(O.Q4K, wq, E, n, k, np.zeros((batch, 1, k), np.float32),
                         np.array([[0, 4], [0, 0], [0, 0]], dtype=np.uint32))
