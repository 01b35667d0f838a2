"""GPU parity of the HIP path (through the C ABI) against the CPU oracle.

Bars: quantizers and dequantizers bit-exact; matmul max|d| <= 1e-3 * max|y row|
(the tolerance BASELINE.json's north_star states); routed experts also mean
relative error < 1e-4 against a dense f32 reference
(lloom-tensor/tests/moe_routed_metal.rs:148-154, 244-327).
"""
import os

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

MATMUL_TOL = 1e-3  # max|got - want| <= MATMUL_TOL * max|want row|


@pytest.fixture(scope="module")
def L():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lloom_amd

    lloom_amd.lib()
    return lloom_amd


DEV = "cuda:0"


def _cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def assert_rows_close(got, want, tol=MATMUL_TOL, what=""):
    got = np.asarray(got, dtype=np.float64).reshape(-1, want.shape[-1])
    want = np.asarray(want, dtype=np.float64).reshape(-1, want.shape[-1])
    bound = tol * np.abs(want).max(axis=1, keepdims=True) + 1e-30
    err = np.abs(got - want)
    bad = err > bound
    assert not bad.any(), f"{what}: {bad.sum()} outputs out of tolerance, worst ratio {(err / bound).max():.3g}"


def ggml_like(n, offset=0.0):
    i = np.arange(n, dtype=np.float32)
    return (np.float32(0.1) + np.float32(2.0) * np.cos(i + np.float32(offset))).astype(np.float32)


def edge_inputs(k, rows=4, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[0, :256] = 0.0  # an all-zero block
    x[1, :32] = 7.25  # constant block
    x[1, 40] = -3.0   # tie on |x| with a later +3.0
    x[1, 41] = 3.0
    x[2] *= np.float32(1e-38)  # subnormal range
    x[3, ::7] *= 1000.0  # outliers
    return x


# ------------------------------------------------------------ quantize ---

@pytest.mark.parametrize("vt", [O.Q8_0, O.Q8K])
def test_quantize_act_bit_exact(L, vt):
    for x in [edge_inputs(1024), L.synth_normal(5, 9 * 2048).reshape(9, 2048)]:
        got = L.quantize_act(_cuda(x), vt).cpu().numpy()
        want = np.concatenate([O.quantize(vt, r) for r in x])
        assert np.array_equal(got, want)


def test_quantize_act_q8k_max_at_every_position(L):
    """The block max is a cross-lane reduction: put it at each of the 256
    positions (and a tie after it) and check the exact bytes."""
    x = np.full((256, 256), 0.5, np.float32)
    for i in range(256):
        x[i, i] = -3.0
        x[i, (i + 97) % 256] = 3.0  # same |x|: the first index must win
    got = L.quantize_act(_cuda(x), O.Q8K).cpu().numpy()
    assert np.array_equal(got, np.concatenate([O.quantize(O.Q8K, r) for r in x]))


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
def test_weight_quantize_bit_exact(L, dt):
    cases = [
        L.synth_normal(7, 64 * 2048, 0.0, 0.02).reshape(64, 2048),
        ggml_like(4096).reshape(2, 2048),
        (np.arange(1024, dtype=np.float32) - 512.0).reshape(1, 1024) * np.float32(0.5 / 512),
        edge_inputs(1024, seed=1),
        np.zeros((1, 512), np.float32),
        np.full((1, 256), 0.375, np.float32),
    ]
    for w in cases:
        qt = L.QTensor.quantize(_cuda(w), dt)
        got = qt.data()
        want = O.quantize(dt, w.ravel())
        assert np.array_equal(got, want), f"{dt}: {np.sum(got != want)} bytes differ for shape {w.shape}"


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K, O.Q8K])
def test_dequantize_bit_exact(L, dt):
    w = L.synth_normal(9, 16 * 1024, 0.0, 0.5).astype(np.float32)
    q = O.quantize(dt, w)
    blocks = _cuda(np.concatenate([q, np.zeros(512, np.uint8)]))
    got = L.dequantize(blocks, dt, w.size).cpu().numpy()
    want = O.dequantize(dt, q, w.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = L.dequantize(blocks, dt, w.size, out_f16=True).cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), O.dequantize_f16(dt, q, w.size).view(np.uint16))


def test_qtensor_dequantize_f16_is_rne_of_f32(L):
    """dequantize_f16 == f16(dequantize) exactly (quantized_tests.rs:867-873)."""
    w = _cuda(ggml_like(4096).reshape(16, 256))
    for dt in (L.GgmlDType.Q4K, L.GgmlDType.Q6K, L.GgmlDType.Q8_0):
        qt = L.QTensor.quantize(w, dt)
        a = qt.dequantize().half().cpu().numpy().view(np.uint16)
        b = qt.dequantize_f16().cpu().numpy().view(np.uint16)
        assert np.array_equal(a, b)


# -------------------------------------------------------------- matmul ---

def _qmm(L, dt, w, x):
    qt = L.QTensor.quantize(_cuda(w), dt)
    y = L.QMatMul.from_qtensor(qt).forward(_cuda(x)).cpu().numpy()
    return y, qt.data()


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 7, 8, 13, 16, 17, 33])
def test_qmatmul_matches_oracle(L, dt, m):
    rng = np.random.default_rng(100 + m)
    for n, k in [(1, 256), (7, 768), (65, 2048), (130, 512)]:
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        x = rng.standard_normal((m, k)).astype(np.float32)
        y, q = _qmm(L, dt, w, x)
        assert_rows_close(y, O.matmul(dt, x, q, n), what=f"dt={dt} m={m} n={n} k={k}")


GEMM_SHAPES = [(17, 1, 256), (64, 128, 2048), (100, 7, 768), (128, 300, 512), (96, 200, 2048), (129, 40, 2048),
               (64, 8200, 512), (128, 8200, 256), (200, 129, 1024), (1030, 130, 512), (257, 64, 256),
               (512, 256, 2048), (129, 520, 768), (256, 1000, 2048),
               # int8 planes: more than 128 workgroups of 128 x 256, so the
               # 256-column tiling (the shapes above take the 128-column one)
               (520, 8200, 512), (1100, 4100, 256)]


@pytest.mark.parametrize("m,n,k,mma", [s + (mma,) for s in GEMM_SHAPES for mma in ("f16", "int8")])
def test_prefill_gemm_q4k_shapes(L, m, n, k, mma):
    """Both prefill GEMMs (exact fp16 operands, the default, and int8 scale
    planes) on ragged tiles (m, n not multiples of the tile)."""
    from lloom_amd.quantized import MMA_AUTO, MMA_F16, MMA_INT8, set_prefill_mma

    rng = np.random.default_rng(m * 7 + n)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1, :256] = 0.0  # an all-zero activation block (d = 0, S = 0)
    set_prefill_mma(MMA_INT8 if mma == "int8" else MMA_F16)
    try:
        y, q = _qmm(L, O.Q4K, w, x)
    finally:
        set_prefill_mma(MMA_AUTO)
    assert_rows_close(y, O.matmul(O.Q4K, x, q, n), what=f"gemm {mma} m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [17, 24, 32, 33, 48, 49, 64, 65, 96, 100, 128])
@pytest.mark.parametrize("n,k", [(6152, 2048), (1000, 1280), (40, 256)])
def test_prefill_q4k_few_rows(L, m, n, k):
    """Q4_K with 17..128 activation rows and k <= 2048 (the DMA kernel with
    two to eight 16-row activation tiles): two- and one-tile workgroups,
    ragged n and m, 8, 5 and 1 superblocks, an all-zero activation block."""
    rng = np.random.default_rng(m * 31 + n + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[m - 1, :256] = 0.0
    x[0, 5] = 40.0  # an outlier: its block's scale differs from the rest
    y, q = _qmm(L, O.Q4K, w, x)
    assert_rows_close(y, O.matmul(O.Q4K, x, q, n), what=f"few rows m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [17, 40, 64])
@pytest.mark.parametrize("mma", ["f16", "int8"])
def test_prefill_q4k_few_rows_long_k(L, m, mma):
    """Q4_K with 17..64 rows past k = 2048 keeps the earlier routes: the
    skinny fp16 kernel, or with int8 planes selected the MFMA decode kernel
    with four activation tiles."""
    from lloom_amd.quantized import MMA_AUTO, MMA_F16, MMA_INT8, set_prefill_mma

    n, k = 72, 4608
    rng = np.random.default_rng(m + 7 * k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    set_prefill_mma(MMA_INT8 if mma == "int8" else MMA_F16)
    try:
        y, q = _qmm(L, O.Q4K, w, x)
    finally:
        set_prefill_mma(MMA_AUTO)
    assert_rows_close(y, O.matmul(O.Q4K, x, q, n), what=f"few rows long k {mma} m={m}")


def _same_sign_inputs(kind, m, k, rng):
    """Activations whose Q8_K sub-block sums reach the top of their range
    (|S_j| up to 32 * 127 = 4064, past the integers fp16 holds exactly)."""
    if kind == "bias":
        return (1.0 + 0.05 * rng.standard_normal((m, k))).astype(np.float32)
    if kind == "negbias":
        return (-1.0 + 0.05 * rng.standard_normal((m, k))).astype(np.float32)
    if kind == "ones":
        return np.ones((m, k), np.float32)
    # one huge outlier per 256-element block over a positive background
    x = (0.5 + 0.1 * rng.random((m, k))).astype(np.float32)
    x[:, 17::256] = 900.0
    x[:, 200::256] = -1000.0
    return x


@pytest.mark.parametrize("dt,mma", [(O.Q4K, "f16"), (O.Q4K, "int8"), (O.Q4K, "auto"), (O.Q8_0, "auto"),
                                    (O.Q6K, "auto")])
@pytest.mark.parametrize("m", [17, 128, 600, 2048])
@pytest.mark.parametrize("kind", ["bias", "negbias", "ones", "outlier"])
def test_prefill_same_sign_activations(L, dt, mma, m, kind):
    """Every prefill route on activations whose sub-block sums are large and
    odd (a positive or negative bias), constant, or dominated by an outlier
    per block, against the oracle.  Zero-mean inputs never push the Q8_K
    sums past 2048, where an fp16 copy of them would round."""
    from lloom_amd.quantized import MMA_AUTO, MMA_F16, MMA_INT8, set_prefill_mma

    n, k = (72 if m >= 600 else 200), 2048
    rng = np.random.default_rng(m * 13 + len(kind))
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = _same_sign_inputs(kind, m, k, rng)
    set_prefill_mma({"f16": MMA_F16, "int8": MMA_INT8, "auto": MMA_AUTO}[mma])
    try:
        y, q = _qmm(L, dt, w, x)
    finally:
        set_prefill_mma(MMA_AUTO)
    assert_rows_close(y, O.matmul(dt, x, q, n), what=f"same-sign {kind} dt={dt} {mma} m={m}")


@pytest.mark.parametrize("kind", ["bias", "negbias", "ones", "outlier"])
def test_prefill_int8_wide_tiles_same_sign(L, kind):
    """The int8 planes' 256-column tiling (more than 128 workgroups of
    128 x 256; the shapes above take the 128-column one) on the same
    large-sum activations, ragged in m and n."""
    from lloom_amd.quantized import MMA_AUTO, MMA_INT8, set_prefill_mma

    m, n, k = 1100, 4100, 256
    rng = np.random.default_rng(len(kind) + 5)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = _same_sign_inputs(kind, m, k, rng)
    set_prefill_mma(MMA_INT8)
    try:
        y, q = _qmm(L, O.Q4K, w, x)
    finally:
        set_prefill_mma(MMA_AUTO)
    assert_rows_close(y, O.matmul(O.Q4K, x, q, n), what=f"int8 wide tiles same-sign {kind}")


def _random_shapes(count, seed=20261202):
    """(dt, m, n, k) drawn across every routing band: m from each of
    1-2, 3-4, 5-16, 17-64, 65-128, 129-600 and 601-1100 rows (the last: the
    int8 Q4_K route and the two-plane Q6_K route); k in whole blocks up to
    4608 (Q4_K / Q6_K in superblocks, Q8_0 in 32-element blocks); n ragged;
    m * n * k kept below 2.5e8 so the oracle stays fast."""
    rng = np.random.default_rng(seed)
    bands = [(1, 2), (3, 4), (5, 16), (17, 64), (65, 128), (129, 600), (601, 1100)]
    out = []
    while len(out) < count:
        dt = [O.Q8_0, O.Q4K, O.Q6K][len(out) % 3]
        lo, hi = bands[(len(out) // 3) % len(bands)]
        m = int(rng.integers(lo, hi + 1))
        be = 32 if dt == O.Q8_0 else 256
        k = be * int(rng.integers(1, 4608 // be + 1))
        n = int(rng.integers(1, 3000))
        if m * n * k <= 2.5e8:
            out.append((dt, m, n, k))
    return out


# LLOOM_HIP_PARITY_SEEDS=s draws 54 shapes from each of s seeds (default 1)
_SEEDS = int(os.environ.get("LLOOM_HIP_PARITY_SEEDS", "1"))


@pytest.mark.parametrize("dt,m,n,k", [c for i in range(_SEEDS) for c in _random_shapes(63, seed=20261202 + i)])
def test_random_shapes_all_routes(L, dt, m, n, k):
    """Seeded random shapes through every route against the oracle."""
    rng = np.random.default_rng(m * 131 + n * 7 + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y, q = _qmm(L, dt, w, x)
    assert_rows_close(y, O.matmul(dt, x, q, n), what=f"random dt={dt} m={m} n={n} k={k}")


@pytest.mark.parametrize("dt,m", [(O.Q4K, 3), (O.Q4K, 16), (O.Q4K, 17), (O.Q4K, 100), (O.Q6K, 5), (O.Q6K, 16)])
@pytest.mark.parametrize("n", [15, 16, 17, 6136, 6144, 6152])
def test_dma_kernel_tile_thresholds(L, dt, m, n):
    """The DMA kernel at k = 2048 around its tile edges: a partial first
    tile, exactly one, one row past; and around 384 weight tiles, where a
    workgroup takes two (6136 = 383.5 tiles, 6144, 6152)."""
    k = 2048
    rng = np.random.default_rng(n * 17 + m)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y, q = _qmm(L, dt, w, x)
    assert_rows_close(y, O.matmul(dt, x, q, n), what=f"tile edges dt={dt} m={m} n={n}")


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES + [(40, 33, 96), (300, 70, 160)])
def test_prefill_gemm_q8_0_shapes(L, m, n, k):
    """The Q8_0 prefill GEMM (K in whole 256-element steps) on ragged tiles,
    an all-zero activation block and a block holding one huge value; K
    not a multiple of 256 takes the 16-row decode tiles instead."""
    rng = np.random.default_rng(m * 5 + n)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[min(3, n - 1), :32] *= 50.0  # one weight block with a much larger scale
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1, :32] = 0.0  # an all-zero activation block (d = 0)
    x[min(2, m - 1), 37] = 1e4
    y, q = _qmm(L, O.Q8_0, w, x)
    assert_rows_close(y, O.matmul(O.Q8_0, x, q, n), what=f"q8_0 gemm m={m} n={n} k={k}")


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES + [(40, 33, 768), (300, 70, 1280), (200, 100, 8448), (129, 64, 4096),
                                                 (520, 130, 2304), (2048, 136, 8192), (320, 70, 8192)])
def test_prefill_gemm_q6k_shapes(L, m, n, k):
    """The Q6_K prefill GEMM on ragged tiles, an odd number of superblocks a
    row (rows then start 2 bytes off a 4-byte boundary), K split over
    workgroups (few tiles, long K: 33 superblocks in 7 splits of 5), an
    all-zero activation block and a weight row of extreme scales."""
    rng = np.random.default_rng(m * 3 + n)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[min(3, n - 1), :256] *= 80.0
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1, :256] = 0.0  # an all-zero activation block (d = 0)
    x[min(2, m - 1), 37] = 1e4
    y, q = _qmm(L, O.Q6K, w, x)
    assert_rows_close(y, O.matmul(O.Q6K, x, q, n), what=f"q6k gemm m={m} n={n} k={k}")


def test_q6k_plane_route_forced(L):
    """The Q6_K two-plane route forced on from the GEMM's first row count
    (LLOOM_HIP_Q6_PLANES=1 is read once per process, so in a child pytest):
    the Q6_K GEMM shape and split-K store tests again, which puts their
    shapes of 48 rows and up on it: single and ragged 256-row blocks, ragged
    columns, odd superblock counts, and up to eight K splits."""
    import subprocess
    import sys

    env = dict(os.environ, LLOOM_HIP_Q6_PLANES="1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", os.path.abspath(__file__),
                        "-k", "prefill_gemm_q6k_shapes or q6k_split_k_epilogues"],
                       env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    assert " passed" in r.stdout and "skipped" not in r.stdout.splitlines()[-1], r.stdout[-500:]


def test_prefill_gemm_q8_0_epilogues(L):
    """SiLU and multiply-into stores on the Q8_0 GEMM route."""
    rng = np.random.default_rng(21)
    m, n, k = 150, 200, 512
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    g = rng.standard_normal((m, n)).astype(np.float32)
    qt = L.QTensor.quantize(_cuda(w), O.Q8_0)
    mm = L.QMatMul.from_qtensor(qt)
    plain = mm.forward(_cuda(x)).cpu().numpy()
    want = O.matmul(O.Q8_0, x, qt.data(), n)
    assert_rows_close(plain, want, what="q8_0 plain")
    silu = mm.forward_silu(_cuda(x)).cpu().numpy()
    np.testing.assert_allclose(silu, _silu32(plain), rtol=2e-6, atol=1e-7)
    gg = _cuda(g)
    mm.forward_mul_into(_cuda(x), gg)
    assert np.array_equal(gg.cpu().numpy().view(np.uint32), (g * plain).astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
def test_qmatmul_closed_form_inputs(L, dt):
    """The reference's closed-form GEMM inputs (quantized_tests.rs:1769-1903)."""
    for m in [2, 17, 33]:
        for n in [1, 2, 3, 4, 7, 65]:
            for k in [256, 768]:
                lhs = (((np.arange(m * k) * 17 % 211).astype(np.float32) - 103) / 73).astype(np.float32).reshape(m, k)
                wts = (((np.arange(n * k) * 31 % 173).astype(np.float32) - 87) / 61).astype(np.float32).reshape(n, k)
                y, q = _qmm(L, dt, wts, lhs)
                assert_rows_close(y, O.matmul(dt, lhs, q, n), what=f"closed form dt={dt} {m},{n},{k}")


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
def test_decode_rows_batch_invariant(L, dt):
    """Within one decode kernel every activation row is computed alone, so a
    row's output does not depend on its batch (qmm_batch,
    quantized_tests.rs:239-275, exact on the CPU arm).  Q4_K and Q6_K with
    up to 16 rows run the MFMA kernels (3..4 rows at this k the
    single-launch variant, whose per-output arithmetic and partial-sum order
    are the two-launch kernel's) above the dot4 kernel's rows (1..2; Q4_K on
    a weight this small 1..4): each group is
    checked against its own full batch (across the two kernels only the
    tolerance holds, as on the reference's CUDA and Metal arms).  Q8_0 runs
    the 8-wave dot4 kernel for 1..2 rows and the 4-wave one above that (their
    lane partials meet in different reduction trees), and keeps one K-chunk
    (so one task set per lane) up to 4 rows at k = 1024; from 5 to 32 rows
    it runs the split-K GEMM (one configuration: the same sum order for
    every row)."""
    rng = np.random.default_rng(3)
    n, k = 96, 1024
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((32, k)).astype(np.float32)
    qt = L.QTensor.quantize(_cuda(w), dt)
    mm = L.QMatMul.from_qtensor(qt)
    groups = {O.Q4K: [(4, (1, 2, 3)), (16, (5, 8, 13))], O.Q6K: [(2, (1,)), (16, (3, 5, 8, 13))],
              O.Q8_0: [(2, (1,)), (4, (3,)), (32, (5, 9, 17))]}[dt]
    for full_m, ms in groups:
        full = mm.forward(_cuda(x[:full_m])).cpu().numpy()
        for m in ms:
            part = mm.forward(_cuda(x[:m])).cpu().numpy()
            assert np.array_equal(part.view(np.uint32), full[:m].view(np.uint32)), (full_m, m)


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
def test_mfma_decode_repeatable(L, dt):
    """3..16 rows run the workspace quantizer and the MFMA decode kernel:
    calls of other shapes in between (other k, other row counts, the shared
    workspace rewritten) must leave every repeat of a call bit-identical and
    within tolerance of the oracle."""
    rng = np.random.default_rng(21)
    shapes = [(1000, 4096, 5), (4100, 2048, 16), (300, 8192, 9), (64, 512, 3)]
    prepared = []
    for n, k, m in shapes:
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        x = rng.standard_normal((m, k)).astype(np.float32)
        qt = L.QTensor.quantize(_cuda(w), dt)
        prepared.append((L.QMatMul.from_qtensor(qt), _cuda(x), x, qt.data(), n))
    first = [mm.forward(xd).cpu().numpy() for mm, xd, _, _, _ in prepared]
    for (mm, xd, x, q, n), y in zip(prepared, first):
        assert_rows_close(y, O.matmul(dt, x, q, n), what=f"decode dt={dt} n={n} m={x.shape[0]}")
    for _ in range(2):
        for (mm, xd, _, _, _), y in zip(prepared[::-1], first[::-1]):
            again = mm.forward(xd).cpu().numpy()
            assert np.array_equal(again.view(np.uint32), y.view(np.uint32))


def test_qmatmul_rank3_input(L):
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((40, 512)) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, 3, 512)).astype(np.float32)
    qt = L.QTensor.quantize(_cuda(w), L.GgmlDType.Q4K)
    y = L.QMatMul.from_qtensor(qt).forward(_cuda(x)).cpu().numpy()
    assert y.shape == (2, 3, 40)
    assert_rows_close(y.reshape(6, 40), O.matmul(O.Q4K, x.reshape(6, 512), qt.data(), 40))


# BASELINE.json configs at their full shapes (the decode ones whole, the
# prefill one on a column subset the oracle finishes quickly).
def test_baseline_c1_q8_0_decode(L):
    w = L.synth_normal(0, 8192 * 2048, 0.0, 0.02).reshape(8192, 2048)
    x = L.synth_normal(1000, 2048).reshape(1, 2048)
    y, q = _qmm(L, O.Q8_0, w, x)
    assert_rows_close(y, O.matmul(O.Q8_0, x, q, 8192), what="C1")


@pytest.mark.parametrize("b", [1, 2, 4, 8, 16])
def test_baseline_c2_q4k_decode_sweep(L, b):
    w = L.synth_normal(1, 6144 * 2048, 0.0, 0.02).reshape(6144, 2048)
    x = L.synth_normal(1001 + b, b * 2048).reshape(b, 2048)
    y, q = _qmm(L, O.Q4K, w, x)
    assert_rows_close(y, O.matmul(O.Q4K, x, q, 6144), what=f"C2 b={b}")


@pytest.mark.parametrize("m", [64, 512])
def test_baseline_c3_q4k_prefill_subset(L, m):
    n, k = 8192, 2048
    w = L.synth_normal(2, n * k, 0.0, 0.02).reshape(n, k)
    x = L.synth_normal(2002 + m, m * k).reshape(m, k)
    y, q = _qmm(L, O.Q4K, w, x)
    cols = np.arange(0, n, 61)
    rowbytes = (k // 256) * 144
    qsub = np.concatenate([q[c * rowbytes:(c + 1) * rowbytes] for c in cols])
    rows = np.arange(0, m, 7) if m > 64 else np.arange(m)
    want = O.matmul(O.Q4K, x[rows], qsub, len(cols))
    assert_rows_close(y[np.ix_(rows, cols)], want, what=f"C3 m={m}")


@pytest.mark.parametrize("b", [1, 4, 16])
def test_baseline_c4_q6k_down_proj(L, b):
    w = L.synth_normal(3, 2048 * 8192, 0.0, 0.02).reshape(2048, 8192)
    x = L.synth_normal(3003, b * 8192).reshape(b, 8192)
    y, q = _qmm(L, O.Q6K, w, x)
    assert_rows_close(y, O.matmul(O.Q6K, x, q, 2048), what=f"C4 down b={b}")


# -------------------------------------------------------- routed experts ---

def _moe_case(L, dt, n_experts, n, k, batch, topk, in_dim1, seed, ids=None):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n_experts, n, k)) * 0.05).astype(np.float32)
    x = rng.standard_normal((batch, in_dim1, k)).astype(np.float32)
    if ids is None:
        ids = rng.integers(0, n_experts, (batch, topk)).astype(np.uint32)
        ids[0, :] = ids[0, 0]  # the same expert in several slots
        if batch > 1:
            ids[1, 0] = ids[0, 0]  # and across the batch
    qt = L.QTensor.quantize(_cuda(w), dt)
    got = qt.indexed_moe_forward(_cuda(x), _cuda(ids.astype(np.int32))).cpu().numpy()
    q = qt.data()
    want = O.matmul_indexed(dt, q, n_experts, n, k, x, ids)
    dense = O.dequantize(dt, q, w.size).reshape(n_experts, n, k).astype(np.float64)
    ref = np.empty((batch, topk, n))
    for b in range(batch):
        for t in range(topk):
            ref[b, t] = dense[ids[b, t]] @ x[b, 0 if in_dim1 == 1 else t].astype(np.float64)
    return got, want, ref


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
@pytest.mark.parametrize("in_dim1_is_topk", [False, True])
@pytest.mark.parametrize("n", [40, 37])
def test_moe_matches_oracle_and_dense(L, dt, in_dim1_is_topk, n):
    topk = 4
    got, want, ref = _moe_case(L, dt, 8, n, 512, 5, topk, topk if in_dim1_is_topk else 1, seed=n)
    assert_rows_close(got, want, what="moe vs oracle")
    rel = np.mean(np.abs(ref - got) / (np.abs(ref) + 1e-4))
    assert rel < 1e-4, rel


def test_moe_short_rows_and_many_experts(L):
    """k = 768 (the down projection's), 64 experts top-10."""
    got, want, ref = _moe_case(L, O.Q4K, 64, 48, 768, 6, 10, 10, seed=9)
    assert_rows_close(got, want, what="moe k=768")


def test_moe_run_to_run_identical(L):
    a, _, _ = _moe_case(L, O.Q4K, 16, 64, 1024, 8, 4, 1, seed=5)
    b, _, _ = _moe_case(L, O.Q4K, 16, 64, 1024, 8, 4, 1, seed=5)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_moe_many_planes_and_magnitudes(L):
    """Q4_K experts with dense routing (about 24 planes an expert: more than
    one pass of staged planes) and planes of very different magnitude (the
    fp16 operand path scales each plane by its own power of two): 1e4-scaled,
    1e-6-scaled, all-zero, and one element past the fp16 range."""
    rng = np.random.default_rng(21)
    E, n, k, batch, topk = 4, 80, 1024, 24, 4
    w = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    x = rng.standard_normal((batch, 1, k)).astype(np.float32)
    x[0] *= np.float32(1e4)
    x[1] *= np.float32(1e-6)
    x[2] = 0.0
    x[3, 0, 5] = 70000.0
    ids = rng.integers(0, E, (batch, topk)).astype(np.uint32)
    qt = L.QTensor.quantize(_cuda(w), O.Q4K)
    got = qt.indexed_moe_forward(_cuda(x), _cuda(ids.astype(np.int32))).cpu().numpy()
    q = qt.data()
    want = O.matmul_indexed(O.Q4K, q, E, n, k, x, ids)
    assert_rows_close(got, want, what="moe many planes")
    assert np.all(got[2] == 0.0)
    dense = O.dequantize(O.Q4K, q, w.size).reshape(E, n, k).astype(np.float64)
    ref = np.stack([np.stack([dense[ids[b, t]] @ x[b, 0].astype(np.float64) for t in range(topk)])
                    for b in range(batch)])
    scale = np.abs(ref).max(axis=2, keepdims=True) + 1e-30
    assert np.max(np.abs(ref - got) / scale) < 1e-5


@pytest.mark.parametrize("dt", [O.Q4K, O.Q8_0])
def test_moe_more_planes_than_one_list(L, dt):
    """1200 planes: past the in-kernel routing list, so the routing kernel
    sorts the planes first; a bad id among them is refused and its planes
    zeroed."""
    rng = np.random.default_rng(31)
    E, n, k, batch, topk = 8, 24, 256, 300, 4
    got, want, _ = _moe_case(L, dt, E, n, k, batch, topk, 1, seed=31)
    assert_rows_close(got, want, what="moe 1200 planes")
    w = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    qt = L.QTensor.quantize(_cuda(w), dt)
    ids = rng.integers(0, E, (batch, topk)).astype(np.int32)
    ids[7, 2] = E
    x = _cuda(rng.standard_normal((batch, 1, k)).astype(np.float32))
    with pytest.raises(L.LloomHipError):
        qt.indexed_moe_forward(x, _cuda(ids))
    y = qt.indexed_moe_forward(x, _cuda(ids), strict=False).cpu().numpy()
    assert np.all(y[7, 2] == 0) and np.any(y[7, 1] != 0)
    from lloom_amd.quantized import _ctx
    from lloom_amd.lib import lib

    assert lib().lloom_hip_ctx_sync(_ctx(0)) == 4


def test_moe_out_of_range_expert_is_refused(L):
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((4, 8, 256)) * 0.05).astype(np.float32)
    qt = L.QTensor.quantize(_cuda(w), L.GgmlDType.Q4K)
    x = _cuda(rng.standard_normal((2, 1, 256)).astype(np.float32))
    bad = _cuda(np.array([[0, 4], [1, 2]], dtype=np.int32))
    with pytest.raises(L.LloomHipError) as e:
        qt.indexed_moe_forward(x, bad)
    assert e.value.name == "EEXPERT"
    # deferred: the call returns, the next sync reports, then it is cleared
    y = qt.indexed_moe_forward(x, bad, strict=False)
    assert np.all(y[0, 1].cpu().numpy() == 0)
    from lloom_amd.quantized import _ctx
    from lloom_amd.lib import lib

    assert lib().lloom_hip_ctx_sync(_ctx(0)) == 4
    assert lib().lloom_hip_ctx_sync(_ctx(0)) == 0
    good = qt.indexed_moe_forward(x, _cuda(np.array([[0, 3], [1, 2]], dtype=np.int32)))
    assert np.isfinite(good.cpu().numpy()).all()


# ------------------------------------------------ store epilogues (f3) ---

def _silu32(v):
    v = np.asarray(v, dtype=np.float32)
    return (v / (np.float32(1) + np.exp(-v))).astype(np.float32)


@pytest.mark.parametrize("m", [64, 160, 700])
def test_q6k_split_k_epilogues(L, m):
    """SiLU and multiply-into stores where the Q6_K GEMM splits K over
    workgroups (one or two column tiles, 16 superblocks a row; m = 700 on
    the two-plane route, whose last row block is ragged): the stores
    are applied once, by the pass that adds the partial sums in split order,
    and a second, smaller call reuses the workspace the first one sized."""
    rng = np.random.default_rng(70 + m)
    n, k = 64, 4096
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    qt = L.QTensor.quantize(_cuda(w), O.Q6K)
    mm = L.QMatMul.from_qtensor(qt)
    xd = _cuda(x)
    plain = mm.forward(xd).cpu().numpy()
    want = O.matmul(O.Q6K, x, qt.data(), n)
    assert_rows_close(plain, want, what=f"q6k split-k m={m}")
    silu = mm.forward_silu(xd).cpu().numpy()
    np.testing.assert_allclose(silu, _silu32(plain), rtol=2e-6, atol=1e-7)
    gate = rng.standard_normal((m, n)).astype(np.float32)
    g = _cuda(gate)
    mm.forward_mul_into(xd, g)
    assert np.array_equal(g.cpu().numpy().view(np.uint32), (gate * plain).astype(np.float32).view(np.uint32))
    small = mm.forward(_cuda(x[:48])).cpu().numpy()
    assert_rows_close(small, want[:48], what="q6k split-k after a larger call")


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
@pytest.mark.parametrize("m", [1, 2, 5, 16, 40, 64, 200])
def test_forward_silu_and_mul_into(L, dt, m):
    """QMatMul::forward_silu / forward_mul_into (mod.rs:2102-2156): the
    stored value is silu(v) (resp. gate * v) of the product the plain
    forward stores.  Against the oracle: silu is 1.1-Lipschitz, so the
    matmul bar scaled by 1.1 bounds it; the product into the gate is bounded
    by the bar times |gate|.  Against the plain forward on the GPU the SiLU
    store is the same sum through v / (1 + exp(-v))."""
    rng = np.random.default_rng(40 + m)
    n, k = 300, 1024
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    qt = L.QTensor.quantize(_cuda(w), dt)
    mm = L.QMatMul.from_qtensor(qt)
    xd = _cuda(x)
    plain = mm.forward(xd).cpu().numpy()
    want = O.matmul(dt, x, qt.data(), n)
    rowmax = np.abs(want).max(axis=1, keepdims=True)
    silu = mm.forward_silu(xd).cpu().numpy()
    assert np.all(np.abs(silu - _silu32(want)) <= 1.1 * MATMUL_TOL * rowmax + 1e-30)
    np.testing.assert_allclose(silu, _silu32(plain), rtol=2e-6, atol=1e-7)
    gate = rng.standard_normal((m, n)).astype(np.float32)
    g = _cuda(gate)
    mm.forward_mul_into(xd, g)
    got = g.cpu().numpy()
    assert np.all(np.abs(got - gate * want) <= MATMUL_TOL * rowmax * np.abs(gate) + 1e-30)
    assert np.array_equal(got.view(np.uint32), (gate * plain).astype(np.float32).view(np.uint32))


def test_swiglu_silu_then_mul_into(L):
    """The SwiGLU as two launches: gate's forward_silu, then up's
    forward_mul_into its buffer = silu(g) * u (silu_mul order)."""
    rng = np.random.default_rng(7)
    n, k, m = 512, 2048, 4
    wg = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wu = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = _cuda(rng.standard_normal((m, k)).astype(np.float32))
    g = L.QMatMul.from_qtensor(L.QTensor.quantize(_cuda(wg), L.GgmlDType.Q4K))
    u = L.QMatMul.from_qtensor(L.QTensor.quantize(_cuda(wu), L.GgmlDType.Q4K))
    buf = g.forward_silu(x)
    u.forward_mul_into(x, buf)
    ref = (_silu32(g.forward(x).cpu().numpy()) * u.forward(x).cpu().numpy()).astype(np.float32)
    np.testing.assert_allclose(buf.cpu().numpy(), ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
@pytest.mark.parametrize("k", [768, 2048])
def test_moe_pair_and_glu(L, dt, k):
    """indexed_moe_forward_pair: each half bit for bit the single call's;
    _glu_as: silu(g) * u of those halves (mod.rs:1365-1531)."""
    rng = np.random.default_rng(k + dt)
    E, n, batch, topk = 16, 96, 6, 4
    wg = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    wu = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    x = _cuda(rng.standard_normal((batch, 1, k)).astype(np.float32))
    ids = _cuda(rng.integers(0, E, (batch, topk)).astype(np.int32))
    qg, qu = L.QTensor.quantize(_cuda(wg), dt), L.QTensor.quantize(_cuda(wu), dt)
    sg = qg.indexed_moe_forward(x, ids).cpu().numpy()
    su = qu.indexed_moe_forward(x, ids).cpu().numpy()
    pg, pu = qg.indexed_moe_forward_pair(qu, x, ids)
    assert np.array_equal(pg.cpu().numpy().view(np.uint32), sg.view(np.uint32))
    assert np.array_equal(pu.cpu().numpy().view(np.uint32), su.view(np.uint32))
    glu = qg.indexed_moe_forward_glu_as(qu, x, ids).cpu().numpy()
    np.testing.assert_allclose(glu, _silu32(sg) * su, rtol=2e-6, atol=1e-7)
    want = O.matmul_indexed(dt, qg.data(), E, n, k, x.cpu().numpy(), ids.cpu().numpy().astype(np.uint32))
    assert_rows_close(sg, want, what="moe gate vs oracle")


def test_moe_pair_bad_id_zeroes_both(L):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((4, 8, 256)) * 0.05).astype(np.float32)
    qg = L.QTensor.quantize(_cuda(w), L.GgmlDType.Q4K)
    qu = L.QTensor.quantize(_cuda(w * 2), L.GgmlDType.Q4K)
    x = _cuda(rng.standard_normal((2, 1, 256)).astype(np.float32))
    bad = _cuda(np.array([[0, 4], [1, 2]], dtype=np.int32))
    with pytest.raises(L.LloomHipError) as e:
        qg.indexed_moe_forward_pair(qu, x, bad)
    assert e.value.name == "EEXPERT"
    yg, yu = qg.indexed_moe_forward_pair(qu, x, bad, strict=False)
    assert np.all(yg[0, 1].cpu().numpy() == 0) and np.all(yu[0, 1].cpu().numpy() == 0)
    from lloom_amd.quantized import _ctx
    from lloom_amd.lib import lib

    assert lib().lloom_hip_ctx_sync(_ctx(0)) == 4
    with pytest.raises(L.LloomHipError):
        qg.indexed_moe_forward_pair(L.QTensor.quantize(_cuda(w[:, :4]), L.GgmlDType.Q4K), x, bad)


@pytest.mark.parametrize("n,k,in_dim1_is_topk,batch", [(100, 768, True, 20), (37, 2048, False, 20),
                                                     (256, 512, True, 300)])
def test_moe_dense_routing(L, n, k, in_dim1_is_topk, batch):
    """Q4_K experts with prefill-dense routing (at least 8 planes an active
    expert: the fp16-MFMA kernel, 16 planes a pass; 1200 planes route
    through the sorting launch): the down projection's shape (k = 768, a
    plane per slot), ragged n, against the oracle and a float64 dense
    reference."""
    topk = 4
    got, want, ref = _moe_case(L, O.Q4K, 4, n, k, batch, topk, topk if in_dim1_is_topk else 1, seed=n + k)
    assert_rows_close(got, want, what=f"moe dense n={n} k={k}")
    scale = np.abs(ref).max(axis=2, keepdims=True) + 1e-30
    assert np.max(np.abs(ref - got) / scale) < 1e-5


def test_moe_dense_pair_glu_and_bad_id(L):
    """Dense routing through the pair and GLU launches (each pair half bit
    for bit the single call's, the GLU silu(g) * u of them), and an
    out-of-range id: refused by the strict call, its plane zeroed in both
    outputs otherwise."""
    rng = np.random.default_rng(33)
    E, n, k, batch, topk = 4, 96, 1024, 24, 4
    wg = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    wu = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    x = _cuda(rng.standard_normal((batch, 1, k)).astype(np.float32))
    idn = rng.integers(0, E, (batch, topk)).astype(np.int32)
    ids = _cuda(idn)
    qg, qu = L.QTensor.quantize(_cuda(wg), O.Q4K), L.QTensor.quantize(_cuda(wu), O.Q4K)
    sg = qg.indexed_moe_forward(x, ids).cpu().numpy()
    su = qu.indexed_moe_forward(x, ids).cpu().numpy()
    pg, pu = qg.indexed_moe_forward_pair(qu, x, ids)
    assert np.array_equal(pg.cpu().numpy().view(np.uint32), sg.view(np.uint32))
    assert np.array_equal(pu.cpu().numpy().view(np.uint32), su.view(np.uint32))
    glu = qg.indexed_moe_forward_glu_as(qu, x, ids).cpu().numpy()
    np.testing.assert_allclose(glu, _silu32(sg) * su, rtol=2e-6, atol=1e-7)
    assert_rows_close(sg, O.matmul_indexed(O.Q4K, qg.data(), E, n, k, x.cpu().numpy(), idn.astype(np.uint32)),
                      what="moe dense gate")
    idn[5, 1] = E
    bad = _cuda(idn)
    with pytest.raises(L.LloomHipError) as e:
        qg.indexed_moe_forward_pair(qu, x, bad)
    assert e.value.name == "EEXPERT"
    yg, yu = qg.indexed_moe_forward_pair(qu, x, bad, strict=False)
    assert np.all(yg[5, 1].cpu().numpy() == 0) and np.all(yu[5, 1].cpu().numpy() == 0)
    assert np.array_equal(yg[4].cpu().numpy().view(np.uint32), sg[4].view(np.uint32))
    from lloom_amd.quantized import _ctx
    from lloom_amd.lib import lib

    assert lib().lloom_hip_ctx_sync(_ctx(0)) == 4


# ---------------------------------------------------------- embedding (f4) ---

@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
def test_embedding_bit_exact(L, dt):
    """QTensor::embedding (mod.rs:1101-1137): rows of to_float, bit-exact,
    ids of any shape; f16 out is the RNE of the f32 rows."""
    rng = np.random.default_rng(dt)
    rows, hidden = 300, 512
    w = rng.standard_normal((rows, hidden)).astype(np.float32)
    qt = L.QTensor.quantize(_cuda(w), dt)
    full = O.dequantize(dt, qt.data(), rows * hidden).reshape(rows, hidden)
    ids = rng.integers(0, rows, (3, 7)).astype(np.int32)
    ids[0, 0] = rows - 1
    ids[0, 1] = 0
    got = qt.embedding(_cuda(ids)).cpu().numpy()
    assert got.shape == (3, 7, hidden)
    assert np.array_equal(got.view(np.uint32), full[ids].view(np.uint32))
    h = qt.embedding(_cuda(ids), f16=True).cpu().numpy()
    assert np.array_equal(h.view(np.uint16), full[ids].astype(np.float16).view(np.uint16))
    assert qt.embedding(_cuda(np.zeros((0,), np.int32))).shape == (0, hidden)


def test_embedding_bad_id(L):
    rng = np.random.default_rng(1)
    qt = L.QTensor.quantize(_cuda(rng.standard_normal((10, 256)).astype(np.float32)), L.GgmlDType.Q4K)
    bad = _cuda(np.array([3, 10, 2], dtype=np.int32))
    with pytest.raises(L.LloomHipError) as e:
        qt.embedding(bad)
    assert e.value.name == "EEXPERT" and "out of range" in str(e.value)
    y = qt.embedding(bad, strict=False).cpu().numpy()
    assert np.all(y[1] == 0) and np.any(y[0] != 0)
    from lloom_amd.quantized import _ctx
    from lloom_amd.lib import lib

    assert lib().lloom_hip_ctx_sync(_ctx(0)) == 4
    assert lib().lloom_hip_ctx_sync(_ctx(0)) == 0


# ------------------------------------------------------------- refusals ---

def test_refusals_are_named(L):
    w = _cuda(np.zeros((4, 256), np.float32))
    with pytest.raises(L.LloomHipError) as e:
        L.QTensor.quantize(_cuda(np.zeros((4, 100), np.float32)), L.GgmlDType.Q4K)
    assert e.value.name == "ESHAPE"
    qt = L.QTensor.quantize(w, L.GgmlDType.Q4K)
    with pytest.raises(L.LloomHipError) as e:
        L.QMatMul.from_qtensor(qt).forward(_cuda(np.zeros((2, 512), np.float32)))
    assert e.value.name == "ESHAPE"
    with pytest.raises(L.LloomHipError) as e:
        L.QMatMul.from_qtensor(qt).forward(torch.zeros((2, 256), dtype=torch.bfloat16, device=DEV))
    assert e.value.name == "EDTYPE"
    from lloom_amd.quantized import _ctx, _ptr, _stream
    from lloom_amd.lib import lib

    x = _cuda(np.zeros((1, 256), np.float32))
    y = torch.empty((1, 4), device=DEV)
    rc = lib().lloom_hip_qmatmul(_ctx(0), 15, _ptr(qt.storage), 4, 256, _ptr(x), 0, 1, _ptr(y), 0, _stream(x))
    assert rc == 2 and b"Q8K" in lib().lloom_hip_last_error()
    # prefill matrix-core modes: F16 (0), INT8 (1), AUTO (2, the default); others refused
    assert lib().lloom_hip_ctx_set_prefill_mma(_ctx(0), 3) == 1
    assert b"AUTO (2)" in lib().lloom_hip_last_error()
    for mode in (0, 1, 2):
        assert lib().lloom_hip_ctx_set_prefill_mma(_ctx(0), mode) == 0


@pytest.mark.parametrize("dt,m,n,k", [(O.Q8_0, 9, 300, 2048), (O.Q8_0, 100, 300, 2048), (O.Q8_0, 600, 300, 1024),
                                      (O.Q6K, 64, 200, 8192), (O.Q6K, 300, 256, 8192), (O.Q4K, 40, 300, 2048),
                                      (O.Q4K, 700, 300, 2048)])
def test_prefill_repeatable(L, dt, m, n, k):
    """Every prefill route sums in a fixed order (K split over waves or
    workgroups included: the partial sums meet in wave or split order), so a
    repeated call is bit-identical."""
    rng = np.random.default_rng(m + n)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = _cuda(rng.standard_normal((m, k)).astype(np.float32))
    mm = L.QMatMul.from_qtensor(L.QTensor.quantize(_cuda(w), dt))
    a = mm.forward(x).cpu().numpy()
    b = mm.forward(x).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))

