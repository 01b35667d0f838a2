"""GPU parity at BASELINE.json's full workloads (C3 at M = 2048, the six Q4_K
projections of C4, the C5 routed-expert layer), the routed-expert `act`
variants, f16 activations on the dense path, the long-row routed route, and
the workspace contract (reserve, capture refusal, graph replays).

Bars as in test_gpu_parity.py: max|d| <= 1e-3 * max|y row| against the
oracle; routed experts also mean relative error < 1e-4 against a dense
float64 reference (lloom-tensor/tests/moe_routed_metal.rs:148-154).
"""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

MATMUL_TOL = 1e-3
DEV = "cuda:0"


@pytest.fixture(scope="module")
def L():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lloom_amd

    lloom_amd.lib()
    return lloom_amd


def _cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def assert_rows_close(got, want, tol=MATMUL_TOL, what="", extra=0.0):
    got = np.asarray(got, dtype=np.float64).reshape(-1, want.shape[-1])
    want = np.asarray(want, dtype=np.float64).reshape(-1, want.shape[-1])
    bound = tol * np.abs(want).max(axis=1, keepdims=True) + extra + 1e-30
    err = np.abs(got - want)
    bad = err > bound
    assert not bad.any(), f"{what}: {bad.sum()} outputs out of tolerance, worst ratio {(err / bound).max():.3g}"


def _rows_of(q, dt, k, cols):
    rb = (k // O.BLOCK_ELEMS[dt]) * O.BLOCK_BYTES[dt]
    return np.concatenate([q[c * rb:(c + 1) * rb] for c in cols])


# ------------------------------------------------------------------ C3 ---

@pytest.mark.parametrize("mma", ["f16", "int8"])
def test_c3_q4k_prefill_m2048(L, mma):
    """C3 at M = 2048 on W [8192, 2048] (the largest prefill tile, every
    activation row), checked on a column subset that covers every column
    tile and both halves of each."""
    from lloom_amd.quantized import MMA_AUTO, MMA_F16, MMA_INT8, set_prefill_mma

    n, k, m = 8192, 2048, 2048
    w = L.synth_normal(2, n * k, 0.0, 0.02).reshape(n, k)
    x = L.synth_normal(2000 + m, m * k).reshape(m, k)
    qt = L.QTensor.quantize(_cuda(w), O.Q4K)
    set_prefill_mma(MMA_INT8 if mma == "int8" else MMA_F16)
    try:
        y = L.QMatMul.from_qtensor(qt).forward(_cuda(x)).cpu().numpy()
    finally:
        set_prefill_mma(MMA_AUTO)
    cols = np.unique(np.concatenate([np.arange(0, n, 53), np.arange(127, n, 128)]))
    want = O.matmul(O.Q4K, x, _rows_of(qt.data(), O.Q4K, k, cols), len(cols))
    assert_rows_close(y[:, cols], want, what=f"C3 m=2048 {mma}")


# ------------------------------------------------------------------ C4 ---

C4_Q4K = [("q", 2048, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 2048), ("gate", 8192, 2048),
          ("up", 8192, 2048)]


@pytest.mark.parametrize("b", [1, 4, 16])
def test_c4_q4k_projections(L, b):
    """The six Q4_K projections of the C4 decoder layer at their full shapes
    (seeds as bench.py draws them), on the continuous-batching row counts."""
    for i, (name, n, k) in enumerate(C4_Q4K):
        w = L.synth_normal(30 + i, n * k, 0.0, 0.02).reshape(n, k)
        x = L.synth_normal(300 + k + 17 * b, b * k).reshape(b, k)
        qt = L.QTensor.quantize(_cuda(w), O.Q4K)
        y = L.QMatMul.from_qtensor(qt).forward(_cuda(x)).cpu().numpy()
        assert_rows_close(y, O.matmul(O.Q4K, x, qt.data(), n), what=f"C4 {name} b={b}")


# ------------------------------------------------------------------ C5 ---

@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("k", [1024, 2048, 4096, 8192, 16384])
def test_decode_rows_long_k(L, dt, k):
    """3..16 activation rows at short and long K (k_mv_fused, k_mv_dma up to
    2048, k_mv_mfma with K split over waves and workgroups past it: the C4
    Q6_K down projection is k = 8192); ragged n; the SiLU store too."""
    rng = np.random.default_rng(k + dt)
    n = 40
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    q = L.QTensor.quantize(_cuda(w), dt)
    qb = q.data()
    mm = L.QMatMul.from_qtensor(q)
    for m in (3, 5, 16):
        x = rng.standard_normal((m, k)).astype(np.float32)
        want = O.matmul(dt, x, qb, n)
        got = mm.forward(_cuda(x)).cpu().numpy()
        assert_rows_close(got, want, what=f"dt={dt} k={k} m={m}")
        silu = mm.forward_silu(_cuda(x)).cpu().numpy()
        ref = (want / (1.0 + np.exp(-want.astype(np.float64)))).astype(np.float32)
        assert_rows_close(silu, ref, tol=1.1 * MATMUL_TOL, what=f"silu dt={dt} k={k} m={m}")


def _c5_routing(L, T=32, E=128, topk=8, seed=4):
    """top-8 of softmax(U(0,1) logits), descending, ties to the lower index."""
    logits = L.synth_uniform(seed, T * E).reshape(T, E).astype(np.float64)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    return np.argsort(-p, axis=1, kind="stable")[:, :topk].astype(np.uint32)


def _dense_ref(dt, q, E, n, k, x, ids):
    """float64 planes of the exactly dequantized experts, one expert at a time."""
    batch, in_dim1, _ = x.shape
    topk = ids.shape[1]
    eb = n * (k // 256) * O.BLOCK_BYTES[dt]
    ref = np.empty((batch, topk, n))
    for e in np.unique(ids):
        we = O.dequantize(dt, q[e * eb:(e + 1) * eb], n * k).reshape(n, k).astype(np.float64)
        for b, t in zip(*np.nonzero(ids == e)):
            ref[b, t] = we @ x[b, 0 if in_dim1 == 1 else t].astype(np.float64)
    return ref


@pytest.mark.parametrize("proj", ["gate", "up", "down"])
def test_c5_moe_layer(L, proj):
    """C5: 128 Q4_K experts, gate/up [768, 2048] (x [32, 1, 2048]) and down
    [2048, 768] (x [32, 8, 768], one row a slot), 32 tokens top-8."""
    E, ff, hid, T, topk = 128, 768, 2048, 32, 8
    n, k, seed, in_dim1 = {"gate": (ff, hid, 40, 1), "up": (ff, hid, 41, 1), "down": (hid, ff, 42, topk)}[proj]
    ids = _c5_routing(L)
    w = L.synth_normal(seed, E * n * k, 0.0, 0.02).reshape(E, n, k)
    x = L.synth_normal(4000 if in_dim1 == 1 else 4001, T * in_dim1 * k).reshape(T, in_dim1, k)
    qt = L.QTensor.quantize(_cuda(w), O.Q4K)
    got = qt.indexed_moe_forward(_cuda(x), _cuda(ids.astype(np.int32))).cpu().numpy()
    q = qt.data()
    want = O.matmul_indexed(O.Q4K, q, E, n, k, x, ids)
    assert_rows_close(got, want, what=f"C5 {proj}")
    ref = _dense_ref(O.Q4K, q, E, n, k, x, ids)
    rel = np.mean(np.abs(ref - got) / (np.abs(ref) + 1e-4))
    assert rel < 1e-4, rel


def test_c5_swiglu_launch(L):
    """C5 gate and up as one SwiGLU launch: silu(g) * u of the single calls."""
    E, ff, hid, T = 128, 768, 2048, 32
    ids = _cuda(_c5_routing(L).astype(np.int32))
    x = _cuda(L.synth_normal(4000, T * hid).reshape(T, 1, hid))
    qg = L.QTensor.quantize(_cuda(L.synth_normal(40, E * ff * hid, 0.0, 0.02).reshape(E, ff, hid)), O.Q4K)
    qu = L.QTensor.quantize(_cuda(L.synth_normal(41, E * ff * hid, 0.0, 0.02).reshape(E, ff, hid)), O.Q4K)
    g = qg.indexed_moe_forward(x, ids).cpu().numpy()
    u = qu.indexed_moe_forward(x, ids).cpu().numpy()
    glu = qg.indexed_moe_forward_glu_as(qu, x, ids).cpu().numpy()
    silu = (g / (np.float32(1) + np.exp(-g))).astype(np.float32)
    np.testing.assert_allclose(glu, silu * u, rtol=2e-6, atol=1e-7)


# ----------------------------------------------------- long routed rows ---

@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K, O.Q8_0])
def test_moe_rows_too_long_to_stage(L, dt):
    """k = 16640 (65 superblocks): past what one workgroup stages in LDS, so
    the routed planes go through the sorting launch and the row kernel that
    reads the activations from L2; the GLU there is the pair plus the
    silu-multiply pass."""
    rng = np.random.default_rng(dt)
    E, n, k, batch, topk = 6, 40, 16640, 5, 3
    wg = (rng.standard_normal((E, n, k)) * 0.02).astype(np.float32)
    wu = (rng.standard_normal((E, n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((batch, 1, k)).astype(np.float32)
    ids = rng.integers(0, E, (batch, topk)).astype(np.uint32)
    qg, qu = L.QTensor.quantize(_cuda(wg), dt), L.QTensor.quantize(_cuda(wu), dt)
    xd, idd = _cuda(x), _cuda(ids.astype(np.int32))
    g = qg.indexed_moe_forward(xd, idd).cpu().numpy()
    assert_rows_close(g, O.matmul_indexed(dt, qg.data(), E, n, k, x, ids), what="long rows")
    u = qu.indexed_moe_forward(xd, idd).cpu().numpy()
    pg, pu = qg.indexed_moe_forward_pair(qu, xd, idd)
    assert np.array_equal(pg.cpu().numpy().view(np.uint32), g.view(np.uint32))
    assert np.array_equal(pu.cpu().numpy().view(np.uint32), u.view(np.uint32))
    glu = qg.indexed_moe_forward_glu_as(qu, xd, idd).cpu().numpy()
    silu = (g / (np.float32(1) + np.exp(-g))).astype(np.float32)
    np.testing.assert_allclose(glu, silu * u, rtol=2e-6, atol=1e-7)


# ------------------------------------------------------ act = f16 (MoE) ---

def _f16_round(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("dt", [O.Q4K, O.Q8_0, O.Q6K])
def test_moe_forward_as_f16(L, dt):
    """indexed_moe_forward_as / _pair_as / _glu_as with act = f16
    (mod.rs:1403, 1560-1575): what the f32 call computes on x rounded to
    f16; an f16 x with act None is the same computation."""
    rng = np.random.default_rng(50 + dt)
    E, n, k, batch, topk = 8, 72, 768, 6, 4
    wg = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    wu = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    x = (rng.standard_normal((batch, 1, k)) * 3).astype(np.float32)
    x[0, 0, :4] = [1e-6, 65519.0, -3.0e-8, 0.1]  # subnormal in f16, rounding to the top, flush, inexact
    ids = rng.integers(0, E, (batch, topk)).astype(np.uint32)
    qg, qu = L.QTensor.quantize(_cuda(wg), dt), L.QTensor.quantize(_cuda(wu), dt)
    xd, idd = _cuda(x), _cuda(ids.astype(np.int32))
    xr = _f16_round(x)
    got = qg.indexed_moe_forward_as(xd, idd, act=torch.float16).cpu().numpy()
    want_bits = qg.indexed_moe_forward(_cuda(xr), idd).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want_bits.view(np.uint32))
    assert_rows_close(got, O.matmul_indexed(dt, qg.data(), E, n, k, xr, ids), what="moe as f16")
    h = qg.indexed_moe_forward(xd.half(), idd).cpu().numpy()
    assert np.array_equal(h.view(np.uint32), got.view(np.uint32))
    # f32 act of an f32 x is the plain call
    same = qg.indexed_moe_forward_as(xd, idd, act=torch.float32).cpu().numpy()
    assert np.array_equal(same.view(np.uint32), qg.indexed_moe_forward(xd, idd).cpu().numpy().view(np.uint32))
    pg, pu = qg.indexed_moe_forward_pair_as(qu, xd, idd, act=torch.float16)
    assert np.array_equal(pg.cpu().numpy().view(np.uint32), got.view(np.uint32))
    u = qu.indexed_moe_forward(_cuda(xr), idd).cpu().numpy()
    assert np.array_equal(pu.cpu().numpy().view(np.uint32), u.view(np.uint32))
    glu = qg.indexed_moe_forward_glu_as(qu, xd, idd, act=torch.float16).cpu().numpy()
    silu = (got / (np.float32(1) + np.exp(-got))).astype(np.float32)
    np.testing.assert_allclose(glu, silu * u, rtol=2e-6, atol=1e-7)
    with pytest.raises(L.LloomHipError) as e:
        qg.indexed_moe_forward_as(xd, idd, act=torch.bfloat16)
    assert e.value.name == "EDTYPE"


# -------------------------------------------------- f16 dense activations ---

@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4K, O.Q6K])
@pytest.mark.parametrize("m", [1, 3, 16, 40, 300])
def test_qmatmul_f16_activations(L, dt, m):
    """matmul_t_f16 (k_quants.rs:2802-2835): the f16 x widened to f32, the
    f32 path, each sum rounded to f16.  Bit for bit the f32 call on the
    widened x, rounded; within the matmul bar (plus half an f16 ulp of the
    value) of the oracle."""
    rng = np.random.default_rng(60 + m)
    n, k = 200, 1024
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x16 = rng.standard_normal((m, k)).astype(np.float16)
    qt = L.QTensor.quantize(_cuda(w), dt)
    mm = L.QMatMul.from_qtensor(qt)
    y = mm.forward(_cuda(x16))
    assert y.dtype == torch.float16 and y.shape == (m, n)
    y = y.cpu().numpy()
    y32 = mm.forward(_cuda(x16.astype(np.float32))).cpu().numpy()
    assert np.array_equal(y.view(np.uint16), y32.astype(np.float16).view(np.uint16))
    want = O.matmul(dt, x16.astype(np.float32), qt.data(), n)
    ulp = np.abs(want) * 2.0 ** -11
    assert_rows_close(y.astype(np.float32), want, what=f"f16 dt={dt} m={m}", extra=ulp)
    # the store epilogues in f16: SiLU of the f32 sum, then rounded
    s = mm.forward_silu(_cuda(x16)).cpu().numpy()
    assert np.array_equal(s.view(np.uint16), mm.forward_silu(_cuda(x16.astype(np.float32))).cpu().numpy()
                          .astype(np.float16).view(np.uint16))
    gate = rng.standard_normal((m, n)).astype(np.float16)
    g = _cuda(gate)
    mm.forward_mul_into(_cuda(x16), g)
    assert np.array_equal(g.cpu().numpy().view(np.uint16),
                          (gate.astype(np.float32) * y32).astype(np.float16).view(np.uint16))


def test_cast_round_trip(L):
    """lloom_hip_cast: f32 -> f16 is RNE (numpy's), f16 -> f32 exact, ragged
    counts (a tail that is not a multiple of four)."""
    from lloom_amd.quantized import _cast

    rng = np.random.default_rng(8)
    for count in (1, 7, 1024, 100003):
        a = (rng.standard_normal(count) * 100).astype(np.float32)
        a[:min(count, 3)] = [np.float32(65520.0), np.float32(2.0 ** -25), np.float32(-0.0)][:min(count, 3)]
        h = _cast(_cuda(a), torch.float16).cpu().numpy()
        assert np.array_equal(h.view(np.uint16), a.astype(np.float16).view(np.uint16))
        b = _cast(_cuda(h), torch.float32).cpu().numpy()
        assert np.array_equal(b.view(np.uint32), h.astype(np.float32).view(np.uint32))


# --------------------------------------------------- argument refusals ---

def test_into_helpers_refuse_bad_buffers(L):
    rng = np.random.default_rng(9)
    qt = L.QTensor.quantize(_cuda((rng.standard_normal((64, 512)) * 0.02).astype(np.float32)), O.Q4K)
    mm = L.QMatMul.from_qtensor(qt)
    x = _cuda(rng.standard_normal((4, 512)).astype(np.float32))
    with pytest.raises(L.LloomHipError):
        mm.forward_into(x, torch.empty((4, 63), device=DEV))  # too small
    with pytest.raises(L.LloomHipError):
        mm.forward_into(x, torch.empty((4, 64), device=DEV, dtype=torch.float16))  # wrong dtype
    with pytest.raises(L.LloomHipError):
        mm.forward_into(x, torch.empty((64, 4), device=DEV).t())  # not contiguous
    with pytest.raises(L.LloomHipError):
        mm.forward_into(_cuda(rng.standard_normal((512, 4)).astype(np.float32)).t(), torch.empty((4, 64), device=DEV))
    with pytest.raises(L.LloomHipError):
        mm.forward_into(x.cpu(), torch.empty((4, 64), device=DEV))
    y = mm.forward_into(x, torch.empty((4, 64), device=DEV))
    assert_rows_close(y.cpu().numpy(), O.matmul(O.Q4K, x.cpu().numpy(), qt.data(), 64), what="into")
    E = 4
    qe = L.QTensor.quantize(_cuda((rng.standard_normal((E, 16, 256)) * 0.05).astype(np.float32)), O.Q4K)
    xe = _cuda(rng.standard_normal((3, 1, 256)).astype(np.float32))
    ids = _cuda(np.zeros((3, 2), np.int32))
    with pytest.raises(L.LloomHipError):
        qe.indexed_moe_forward_into(xe, ids, torch.empty((3, 2, 15), device=DEV))
    with pytest.raises(L.LloomHipError):
        qe.indexed_moe_forward_into(xe.half(), ids, torch.empty((3, 2, 16), device=DEV))
    with pytest.raises(L.LloomHipError):
        qe.indexed_moe_forward_into(xe, ids.long(), torch.empty((3, 2, 16), device=DEV))
    with pytest.raises(L.LloomHipError):
        qe.indexed_moe_forward_glu_into(qe, xe, ids, torch.empty((3, 2, 16), device=DEV, dtype=torch.float16))


# ------------------------------------------------------------ workspace ---

def test_workspace_reserve_and_capture(L):
    """A call whose workspace would grow during graph capture is refused by
    name; after lloom_hip_ctx_reserve the same call captures, and every
    replay (with eager calls of other shapes in between) equals the eager
    result."""
    from lloom_amd.quantized import qmatmul_workspace_bytes, reserve_workspace

    rng = np.random.default_rng(12)
    n, k, m = 512, 4096, 700  # a prefill shape with a large prepared-activation buffer
    qt = L.QTensor.quantize(_cuda((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), O.Q4K)
    mm = L.QMatMul.from_qtensor(qt)
    x = _cuda(rng.standard_normal((m, k)).astype(np.float32))
    y = torch.empty((m, n), device=DEV)
    need = qmatmul_workspace_bytes(O.Q4K, n, k, m)
    assert need >= m * k  # at least the quantized activations
    from lloom_amd.quantized import _ctx
    from lloom_amd.lib import lib
    import ctypes

    have = ctypes.c_size_t()
    assert lib().lloom_hip_ctx_workspace_bytes(_ctx(0), ctypes.byref(have)) == 0
    big = max(need, have.value) * 4  # surely more than the context holds
    x_big = _cuda(rng.standard_normal((m * 4, k)).astype(np.float32))
    y_big = torch.empty((m * 4, n), device=DEV)
    if qmatmul_workspace_bytes(O.Q4K, n, k, m * 4) > have.value:
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        caught = []
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                y_big.zero_()  # the capture is not empty
                try:
                    mm.forward_into(x_big, y_big)
                except L.LloomHipError as e:
                    caught.append(e)
        torch.cuda.current_stream().wait_stream(s)
        assert caught and caught[0].name == "ENOMEM" and "captured" in str(caught[0])
    torch.cuda.synchronize()
    reserve_workspace(big)
    assert lib().lloom_hip_ctx_workspace_bytes(_ctx(0), ctypes.byref(have)) == 0 and have.value >= big
    eager = mm.forward_into(x, y).clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            mm.forward_into(x, y)
    torch.cuda.current_stream().wait_stream(s)
    other = L.QMatMul.from_qtensor(qt)
    for i in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i
        other.forward(x[: 5 + i])  # eager work of another shape between replays
        torch.cuda.synchronize()
