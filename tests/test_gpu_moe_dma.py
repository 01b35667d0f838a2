"""GPU parity of the decode-routing Q4_K expert kernel (k_moe_dma: 1.75 to
2.5 planes an expert on average, rows of 2048 elements) against the CPU
oracle (matmul_indexed, the reference's matmul_t_indexed arithmetic,
mod.rs:766-810) and a float64 dense reference, through the C ABI.

Cases: row counts off the 32-row tile pair and the 16-row tile (n = 8, 37,
200), 1 to 40 planes on one expert (more than 8 and more than 16 take extra
passes over the staged tiles), runs of several tile pairs a workgroup
(n = 2048), activations one row a token and one row a slot, the pair and
SwiGLU launches bit for bit against the single calls, activations of very
different magnitudes across superblocks (each superblock has its own power
of two), and an out-of-range id.
"""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

MATMUL_TOL = 1e-3


@pytest.fixture(scope="module")
def L():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lloom_amd

    lloom_amd.lib()
    return lloom_amd


def _cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _rows_close(got, want, what):
    bound = MATMUL_TOL * np.abs(want).max(axis=-1, keepdims=True) + 1e-30
    err = np.abs(np.asarray(got, np.float64) - want)
    assert not (err > bound).any(), f"{what}: worst ratio {(err / bound).max():.3g}"


def _dense(q, E, n, k, x, ids):
    dense = O.dequantize(O.Q4K, q, E * n * k).reshape(E, n, k).astype(np.float64)
    batch, in_dim1, _ = x.shape
    topk = ids.shape[1]
    return np.stack([np.stack([dense[ids[b, t]] @ x[b, 0 if in_dim1 == 1 else t].astype(np.float64)
                               for t in range(topk)]) for b in range(batch)])


def _skewed_ids(rng, E, batch, topk, hot, hot_planes):
    """Random ids with `hot_planes` of the planes on expert `hot` (one slot
    of a token at most once per expert is not required by the API)."""
    ids = rng.integers(0, E, (batch, topk)).astype(np.uint32)
    flat = ids.reshape(-1)
    flat[rng.choice(flat.size, hot_planes, replace=False)] = hot
    return ids


# (E, n, k, batch, topk, in_dim1 is topk, planes on the hot expert)
CASES = [(16, 200, 2048, 4, 8, False, 20), (16, 37, 2048, 4, 8, True, 12), (12, 64, 2048, 4, 6, False, 9),
         (9, 8, 2048, 4, 4, True, 5), (20, 96, 2048, 5, 8, False, 17), (24, 48, 2048, 6, 8, True, 1),
         (10, 2048, 2048, 5, 4, False, 3)]


@pytest.mark.parametrize("E,n,k,batch,topk,per_slot,hot", CASES)
def test_moe_dma_matches_oracle(L, E, n, k, batch, topk, per_slot, hot):
    rng = np.random.default_rng(E * 1000 + k + n)
    planes = batch * topk
    assert 7 * E <= 4 * planes < 10 * E  # the routing density k_moe_dma takes
    w = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    in_dim1 = topk if per_slot else 1
    x = rng.standard_normal((batch, in_dim1, k)).astype(np.float32)
    # superblocks of very different magnitude in one row
    x[0, 0, :256] *= 1e4
    x[0, 0, 256:512] *= 1e-4
    ids = _skewed_ids(rng, E, batch, topk, hot=E // 2, hot_planes=hot)
    qt = L.QTensor.quantize(_cuda(w), O.Q4K)
    got = qt.indexed_moe_forward(_cuda(x), _cuda(ids.astype(np.int32))).cpu().numpy()
    q = qt.data()
    _rows_close(got, O.matmul_indexed(O.Q4K, q, E, n, k, x, ids), f"E={E} n={n} k={k}")
    ref = _dense(q, E, n, k, x, ids)
    scale = np.abs(ref).max(axis=2, keepdims=True) + 1e-30
    assert np.max(np.abs(ref - got) / scale) < 1e-5


def test_moe_dma_pair_glu_bits(L):
    """The pair launch is the two single calls bit for bit; the SwiGLU launch
    is silu(gate) * up of them (mod.rs:1365-1531)."""
    rng = np.random.default_rng(77)
    E, n, k, batch, topk = 16, 100, 2048, 4, 8
    wg = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    wu = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    x = _cuda(rng.standard_normal((batch, 1, k)).astype(np.float32))
    ids = _cuda(_skewed_ids(rng, E, batch, topk, hot=3, hot_planes=20).astype(np.int32))
    qg, qu = L.QTensor.quantize(_cuda(wg), O.Q4K), L.QTensor.quantize(_cuda(wu), O.Q4K)
    g = qg.indexed_moe_forward(x, ids).cpu().numpy()
    u = qu.indexed_moe_forward(x, ids).cpu().numpy()
    pg, pu = qg.indexed_moe_forward_pair(qu, x, ids)
    assert np.array_equal(pg.cpu().numpy().view(np.uint32), g.view(np.uint32))
    assert np.array_equal(pu.cpu().numpy().view(np.uint32), u.view(np.uint32))
    glu = qg.indexed_moe_forward_glu_as(qu, x, ids).cpu().numpy()
    silu = (g / (np.float32(1) + np.exp(-g))).astype(np.float32)
    np.testing.assert_allclose(glu, silu * u, rtol=2e-6, atol=1e-7)
    again = qg.indexed_moe_forward(x, ids).cpu().numpy()
    assert np.array_equal(again.view(np.uint32), g.view(np.uint32))


def test_moe_dma_bad_id(L):
    rng = np.random.default_rng(5)
    E, n, k, batch, topk = 8, 40, 2048, 4, 4
    w = (rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)
    qt = L.QTensor.quantize(_cuda(w), O.Q4K)
    x = _cuda(rng.standard_normal((batch, 1, k)).astype(np.float32))
    ids = rng.integers(0, E, (batch, topk)).astype(np.int32)
    ids[2, 1] = E + 3
    with pytest.raises(L.LloomHipError) as e:
        qt.indexed_moe_forward(x, _cuda(ids))
    assert e.value.name == "EEXPERT"
    y = qt.indexed_moe_forward(x, _cuda(ids), strict=False).cpu().numpy()
    assert np.all(y[2, 1] == 0)
    from lloom_amd.quantized import _ctx
    from lloom_amd.lib import lib

    assert lib().lloom_hip_ctx_sync(_ctx(0)) == 4
    good = ids.copy()
    good[2, 1] = 0
    got = qt.indexed_moe_forward(x, _cuda(good)).cpu().numpy()
    _rows_close(got, O.matmul_indexed(O.Q4K, qt.data(), E, n, k, x.cpu().numpy(), good.astype(np.uint32)),
                "after a bad id")


def test_moe_dma_graph_replays(L):
    """The routed call and the SwiGLU launch captured in a graph: every
    replay (eager calls of the other kernels in between) equals the eager
    result bit for bit; the kernel clears its own LDS counters, so nothing
    carries over from one replay to the next."""
    rng = np.random.default_rng(91)
    E, n, k, batch, topk = 16, 96, 2048, 4, 8
    qg = L.QTensor.quantize(_cuda((rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)), O.Q4K)
    qu = L.QTensor.quantize(_cuda((rng.standard_normal((E, n, k)) * 0.05).astype(np.float32)), O.Q4K)
    x = _cuda(rng.standard_normal((batch, 1, k)).astype(np.float32))
    ids = _cuda(_skewed_ids(rng, E, batch, topk, hot=2, hot_planes=10).astype(np.int32))
    y = torch.empty((batch, topk, n), device="cuda")
    yg = torch.empty_like(y)
    eager = qg.indexed_moe_forward_into(x, ids, y).clone()
    eager_glu = qg.indexed_moe_forward_glu_into(qu, x, ids, yg).clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            qg.indexed_moe_forward_into(x, ids, y)
            qg.indexed_moe_forward_glu_into(qu, x, ids, yg)
    torch.cuda.current_stream().wait_stream(s)
    other_ids = _cuda(rng.integers(0, E, (1, topk)).astype(np.int32))
    for i in range(3):
        y.fill_(float("nan"))
        yg.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager) and torch.equal(yg, eager_glu), i
        qu.indexed_moe_forward(x[:1], other_ids)  # eager work on the other routed kernel
        torch.cuda.synchronize()
