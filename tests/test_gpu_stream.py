"""GPU parity of the streaming Q4_K decode kernel (k_mv_stream: weights of
24 MB and more, 2..16 activation rows at k = 4096, 6144 or 8192, 2..4
at k = 2048)
against the CPU oracle, through the C ABI.

Bar: max|d| <= 1e-3 * max|y row|, as every
other matmul test; the kernel's integer sums are k_quants.rs:1540-1620's.
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


def _rows_close(got, want, what):
    bound = MATMUL_TOL * np.abs(want).max(axis=1, keepdims=True) + 1e-30
    err = np.abs(np.asarray(got, np.float64) - want)
    assert not (err > bound).any(), f"{what}: worst ratio {(err / bound).max():.3g}"


def _weights(seed, n, k):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[3, :256] = 0.0            # an all-zero superblock (d = dmin = 0)
    w[n - 1, 256:512] += 0.5    # a superblock with a large offset (dmin term)
    return w


def _x(seed, m, k):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if m > 2:
        x[1, :256] = 0.0          # an all-zero activation block
        x[2] = 1.0 + 0.05 * x[2]  # same-sign row: large sub-block sums
    return x


# (n, k, m): every k the kernel takes (S = k / 2048 superblocks a wave) and
# each row-count rule, with n not a multiple of 16 (the last tile is shifted
# back and stores only its new rows)
CASES = [(43701, 2048, 2), (43701, 2048, 4), (12301, 4096, 4), (12301, 4096, 16), (8200, 6144, 5),
         (8200, 6144, 16), (5470, 8192, 16), (21847, 8192, 2), (21847, 8192, 3)]


@pytest.mark.parametrize("n,k,m", CASES)
def test_stream_matches_oracle(L, n, k, m):
    w = _weights(n + k, n, k)
    qt = L.QTensor.quantize(torch.from_numpy(w).cuda(), L.GgmlDType.Q4K)
    mib = qt.packed_bytes() / 2**20
    assert mib >= (48 if k == 2048 else 96 if m < 4 else 24)
    x = _x(m * 7 + k, m, k)
    y = L.QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    _rows_close(y, O.matmul(O.Q4K, x, qt.data(), n), f"stream n={n} k={k} m={m}")


def test_stream_rows_batch_invariant_and_repeatable(L):
    """Each activation row is computed on its own and the eight waves'
    partial sums meet in a fixed order: a row's output is the same bits in
    a batch of 4 or of 16, and from call to call."""
    n, k = 5470, 8192
    w = _weights(5, n, k)
    qt = L.QTensor.quantize(torch.from_numpy(w).cuda(), L.GgmlDType.Q4K)
    mm = L.QMatMul.from_qtensor(qt)
    x = torch.from_numpy(_x(9, 16, k)).cuda()
    full = mm.forward(x).cpu().numpy()
    again = mm.forward(x).cpu().numpy()
    assert np.array_equal(full.view(np.uint32), again.view(np.uint32))
    for r in (0, 5, 12):
        four = mm.forward(x[r:r + 4].contiguous()).cpu().numpy()
        assert np.array_equal(four.view(np.uint32), full[r:r + 4].view(np.uint32)), f"rows {r}..{r + 3}"


def test_stream_epilogues(L):
    """QMatMul::forward_silu / forward_mul_into (mod.rs:2102-2156) on the
    streaming kernel: the stored value is silu(v) (resp. gate * v) of the sum
    the plain forward stores."""
    n, k, m = 12301, 4096, 4
    w = _weights(11, n, k)
    qt = L.QTensor.quantize(torch.from_numpy(w).cuda(), L.GgmlDType.Q4K)
    mm = L.QMatMul.from_qtensor(qt)
    x = torch.from_numpy(_x(12, m, k)).cuda()
    plain = mm.forward(x).cpu().numpy()
    silu = mm.forward_silu(x).cpu().numpy()
    ref = (plain / (np.float32(1.0) + np.exp(-plain))).astype(np.float32)
    np.testing.assert_allclose(silu, ref, rtol=2e-6, atol=1e-7)
    gate = np.random.default_rng(3).standard_normal((m, n)).astype(np.float32)
    g = torch.from_numpy(gate).cuda()
    mm.forward_mul_into(x, g)
    assert np.array_equal(g.cpu().numpy().view(np.uint32), (gate * plain).astype(np.float32).view(np.uint32))


def test_stream_graph_replays(L):
    """The streaming decode call captured in a graph: every replay (eager
    calls of other shapes in between) equals the eager result bit for bit;
    the kernel's LDS counters are cleared by the kernel itself."""
    n, k, m = 12301, 4096, 8
    qt = L.QTensor.quantize(torch.from_numpy(_weights(21, n, k)).cuda(), L.GgmlDType.Q4K)
    mm = L.QMatMul.from_qtensor(qt)
    x = torch.from_numpy(_x(22, m, k)).cuda()
    y = torch.empty((m, n), device="cuda")
    eager = mm.forward_into(x, y).clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            mm.forward_into(x, y)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i
        mm.forward(x[: 2 + i])  # eager calls on the other decode kernels
        torch.cuda.synchronize()
