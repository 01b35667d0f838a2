"""lloom_hip_qmatmul_noalloc (the allocation-free variant of lloom_hip_qmatmul,
its workspace a static per-GPU device array) against lloom_hip_qmatmul,
through the C ABI: two calls in a row, the second smaller, every route
(decode dot4, MFMA decode with split K, the streaming decode kernel, the
prefill GEMMs), bit for bit the
allocating entry point's output and within the matmul bar of the oracle; a
call needing more than the scratch holds is refused by name."""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def L():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lloom_amd

    lloom_amd.lib()
    return lloom_amd


def _call(L, fn, qt, x, y):
    from lloom_amd.quantized import _ctx, _ptr, _stream

    n, k = qt.shape
    m = x.numel() // k
    a = 1 if x.dtype == torch.float16 else 0
    return fn(_ctx(0), int(qt.dtype), _ptr(qt.storage), n, k, _ptr(x), a, m, _ptr(y), a, _stream(x))


# (dtype, n, k, first m, second m): decode, split-K decode, prefill GEMMs,
# and the streaming decode kernel (a 28 MB Q4_K weight at 16 and 4 rows)
CASES = [(O.Q4K, 6144, 2048, 16, 1), (O.Q6K, 2048, 8192, 9, 4), (O.Q4K, 1024, 2048, 600, 40),
         (O.Q8_0, 512, 2048, 300, 7), (O.Q6K, 256, 4096, 200, 64), (O.Q4K, 12301, 4096, 16, 4)]


@pytest.mark.parametrize("dt,n,k,m1,m2", CASES)
def test_noalloc_matches_qmatmul(L, dt, n, k, m1, m2):
    lib = L.lib()
    rng = np.random.default_rng(n + m1)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    qt = L.QTensor.quantize(torch.from_numpy(w).to(DEV), dt)
    q = qt.data()
    for m in (m1, m2):
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV)
        ya = torch.empty((m, n), device=DEV)
        yb = torch.full((m, n), float("nan"), device=DEV)
        assert _call(L, lib.lloom_hip_qmatmul, qt, x, ya) == 0
        assert _call(L, lib.lloom_hip_qmatmul_noalloc, qt, x, yb) == 0, lib.lloom_hip_last_error()
        torch.cuda.synchronize()
        a, b = ya.cpu().numpy(), yb.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (dt, m)
        want = O.matmul(dt, x.cpu().numpy(), q, n)
        bound = 1e-3 * np.abs(want).max(axis=1, keepdims=True)
        assert np.all(np.abs(b - want) <= bound), (dt, m)


def test_noalloc_f16_and_refusal(L):
    lib = L.lib()
    rng = np.random.default_rng(5)
    n, k = 300, 1024
    qt = L.QTensor.quantize(torch.from_numpy((rng.standard_normal((n, k)) * 0.02).astype(np.float32)).to(DEV), O.Q4K)
    for m in (40, 3):
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(DEV)
        ya = torch.empty((m, n), device=DEV, dtype=torch.float16)
        yb = torch.empty((m, n), device=DEV, dtype=torch.float16)
        assert _call(L, lib.lloom_hip_qmatmul, qt, x, ya) == 0
        assert _call(L, lib.lloom_hip_qmatmul_noalloc, qt, x, yb) == 0
        torch.cuda.synchronize()
        assert torch.equal(ya, yb)
    # past the 32 MiB scratch: refused by name, nothing launched
    big_m = 8192
    x = torch.zeros((big_m, k), device=DEV, dtype=torch.float16)
    y = torch.zeros((big_m, n), device=DEV, dtype=torch.float16)
    assert _call(L, lib.lloom_hip_qmatmul_noalloc, qt, x, y) == 6
    assert b"static scratch" in lib.lloom_hip_last_error()
