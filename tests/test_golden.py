"""The committed golden fixtures (tests/golden/kquants_golden.npz, written by
tests/golden/make_golden.py on the inputs of lloom-tensor/tests/
quantized_tests.rs) against the oracle on the CPU and the HIP path on the GPU.

On the CPU: the oracle still reproduces every fixture bit for bit, and its
quantized matmul on the reference's StdRng inputs still gives the published
3-decimal picks.  On the GPU (through the C ABI): weight and activation
quantization and dequantization bit-exact with the fixture bytes, matmuls
within 1e-3 of the fixture row maximum, the routed matmuls within the same
bar, and the published picks reproduced by the GPU's own outputs.
"""
import os

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
TYPES = {"q8_0": O.Q8_0, "q4k": O.Q4K, "q6k": O.Q6K}
MATMUL_TOL = 1e-3


@pytest.fixture(scope="module")
def G():
    with np.load(os.path.join(HERE, "golden", "kquants_golden.npz")) as d:
        return {k: d[k] for k in d.files}


def picks(y, m, n):
    f = np.asarray(y, dtype=np.float32).ravel()
    return [round(float(v) * 1000.0) / 1000.0 for v in (f[0], f[m * n // 3], f[m * n * 2 // 3], f[m * n - 1])]


def rows_close(got, want, tol=MATMUL_TOL):
    got = np.asarray(got, np.float64).reshape(-1, want.shape[-1])
    want = np.asarray(want, np.float64).reshape(-1, want.shape[-1])
    bound = tol * np.abs(want).max(axis=1, keepdims=True) + 1e-30
    return bool((np.abs(got - want) <= bound).all())


# ------------------------------------------------------------ CPU side ---

@pytest.mark.parametrize("name", sorted(TYPES))
def test_oracle_reproduces_fixtures(G, name):
    dt = TYPES[name]
    q = O.quantize(dt, G["stdrng_rhs"].ravel())
    assert np.array_equal(q, G[f"stdrng_{name}_w"])
    y = O.matmul(dt, G["stdrng_lhs"], q, 21)
    assert np.array_equal(y.view(np.uint32), G[f"stdrng_{name}_y"].view(np.uint32))
    q = O.quantize(dt, G["closed_wf"].ravel())
    assert np.array_equal(q, G[f"closed_{name}_w"])
    y = O.matmul(dt, G["closed_x"], q, 7)
    assert np.array_equal(y.view(np.uint32), G[f"closed_{name}_y"].view(np.uint32))
    q = O.quantize(dt, G["ggml_x"])
    assert np.array_equal(q, G[f"ggml_{name}_q"])
    assert np.array_equal(O.dequantize(dt, q, 4096).view(np.uint32), G[f"ggml_{name}_deq"].view(np.uint32))
    E, n, k = G["indexed_wf"].shape
    q = O.quantize(dt, G["indexed_wf"].ravel())
    for xs in ("1", "t"):
        y = O.matmul_indexed(dt, q, E, n, k, G[f"indexed_x{xs}"], G["indexed_ids"])
        assert np.array_equal(y.view(np.uint32), G[f"indexed_{name}_y{xs}"].view(np.uint32))


def test_oracle_q8k_fixture(G):
    q = O.quantize(O.Q8K, G["ggml_x"])
    assert np.array_equal(q, G["ggml_q8k_q"])


@pytest.mark.parametrize("name", ["q4k", "q6k"])
def test_fixture_outputs_give_the_published_picks(G, name):
    """quantized_tests.rs:1460 (Q4K) and :1514 (Q6K)."""
    assert picks(G[f"stdrng_{name}_y"], 11, 21) == list(G[f"stdrng_{name}_published"])


# ------------------------------------------------------------ GPU side ---

@pytest.fixture(scope="module")
def L():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lloom_amd

    lloom_amd.lib()
    return lloom_amd


def _cuda(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(TYPES))
def test_gpu_quantize_dequantize_match_fixtures(L, G, name):
    dt = TYPES[name]
    for key, w in (("stdrng", G["stdrng_rhs"]), ("closed", G["closed_wf"])):
        got = L.QTensor.quantize(_cuda(w), dt).data()
        assert np.array_equal(got, G[f"{key}_{name}_w"]), key
    q = L.QTensor.quantize(_cuda(G["ggml_x"].reshape(2, 2048)), dt)
    assert np.array_equal(q.data(), G[f"ggml_{name}_q"])
    deq = q.dequantize().cpu().numpy().ravel()
    assert np.array_equal(deq.view(np.uint32), G[f"ggml_{name}_deq"].view(np.uint32))


@pytest.mark.gpu
def test_gpu_activation_quantizer_matches_fixture(L, G):
    got = L.quantize_act(_cuda(G["ggml_x"].reshape(1, 4096)), O.Q8K).cpu().numpy()
    assert np.array_equal(got.ravel(), G["ggml_q8k_q"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(TYPES))
def test_gpu_matmul_matches_fixtures(L, G, name):
    dt = TYPES[name]
    for key, n in (("stdrng", 21), ("closed", 7)):
        x = G["stdrng_lhs"] if key == "stdrng" else G["closed_x"]
        w = G["stdrng_rhs"] if key == "stdrng" else G["closed_wf"]
        q = L.QTensor.quantize(_cuda(w), dt)
        want = G[f"{key}_{name}_y"]
        y = L.QMatMul.from_qtensor(q).forward(_cuda(x)).cpu().numpy()
        assert rows_close(y, want), key
        for r in range(x.shape[0]):  # every row alone: the decode routes
            yr = L.QMatMul.from_qtensor(q).forward(_cuda(x[r:r + 1])).cpu().numpy()
            assert rows_close(yr, want[r:r + 1]), (key, r)
        if key == "stdrng" and f"stdrng_{name}_published" in G:
            assert picks(y, 11, 21) == list(G[f"stdrng_{name}_published"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(TYPES))
def test_gpu_routed_matmul_matches_fixtures(L, G, name):
    dt = TYPES[name]
    q = L.QTensor.quantize(_cuda(G["indexed_wf"]), dt)
    ids = _cuda(G["indexed_ids"].astype(np.int32))
    for xs in ("1", "t"):
        got = q.indexed_moe_forward(_cuda(G[f"indexed_x{xs}"]), ids).cpu().numpy()
        assert rows_close(got, G[f"indexed_{name}_y{xs}"]), xs
