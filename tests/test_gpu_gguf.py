"""GGUF file -> device QTensor (the load seam) on the GPU.

A file written by `gguf_file.write` from device QTensors is read back with
`Content.tensor(..., device)`: the uploaded blocks must be the written bytes
(tail pad included in the allocation), and a matmul, a routed matmul and an
embedding through the loaded tensors must equal, bit for bit, the same calls
through the tensors that were written (the same bytes through the same
kernels), and agree with the oracle.
"""
import io

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


def _cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def test_gguf_round_trip_to_device(L, tmp_path):
    from lloom_amd import gguf_file as G
    from lloom_amd.quantized import _padded_bytes

    D = L.GgmlDType
    rng = np.random.default_rng(11)
    w = {
        "blk.0.attn_q.weight": (D.Q4K, rng.standard_normal((96, 512)).astype(np.float32)),
        "blk.0.ffn_down.weight": (D.Q6K, rng.standard_normal((40, 768)).astype(np.float32)),
        "output.weight": (D.Q8_0, rng.standard_normal((72, 320)).astype(np.float32)),
        "blk.0.ffn_gate_exps.weight": (D.Q4K, rng.standard_normal((4, 24, 256)).astype(np.float32)),
        "token_embd.weight": (D.Q6K, rng.standard_normal((50, 256)).astype(np.float32)),
    }
    qts = {name: L.QTensor.quantize(_cuda(x), dt) for name, (dt, x) in w.items()}
    norm = rng.standard_normal(512).astype(np.float32)
    half = rng.standard_normal((3, 8)).astype(np.float16)
    qts["blk.0.attn_norm.weight"] = L.QTensor.from_data(norm.tobytes(), (512,), D.F32, device=DEV)
    qts["blk.0.f16.weight"] = L.QTensor.from_data(half.tobytes(), (3, 8), D.F16, device=DEV)
    md = [("general.architecture", G.Value(G.ValueType.String, "llama")),
          ("llama.block_count", G.Value(G.ValueType.U32, 1))]
    path = tmp_path / "m.gguf"
    with open(path, "wb") as f:
        G.write(f, md, list(qts.items()))

    with open(path, "rb") as f:
        c = G.Content.read(f)
        assert c.metadata["general.architecture"].to_string() == "llama"
        assert set(c.tensor_infos) == set(qts)
        c.validate_payloads(f)
        back = {name: c.tensor(f, name, device=DEV) for name in qts}

    for name, q in qts.items():
        b = back[name]
        assert b.shape == q.shape and b.dtype == q.dtype, name
        assert np.array_equal(b.data(), q.data()), name
        packed, alloc = _padded_bytes(q.dtype, int(np.prod(q.shape[:-1])), q.shape[-1])
        assert b.storage.numel() == alloc and not b.storage[packed:].any().item(), name
    assert np.array_equal(back["blk.0.attn_norm.weight"].dequantize().cpu().numpy(), norm)
    assert np.array_equal(back["blk.0.f16.weight"].dequantize_f16().cpu().numpy().view(np.uint16),
                          half.view(np.uint16))

    for name in ("blk.0.attn_q.weight", "blk.0.ffn_down.weight", "output.weight"):
        q, b = qts[name], back[name]
        n, k = q.shape
        for m in (1, 5, 80):
            x = _cuda(rng.standard_normal((m, k)).astype(np.float32))
            ya = L.QMatMul.from_qtensor(q).forward(x)
            yb = L.QMatMul.from_qtensor(b).forward(x)
            assert torch.equal(ya, yb), (name, m)
        want = O.matmul(q.dtype, x.cpu().numpy(), q.data(), n)
        got = yb.cpu().numpy()
        assert np.all(np.abs(got - want) <= 1e-3 * np.abs(want).max(axis=1, keepdims=True) + 1e-30), name

    ex = "blk.0.ffn_gate_exps.weight"
    x = _cuda(rng.standard_normal((3, 1, 256)).astype(np.float32))
    ids = _cuda(np.array([[0, 3], [2, 2], [1, 0]], dtype=np.int32))
    assert torch.equal(qts[ex].indexed_moe_forward(x, ids), back[ex].indexed_moe_forward(x, ids))

    emb = "token_embd.weight"
    tok = _cuda(np.array([[0, 49, 7]], dtype=np.int32))
    assert torch.equal(qts[emb].embedding(tok), back[emb].embedding(tok))

    with pytest.raises(L.LloomHipError, match="not a quantized matmul"):
        L.QMatMul.from_qtensor(back["blk.0.f16.weight"])
