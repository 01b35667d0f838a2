"""Writes tests/golden/kquants_golden.npz: inputs and expected outputs of the
quantized path on the reference's own test inputs, computed by the pinned
oracle.  Run from the repository root:  python tests/golden/make_golden.py

Inputs (lloom-tensor/tests/quantized_tests.rs):
  * stdrng_*: get_random_tensors(11, 512, 21) with StdRng::seed_from_u64(
    314159265358979) (:1267-1287), the inputs of quantized_matmul_q4k/q6k
    (:1441-1542), whose published 3-decimal picks are stored beside the
    full outputs;
  * closed_*: the prompt-GEMM closed form of :1769-1903 (m = 17, n = 7,
    k = 768);
  * ggml_*: create_ggml_like_vector(0.0) (:527-532), the quantization tests'
    input;
  * indexed_*: a 4-expert routed case (in_dim1 = 1 and = topk).
Everything is plain arrays (np.savez_compressed, no pickles).
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402
from tests.stdrng import StdRng  # noqa: E402

TYPES = {"q8_0": O.Q8_0, "q4k": O.Q4K, "q6k": O.Q6K}
PUBLISHED = {"q4k": [1.094, 1.442, -0.196, 1.587], "q6k": [1.293, 1.497, -0.159, 1.737]}  # :1460, :1514


def build():
    out = {}
    rng = StdRng(314159265358979)
    lhs = (rng.random_f32(11 * 512) - np.float32(0.5)).astype(np.float32).reshape(11, 512)
    rhs = (rng.random_f32(21 * 512) - np.float32(0.5)).astype(np.float32).reshape(21, 512)
    out["stdrng_lhs"], out["stdrng_rhs"] = lhs, rhs
    for name, dt in TYPES.items():
        q = O.quantize(dt, rhs.ravel())
        out[f"stdrng_{name}_w"] = q
        out[f"stdrng_{name}_y"] = O.matmul(dt, lhs, q, 21)
        if name in PUBLISHED:
            out[f"stdrng_{name}_published"] = np.array(PUBLISHED[name], dtype=np.float64)

    m, n, k = 17, 7, 768
    lhs = (((np.arange(m * k) * 17 % 211).astype(np.float32) - np.float32(103)) / np.float32(73)).astype(np.float32)
    wts = (((np.arange(n * k) * 31 % 173).astype(np.float32) - np.float32(87)) / np.float32(61)).astype(np.float32)
    out["closed_x"], out["closed_wf"] = lhs.reshape(m, k), wts.reshape(n, k)
    for name, dt in TYPES.items():
        q = O.quantize(dt, wts)
        out[f"closed_{name}_w"] = q
        out[f"closed_{name}_y"] = O.matmul(dt, lhs.reshape(m, k), q, n)

    i = np.arange(32 * 128, dtype=np.float32)
    g = (np.float32(0.1) + np.float32(2.0) * np.cos(i)).astype(np.float32)
    out["ggml_x"] = g
    for name, dt in list(TYPES.items()) + [("q8k", O.Q8K)]:
        q = O.quantize(dt, g)
        out[f"ggml_{name}_q"] = q
        out[f"ggml_{name}_deq"] = O.dequantize(dt, q, g.size)

    r = np.random.default_rng(5)
    E, n, k, batch, topk = 4, 16, 256, 3, 2
    wf = (r.standard_normal(E * n * k) * 0.05).astype(np.float32)
    ids = np.array([[0, 3], [2, 2], [1, 0]], dtype=np.uint32)
    out["indexed_wf"], out["indexed_ids"] = wf.reshape(E, n, k), ids
    out["indexed_x1"] = r.standard_normal((batch, 1, k)).astype(np.float32)
    out["indexed_xt"] = r.standard_normal((batch, topk, k)).astype(np.float32)
    for name, dt in TYPES.items():
        q = O.quantize(dt, wf)
        out[f"indexed_{name}_w"] = q
        out[f"indexed_{name}_y1"] = O.matmul_indexed(dt, q, E, n, k, out["indexed_x1"], ids)
        out[f"indexed_{name}_yt"] = O.matmul_indexed(dt, q, E, n, k, out["indexed_xt"], ids)
    return out


if __name__ == "__main__":
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kquants_golden.npz")
    np.savez_compressed(path, **build())
    print(path, os.path.getsize(path), "bytes")
