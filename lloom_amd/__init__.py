"""lloom_amd -- MI355X (gfx950) quantized-weight matmul for lloom.

The compute lives in ``liblloom_hip.so`` (hand-written HIP kernels behind the
C ABI of ``include/lloom_hip.h``).  This package is the host-side mirror of
lloom-tensor's ``quantized`` surface (``QTensor``, ``QMatMul``,
``GgmlDType``; lloom-tensor/src/quantized/mod.rs) over that ABI, used by the
tests and the benchmark.  PyTorch only provides device memory and streams.
There is no CPU fallback: without the built library every call raises.
"""
from .lib import LloomHipError, lib, lib_path  # noqa: F401
from . import gguf_file  # noqa: F401
from .quantized import (  # noqa: F401
    GgmlDType,
    MoeArm,
    MvStore,
    QMatMul,
    QTensor,
    dequantize,
    quantize_act,
    synth_normal,
    synth_uniform,
)
