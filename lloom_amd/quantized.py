"""Host mirror of lloom-tensor's quantized surface on the HIP arm.

Names, argument meaning and refusals follow lloom-tensor/src/quantized/mod.rs:
  GgmlDType            mod.rs:404-437, ids mod.rs:505-568
  QTensor.quantize     mod.rs:919-938   (QStorage::quantize on the device)
  QTensor.from_data    mod.rs:136-223   (QStorage::from_data: an upload)
  QTensor.dequantize   mod.rs:1065-1086 (and dequantize_f16)
  QTensor.indexed_moe_forward{,_with,_as}  mod.rs:1560-1645
  QTensor.indexed_moe_forward_pair{,_with,_as} / _glu_as  mod.rs:1365-1531
  QTensor.embedding    mod.rs:1101-1137
  QMatMul.from_qtensor / forward          mod.rs:1698-1729, 2022-2025
  QMatMul.forward_silu / forward_mul_into, MvStore  mod.rs:1667-1696, 2102-2156
  MoeArm               mod.rs:2290-2310
F32 / F16 / BF16 QTensors (norms and biases a GGUF file holds) are uploaded
as is and dequantize by reinterpretation; they are not matmul weights here.
Tensors are torch tensors on the GPU (device memory and streams only); the
arithmetic is the C ABI's.
"""
import ctypes
import enum
import threading

import numpy as np
import torch

from .lib import LloomHipError, check, lib


class GgmlDType(enum.IntEnum):
    F32 = 0
    F16 = 1
    Q8_0 = 8
    Q4K = 12
    Q6K = 14
    Q8K = 15
    BF16 = 30

    def block_size(self):
        return {GgmlDType.F32: 1, GgmlDType.F16: 1, GgmlDType.BF16: 1, GgmlDType.Q8_0: 32}.get(self, 256)

    def type_size(self):
        return {GgmlDType.F32: 4, GgmlDType.F16: 2, GgmlDType.BF16: 2, GgmlDType.Q8_0: 34, GgmlDType.Q4K: 144,
                GgmlDType.Q6K: 210, GgmlDType.Q8K: 292}[self]

    def is_float(self):
        return self in (GgmlDType.F32, GgmlDType.F16, GgmlDType.BF16)

    def vec_dot_type(self):
        return GgmlDType.Q8_0 if self == GgmlDType.Q8_0 else GgmlDType.Q8K


class MoeArm(enum.Enum):
    """The kernel family of a routed matmul (mod.rs:2290-2310).  The HIP arm
    has one kernel (f32 dots, as the CPU arm) and, like the CPU and CUDA
    arms, ignores it; it is kept so callers pass it unchanged."""
    MatVec = 0
    Gemm = 1

    @staticmethod
    def for_rows(rows, mm_from=64):
        return MoeArm.Gemm if mm_from > 0 and rows >= mm_from else MoeArm.MatVec


# ------------------------------------------------------------- context --

_ctx_lock = threading.Lock()
_ctxs = {}


def _ctx(device_index):
    with _ctx_lock:
        c = _ctxs.get(device_index)
        if c is None:
            p = ctypes.c_void_p()
            check(lib().lloom_hip_ctx_create(device_index, ctypes.byref(p)))
            c = p.value
            _ctxs[device_index] = c
        return c


def _dev_index(t):
    if not t.is_cuda:
        raise LloomHipError(1, "tensor is not on a HIP device")
    return t.device.index if t.device.index is not None else torch.cuda.current_device()


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


_ACT_IDS = {torch.float32: 0, torch.float16: 1}


def _act_id(dtype, what):
    if dtype not in _ACT_IDS:
        raise LloomHipError(2, f"{what}: {dtype} is not an activation dtype of the HIP arm (F32 or F16)")
    return _ACT_IDS[dtype]


def _cast(t, dtype):
    """Tensor::to_dtype between f32 and f16 on the device (RNE), through the
    C ABI; the same tensor when it already has that dtype."""
    if t.dtype == dtype:
        return t
    src_id, dst_id = _act_id(t.dtype, "cast"), _act_id(dtype, "cast")
    t = t.contiguous()
    out = torch.empty(t.shape, dtype=dtype, device=t.device)
    check(lib().lloom_hip_cast(_ctx(_dev_index(t)), _ptr(t), src_id, _ptr(out), dst_id, t.numel(), _stream(t)))
    return out


def _check_out(y, shape, dtype, device, what):
    """A caller's output buffer: contiguous, of the call's dtype, shape and device."""
    if (not isinstance(y, torch.Tensor) or y.dtype != dtype or not y.is_contiguous() or y.device != device
            or y.numel() != int(np.prod(shape))):
        raise LloomHipError(3, f"{what}: y {tuple(getattr(y, 'shape', ()))} {getattr(y, 'dtype', None)} does not "
                               f"fit the contiguous {dtype} output {tuple(shape)} on {device}")


def reserve_workspace(nbytes, device=0):
    """Grow the device context's workspace now (before a graph capture)."""
    check(lib().lloom_hip_ctx_reserve(_ctx(device), int(nbytes)))


def qmatmul_workspace_bytes(dtype, n, k, m, x_dtype=torch.float32, y_dtype=torch.float32, device=0):
    out = ctypes.c_size_t()
    check(lib().lloom_hip_qmatmul_workspace_bytes(_ctx(device), int(GgmlDType(dtype)), n, k, m,
                                                  _act_id(x_dtype, "workspace"), _act_id(y_dtype, "workspace"),
                                                  ctypes.byref(out)))
    return out.value


def set_mv_rows_max(rows, device=0):
    check(lib().lloom_hip_ctx_set_mv_rows_max(_ctx(device), rows))


MMA_F16, MMA_INT8, MMA_AUTO = 0, 1, 2


def set_prefill_mma(mode, device=0):
    """Matrix-core family of the Q4_K prefill GEMM: MMA_F16 (the exact
    integer operands on fp16 MFMA), MMA_INT8 (two int8 scale planes) or
    MMA_AUTO (the default: F16 up to 320 rows, INT8 past).  All compute the
    CPU arm's integer sums exactly."""
    check(lib().lloom_hip_ctx_set_prefill_mma(_ctx(device), mode))


class MvStore(enum.IntEnum):
    """The matmul's store block (MvStore, mod.rs:1667-1696): the value
    stored is silu(v) or y * v instead of v (LLOOM_HIP_STORE_*)."""
    Silu = 1
    MulInto = 2


# ------------------------------------------------------------ QTensor ---

_FLOAT_TORCH = {GgmlDType.F32: torch.float32, GgmlDType.F16: torch.float16, GgmlDType.BF16: torch.bfloat16}


def _padded_bytes(dtype, n_rows, k):
    if dtype.is_float():
        # Unblocked storage (norms, biases): read by reinterpretation, no kernel tail pad.
        b = n_rows * k * dtype.type_size()
        return b, b
    packed, alloc = ctypes.c_size_t(), ctypes.c_size_t()
    check(lib().lloom_hip_weight_bytes(int(dtype), n_rows, k, ctypes.byref(packed), ctypes.byref(alloc)))
    return packed.value, alloc.value


class QTensor:
    """Packed GGUF blocks in device memory with a logical shape whose last
    dimension is k (a multiple of the block size)."""

    def __init__(self, storage, shape, dtype):
        self.storage = storage  # torch.uint8 on the GPU, with the tail pad
        self.shape = tuple(int(s) for s in shape)
        self.dtype = GgmlDType(dtype)

    # QTensor::quantize (mod.rs:919-938); check_shape (mod.rs:900-907)
    @staticmethod
    def quantize(src, dtype):
        dtype = GgmlDType(dtype)
        if dtype.is_float():
            raise LloomHipError(2, f"{dtype.name} is not a block type on the HIP quantized path")
        shape = tuple(src.shape)
        bs = dtype.block_size()
        if len(shape) == 0 or shape[-1] % bs:
            raise LloomHipError(3, f"quantized tensor must have their last dim divisible by block size {shape} {bs}")
        src = src.to(torch.float32).contiguous()
        elems = src.numel()
        packed, alloc = _padded_bytes(dtype, elems // shape[-1], shape[-1])
        storage = torch.zeros(alloc, dtype=torch.uint8, device=src.device)
        check(lib().lloom_hip_quantize(_ctx(_dev_index(src)), int(dtype), _ptr(src), elems, _ptr(storage),
                                       _stream(src)))
        return QTensor(storage, shape, dtype)

    # QStorage::from_data (mod.rs:136-223): raw GGUF bytes, uploaded as is
    @staticmethod
    def from_data(data, shape, dtype, device="cuda"):
        dtype = GgmlDType(dtype)
        shape = tuple(shape)
        buf = np.frombuffer(bytes(data) if not isinstance(data, np.ndarray) else data.tobytes(), dtype=np.uint8)
        packed, alloc = _padded_bytes(dtype, int(np.prod(shape[:-1])), shape[-1])
        if buf.size != packed:
            raise LloomHipError(3, f"{buf.size} bytes do not hold a {dtype.name} tensor of shape {shape} ({packed} bytes)")
        storage = torch.zeros(alloc, dtype=torch.uint8, device=device)
        storage[:packed].copy_(torch.from_numpy(buf.copy()))
        return QTensor(storage, shape, dtype)

    def packed_bytes(self):
        return _padded_bytes(self.dtype, int(np.prod(self.shape[:-1])), self.shape[-1])[0]

    def data(self):
        """The packed GGUF bytes (numpy uint8)."""
        return self.storage[:self.packed_bytes()].cpu().numpy()

    def elem_count(self):
        return int(np.prod(self.shape))

    def _dequant(self, out_dtype, torch_dtype):
        if self.dtype.is_float():
            # F32 / F16 / BF16 storage: a reinterpretation, then a conversion
            return self.storage[:self.packed_bytes()].view(_FLOAT_TORCH[self.dtype]).reshape(self.shape) \
                .to(torch_dtype)
        y = torch.empty(self.shape, dtype=torch_dtype, device=self.storage.device)
        check(lib().lloom_hip_dequantize(_ctx(_dev_index(self.storage)), int(self.dtype), _ptr(self.storage),
                                         self.elem_count(), _ptr(y), out_dtype, _stream(self.storage)))
        return y

    def dequantize(self):
        return self._dequant(0, torch.float32)

    def dequantize_f16(self):
        return self._dequant(1, torch.float16)

    # indexed_moe_forward{,_with,_as} (mod.rs:1370-1645); the arm is ignored
    def _moe_shapes(self, x, ids, what="indexed_moe_forward"):
        if len(self.shape) != 3:
            raise LloomHipError(3, f"{what}: weight {self.shape} is not [experts, n, k]")
        n_experts, n, k = self.shape
        if x.dim() != 3 or ids.dim() != 2:
            raise LloomHipError(3, f"{what}: x {tuple(x.shape)} / ids {tuple(ids.shape)} do not fit weight {self.shape}")
        batch, in_dim1, k_in = x.shape
        batch_ids, topk = ids.shape
        if k_in != k or batch != batch_ids or (in_dim1 != 1 and in_dim1 != topk):
            raise LloomHipError(3, f"{what}: x {tuple(x.shape)} / ids {tuple(ids.shape)} do not fit weight {self.shape}")
        return n_experts, n, k, batch, in_dim1, topk

    @staticmethod
    def _moe_x(x, act):
        """x as the CPU arm reads it: cast to `act` first when it differs
        (mod.rs:1567-1571), then to f32 (mod.rs:1627), contiguous."""
        act = x.dtype if act is None else act
        _act_id(act, "indexed_moe_forward_as")
        _act_id(x.dtype, "indexed_moe_forward_as")
        return _cast(_cast(x, act), torch.float32).contiguous()

    def indexed_moe_forward_as(self, x, ids, arm=None, act=None, strict=True):
        """What indexed_moe_forward computes for x cast to `act` (torch.float32
        or torch.float16; None: x's own dtype), bit for bit (mod.rs:1560-1575):
        an f32 x with act f16 is rounded to f16 first.  y is f32
        [batch, topk, n], as the CPU arm returns it."""
        n_experts, n, k, batch, in_dim1, topk = self._moe_shapes(x, ids)
        x = self._moe_x(x, act)
        ids = ids.to(torch.int32).contiguous()
        y = torch.empty((batch, topk, n), dtype=torch.float32, device=x.device)
        check(lib().lloom_hip_moe_matmul(_ctx(_dev_index(x)), int(self.dtype), _ptr(self.storage), n_experts, n,
                                         k, _ptr(x), batch, in_dim1, _ptr(ids), topk, _ptr(y), 1 if strict else 0,
                                         _stream(x)))
        return y

    def indexed_moe_forward(self, x, ids, arm=None, strict=True):
        return self.indexed_moe_forward_as(x, ids, arm, None, strict)

    indexed_moe_forward_with = indexed_moe_forward

    def _moe_into_check(self, x, ids, y, shape_of_y):
        if x.dtype != torch.float32 or not x.is_contiguous():
            raise LloomHipError(2, f"indexed_moe_forward_into: x must be contiguous f32, got {x.dtype}")
        if ids.dtype != torch.int32 or not ids.is_contiguous() or ids.device != x.device:
            raise LloomHipError(2, "indexed_moe_forward_into: ids must be contiguous int32 on x's device")
        if x.device != self.storage.device:
            raise LloomHipError(1, "indexed_moe_forward_into: x is not on the weight's device")
        _check_out(y, shape_of_y, torch.float32, x.device, "indexed_moe_forward_into")

    def indexed_moe_forward_into(self, x, ids, y):
        """indexed_moe_forward into a preallocated contiguous f32 y
        [batch, topk, n] (x contiguous f32, ids contiguous int32, all on the
        weight's device); non-strict (no stream sync), so it can be captured
        in a graph; lloom_hip_ctx_sync reports a bad id afterwards."""
        n_experts, n, k, batch, in_dim1, topk = self._moe_shapes(x, ids)
        self._moe_into_check(x, ids, y, (batch, topk, n))
        check(lib().lloom_hip_moe_matmul(_ctx(_dev_index(x)), int(self.dtype), _ptr(self.storage), n_experts, n,
                                         k, _ptr(x), batch, in_dim1, _ptr(ids), topk, _ptr(y), 0, _stream(x)))
        return y

    def _moe_check(self, up, x, ids):
        if len(self.shape) != 3:
            raise LloomHipError(3, f"indexed_moe_forward: weight {self.shape} is not [experts, n, k]")
        if up.dtype != self.dtype or up.shape != self.shape:
            raise LloomHipError(3, f"indexed_moe_forward_pair: gate {self.dtype.name}{list(self.shape)} and "
                                   f"up {up.dtype.name}{list(up.shape)} differ")
        return self._moe_shapes(x, ids)

    def indexed_moe_forward_pair_as(self, up, x, ids, arm=None, act=None, strict=True):
        """Gate and up of one routed layer in ONE launch (the reference's
        Metal kernel_mul_mv_id2, mod.rs:1365-1455), computed in `act`: each
        half is bit for bit what indexed_moe_forward_as computes for it."""
        n_experts, n, k, batch, in_dim1, topk = self._moe_check(up, x, ids)
        x = self._moe_x(x, act)
        ids = ids.to(torch.int32).contiguous()
        yg = torch.empty((batch, topk, n), dtype=torch.float32, device=x.device)
        yu = torch.empty_like(yg)
        check(lib().lloom_hip_moe_matmul_pair(_ctx(_dev_index(x)), int(self.dtype), _ptr(self.storage),
                                              _ptr(up.storage), n_experts, n, k, _ptr(x), batch, in_dim1, _ptr(ids),
                                              topk, _ptr(yg), _ptr(yu), 1 if strict else 0, _stream(x)))
        return yg, yu

    def indexed_moe_forward_pair(self, up, x, ids, arm=None, strict=True):
        return self.indexed_moe_forward_pair_as(up, x, ids, arm, None, strict)

    indexed_moe_forward_pair_with = indexed_moe_forward_pair

    def indexed_moe_forward_glu_as(self, up, x, ids, arm=None, act=None, strict=True):
        """silu(gate) * up of indexed_moe_forward_pair_as's halves in ONE
        launch (mod.rs:1457-1531), computed in `act` (x rounded to f16 first
        when act is f16 and x is not).  The reference returns None off Metal
        and the caller composes; here the fused launch always serves, with y
        f32 as the CPU arm's halves are."""
        n_experts, n, k, batch, in_dim1, topk = self._moe_check(up, x, ids)
        x = self._moe_x(x, act)
        ids = ids.to(torch.int32).contiguous()
        y = torch.empty((batch, topk, n), dtype=torch.float32, device=x.device)
        check(lib().lloom_hip_moe_matmul_glu(_ctx(_dev_index(x)), int(self.dtype), _ptr(self.storage),
                                             _ptr(up.storage), n_experts, n, k, _ptr(x), batch, in_dim1, _ptr(ids),
                                             topk, _ptr(y), 1 if strict else 0, _stream(x)))
        return y

    def indexed_moe_forward_glu_into(self, up, x, ids, y):
        """indexed_moe_forward_glu_as into a preallocated contiguous f32 y
        [batch, topk, n]; non-strict and allocation-free (graph-capturable)."""
        n_experts, n, k, batch, in_dim1, topk = self._moe_check(up, x, ids)
        self._moe_into_check(x, ids, y, (batch, topk, n))
        check(lib().lloom_hip_moe_matmul_glu(_ctx(_dev_index(x)), int(self.dtype), _ptr(self.storage),
                                             _ptr(up.storage), n_experts, n, k, _ptr(x), batch, in_dim1, _ptr(ids),
                                             topk, _ptr(y), 0, _stream(x)))
        return y

    # QTensor::embedding (mod.rs:1101-1137)
    def embedding(self, ids, strict=True, f16=False):
        """Rows ids of a [rows, hidden] weight, dequantized: out shape
        ids.shape + (hidden,), f32 (or f16, the RNE of the f32 value)."""
        if len(self.shape) != 2:
            raise LloomHipError(3, f"embedding: weight {self.shape} is not [rows, hidden]")
        rows, hidden = self.shape
        bs = self.dtype.block_size()
        if hidden % bs:
            raise LloomHipError(3, f"quantized embedding hidden size {hidden} is not divisible by block size {bs}")
        out_shape = tuple(ids.shape) + (hidden,)
        flat = ids.to(device=self.storage.device, dtype=torch.int32).reshape(-1).contiguous()
        y = torch.empty(out_shape, dtype=torch.float16 if f16 else torch.float32, device=self.storage.device)
        check(lib().lloom_hip_embedding(_ctx(_dev_index(self.storage)), int(self.dtype), _ptr(self.storage), rows,
                                        hidden, _ptr(flat), flat.numel(), _ptr(y), 1 if f16 else 0,
                                        1 if strict else 0, _stream(self.storage)))
        return y

    def __repr__(self):
        return f"QTensor[{list(self.shape)}; {self.dtype.name}]"


# ------------------------------------------------------------ QMatMul ---

class QMatMul:
    """QMatMul::QTensor (mod.rs:1698-1729): forward(x) = x . W^T with W
    packed.  x is [.., k] f32 (rank >= 2, contiguous); the result is [.., n]."""

    def __init__(self, qtensor):
        if len(qtensor.shape) != 2:
            raise LloomHipError(3, f"QMatMul weight must be [n, k], got {qtensor.shape}")
        if qtensor.dtype.is_float() or qtensor.dtype == GgmlDType.Q8K:
            raise LloomHipError(2, f"QMatMul over a {qtensor.dtype.name} weight is not a quantized matmul "
                                   f"(the HIP arm multiplies Q8_0, Q4K, Q6K)")
        self.qtensor = qtensor

    @staticmethod
    def from_qtensor(qtensor):
        return QMatMul(qtensor)

    def _check_x(self, xs):
        n, k = self.qtensor.shape
        if xs.dim() < 2:
            raise LloomHipError(3, f"input tensor has only one dimension {tuple(xs.shape)}")
        if xs.shape[-1] != k:
            raise LloomHipError(3, f"input tensor {tuple(xs.shape)} incompatible with {self.qtensor.shape}")
        if xs.dtype not in _ACT_IDS:
            raise LloomHipError(2, f"Expected f32/f16 activations, got {xs.dtype}")
        if not xs.is_contiguous():
            raise LloomHipError(1, f"input tensor is not contiguous {tuple(xs.shape)}")
        if xs.device != self.qtensor.storage.device:
            raise LloomHipError(1, f"input tensor is on {xs.device}, the weight on {self.qtensor.storage.device}")
        return n, k, xs.numel() // k

    def forward(self, xs):
        """x . W^T; an f16 x gives an f16 y (matmul_t_f16, mod.rs:1983-1994:
        x widened to f32, the f32 path, each sum rounded to f16)."""
        n, k, m = self._check_x(xs)
        y = torch.empty(tuple(xs.shape[:-1]) + (n,), dtype=xs.dtype, device=xs.device)
        a = _ACT_IDS[xs.dtype]
        check(lib().lloom_hip_qmatmul(_ctx(_dev_index(xs)), int(self.qtensor.dtype), _ptr(self.qtensor.storage), n,
                                      k, _ptr(xs), a, m, _ptr(y), a, _stream(xs)))
        return y

    __call__ = forward

    def _store(self, xs, y, store):
        n, k, m = self._check_x(xs)
        _check_out(y, tuple(xs.shape[:-1]) + (n,), xs.dtype, xs.device, "qmatmul store")
        a = _ACT_IDS[xs.dtype]
        check(lib().lloom_hip_qmatmul_store(_ctx(_dev_index(xs)), int(self.qtensor.dtype), _ptr(self.qtensor.storage),
                                            n, k, _ptr(xs), a, m, _ptr(y), a, int(store), _stream(xs)))
        return y

    def forward_silu(self, xs):
        """silu(x . W^T) with the SiLU on the matmul's store, one launch
        (QMatMul::forward_silu, mod.rs:2102-2120; MvStore::Silu)."""
        n, _ = self.qtensor.shape
        y = torch.empty(tuple(xs.shape[:-1]) + (n,), dtype=xs.dtype, device=xs.device)
        return self._store(xs, y, MvStore.Silu)

    def forward_mul_into(self, xs, gate):
        """gate <- gate * (x . W^T) at the store, one launch
        (QMatMul::forward_mul_into, mod.rs:2122-2156; MvStore::MulInto).
        gate is a contiguous [.., n] of x's dtype and is overwritten."""
        self._store(xs, gate, MvStore.MulInto)

    def forward_into(self, xs, y):
        """forward into a preallocated contiguous y [.., n] of x's dtype (xs
        [.., k] contiguous, on the weight's device): no allocation once the
        context workspace holds the call's (reserve_workspace), so it can be
        captured in a graph."""
        n, k, m = self._check_x(xs)
        _check_out(y, tuple(xs.shape[:-1]) + (n,), xs.dtype, xs.device, "forward_into")
        a = _ACT_IDS[xs.dtype]
        check(lib().lloom_hip_qmatmul(_ctx(_dev_index(xs)), int(self.qtensor.dtype), _ptr(self.qtensor.storage), n,
                                      k, _ptr(xs), a, m, _ptr(y), a, _stream(xs)))
        return y


# ---------------------------------------------------------- functions ---

def quantize_act(x, vec_dot_dtype):
    """[m, k] f32 -> packed Q8_0 / Q8K blocks (uint8), as k_quants::matmul
    quantizes its lhs (k_quants.rs:2477-2508)."""
    vec_dot_dtype = GgmlDType(vec_dot_dtype)
    x = x.contiguous()
    m, k = x.shape
    bs = vec_dot_dtype.block_size()
    nbytes = m * (k // bs) * vec_dot_dtype.type_size() if k % bs == 0 else 0
    out = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    check(lib().lloom_hip_quantize_act(_ctx(_dev_index(x)), int(vec_dot_dtype), _ptr(x), m, k, _ptr(out),
                                       _stream(x)))
    return out[:nbytes]


def dequantize(blocks, dtype, elems, out_f16=False):
    y = torch.empty(elems, dtype=torch.float16 if out_f16 else torch.float32, device=blocks.device)
    check(lib().lloom_hip_dequantize(_ctx(_dev_index(blocks)), int(GgmlDType(dtype)), _ptr(blocks), elems, _ptr(y),
                                     1 if out_f16 else 0, _stream(blocks)))
    return y


def synth_normal(seed, count, mean=0.0, std=1.0):
    """Deterministic N(mean, std) f32 (SplitMix64 -> xoshiro256**, Box-Muller)."""
    out = np.empty(count, dtype=np.float32)
    check(lib().lloom_hip_synth_normal(seed, mean, std, out.ctypes.data_as(ctypes.c_void_p), count))
    return out


def synth_uniform(seed, count, lo=0.0, hi=1.0):
    out = np.empty(count, dtype=np.float32)
    check(lib().lloom_hip_synth_uniform(seed, lo, hi, out.ctypes.data_as(ctypes.c_void_p), count))
    return out
