"""GGUF container: header reader, writer, and the load -> device upload seam.

Host mirror of lloom-tensor/src/quantized/gguf_file.rs (and the part of
ggml_file.rs the GGUF reader calls):
  Value / ValueType (ids, to_* accessors, to_count)   gguf_file.rs:196-530
  Content.read (magic, counts, caps, kv, tensor infos, alignment)  :532-654
  TensorInfo.size_in_bytes / validate_payload / read  gguf_file.rs:81-171
  Content.validate_payloads / tensor                  gguf_file.rs:656-677
  packed_offsets / write_header / write               gguf_file.rs:691-781
  qtensor_from_ggml                                   ggml_file.rs:180-228
The same caps, the same checked arithmetic (u64 for header geometry, host
usize / isize limits for materialisation) and the same refusal wording, so a
file the reference refuses is refused here with the same cause.

Everything in this module is host I/O on a seekable binary reader; the one
device step is the final upload, `QTensor.from_data`, which lays the packed
blocks into HBM with the tail pad the kernels read past.  Q8_0, Q4_K and Q6_K
tensors become device QTensors the matmul path takes; F32 / F16 / BF16
tensors (norms, biases) become device QTensors that dequantize by
reinterpretation; every other block type is parsed (its geometry is known)
but refused at materialisation, since this library has no kernel for it.
"""
import enum
import struct

import numpy as np

from .lib import LloomHipError

DEFAULT_ALIGNMENT = 32

GGUF_MAX_STRING_LENGTH = 1 << 30
GGUF_MAX_ARRAY_ELEMENTS = 1 << 30
GGUF_MAX_TENSOR_DIMS = 4
GGUF_MAX_VALUE_DEPTH = 64

_U64_MAX = (1 << 64) - 1
_USIZE_MAX = _U64_MAX          # 64-bit hosts only
_ISIZE_MAX = (1 << 63) - 1

GGUF_TYPE_FP8_E4M3 = 1 << 24


class GgufError(LloomHipError):
    """A refused GGUF file or tensor; the message names the cause."""

    def __init__(self, msg):
        super().__init__(3, msg)


def _bail(msg):
    raise GgufError(msg)


# ------------------------------------------------------------ dtypes ---
# Every GGML type id a GGUF header may name (mod.rs:505-568), with its block
# geometry (mod.rs:663-713): id -> (name, elements per block, bytes per block).
FILE_TYPES = {
    0: ("F32", 1, 4),
    1: ("F16", 1, 2),
    2: ("Q4_0", 32, 18),
    3: ("Q4_1", 32, 20),
    6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24),
    8: ("Q8_0", 32, 34),
    9: ("Q8_1", 32, 36),
    10: ("Q2K", 256, 84),
    11: ("Q3K", 256, 110),
    12: ("Q4K", 256, 144),
    13: ("Q5K", 256, 176),
    14: ("Q6K", 256, 210),
    15: ("Q8K", 256, 292),
    16: ("IQ2XXS", 256, 66),
    17: ("IQ2XS", 256, 74),
    18: ("IQ3XXS", 256, 98),
    20: ("IQ4NL", 32, 18),
    21: ("IQ3S", 256, 110),
    22: ("IQ2S", 256, 82),
    23: ("IQ4XS", 256, 136),
    30: ("BF16", 1, 2),
    39: ("MXFP4", 32, 17),
    42: ("Q2_0", 64, 18),
    GGUF_TYPE_FP8_E4M3: ("FP8E4M3", 32, 34),
}
_ACTIVATION_ONLY = (9, 15)      # Q8_1, Q8K: no file stores a weight in them


class FileType:
    """A GGML type as a GGUF header names it (GgmlDType in the reference)."""

    __slots__ = ("id",)

    def __init__(self, type_id):
        if type_id not in FILE_TYPES:
            _bail(f"unknown dtype for tensor {type_id}")
        self.id = int(type_id)

    name = property(lambda self: FILE_TYPES[self.id][0])

    def block_size(self):
        return FILE_TYPES[self.id][1]

    def type_size(self):
        return FILE_TYPES[self.id][2]

    def validate_file_weight(self):
        """GgmlDType::validate_file_weight (mod.rs:448-475)."""
        if self.id in _ACTIVATION_ONLY:
            _bail(f"quantized type {self.name} is not supported yet")

    def __eq__(self, other):
        if isinstance(other, FileType):
            return other.id == self.id
        return isinstance(other, int) and other == self.id

    def __hash__(self):
        return hash(self.id)

    def __int__(self):
        return self.id

    def __repr__(self):
        return self.name


# ------------------------------------------------------------ values ---

class ValueType(enum.IntEnum):
    """gguf_file.rs:483-519 (on-disk ids)."""
    U8 = 0
    I8 = 1
    U16 = 2
    I16 = 3
    U32 = 4
    I32 = 5
    F32 = 6
    Bool = 7
    String = 8
    Array = 9
    U64 = 10
    I64 = 11
    F64 = 12

    @staticmethod
    def from_u32(v):
        try:
            return ValueType(v)
        except ValueError:
            _bail(f"unrecognized value-type {v:#08x}")

    def min_disk_size(self, prefix):
        """Smallest encoding of one value (gguf_file.rs:521-530)."""
        if self in (ValueType.U8, ValueType.I8, ValueType.Bool):
            return 1
        if self in (ValueType.U16, ValueType.I16):
            return 2
        if self in (ValueType.U32, ValueType.I32, ValueType.F32):
            return 4
        if self in (ValueType.U64, ValueType.I64, ValueType.F64):
            return 8
        if self == ValueType.String:
            return prefix
        return 4 + prefix


_SCALAR = {
    ValueType.U8: "<B", ValueType.I8: "<b", ValueType.U16: "<H", ValueType.I16: "<h",
    ValueType.U32: "<I", ValueType.I32: "<i", ValueType.U64: "<Q", ValueType.I64: "<q",
    ValueType.F32: "<f", ValueType.F64: "<d",
}
_UNSIGNED = (ValueType.U8, ValueType.U16, ValueType.U32, ValueType.U64)
_SIGNED = (ValueType.I8, ValueType.I16, ValueType.I32, ValueType.I64)


class Value:
    """A typed metadata value (gguf_file.rs:231-245).  `v` is a Python int,
    float, bool, str, or a list of Value for arrays."""

    __slots__ = ("type", "v")

    def __init__(self, vtype, v):
        self.type = ValueType(vtype)
        self.v = v

    def __repr__(self):
        return f"{self.type.name}({self.v!r})"

    def __eq__(self, other):
        return isinstance(other, Value) and self.type == other.type and self.v == other.v

    def value_type(self):
        return self.type

    def _exact(self, vt, what):
        if self.type != vt:
            _bail(f"not a {what} {self!r}")
        return self.v

    def to_u8(self): return self._exact(ValueType.U8, "u8")
    def to_i8(self): return self._exact(ValueType.I8, "i8")
    def to_u16(self): return self._exact(ValueType.U16, "u16")
    def to_i16(self): return self._exact(ValueType.I16, "i16")
    def to_u32(self): return self._exact(ValueType.U32, "u32")
    def to_i32(self): return self._exact(ValueType.I32, "i32")
    def to_i64(self): return self._exact(ValueType.I64, "i64")
    def to_f32(self): return self._exact(ValueType.F32, "f32")
    def to_f64(self): return self._exact(ValueType.F64, "f64")
    def to_bool(self): return self._exact(ValueType.Bool, "bool")
    def to_vec(self): return self._exact(ValueType.Array, "vec")
    def to_string(self): return self._exact(ValueType.String, "string")

    def to_u64(self):
        """Unsigned widths and bool upcast; nothing signed (gguf_file.rs:321-332)."""
        if self.type in _UNSIGNED:
            return self.v
        if self.type == ValueType.Bool:
            return int(self.v)
        _bail(f"not a u64 or upcastable to u64 {self!r}")

    def to_count(self):
        """Any integer width, refused when negative (gguf_file.rs:334-351)."""
        if self.type in _UNSIGNED:
            return self.v
        if self.type in _SIGNED:
            if self.v < 0:
                _bail(f"negative count {self.v}")
            return self.v
        _bail(f"not a non-negative integer {self!r}")

    # -- encoding (gguf_file.rs:436-480; arrays always carry a u64 length) --
    def write(self, w):
        t = self.type
        if t in _SCALAR:
            w.write(struct.pack(_SCALAR[t], self.v))
        elif t == ValueType.Bool:
            w.write(bytes([1 if self.v else 0]))
        elif t == ValueType.String:
            _write_string(w, self.v)
        else:
            if not self.v:
                inner = ValueType.U32
            else:
                kinds = {e.type for e in self.v}
                if len(kinds) != 1:
                    _bail(f"multiple value-types in the same array {sorted(k.name for k in kinds)}")
                inner = kinds.pop()
            w.write(struct.pack("<IQ", int(inner), len(self.v)))
            for e in self.v:
                e.write(w)


# ------------------------------------------------------------ reading ---

class VersionedMagic(enum.IntEnum):
    GgufV1 = 1
    GgufV2 = 2
    GgufV3 = 3

    def length_prefix_size(self):
        return 4 if self == VersionedMagic.GgufV1 else 8


class _Reader:
    """Little-endian reads over a seekable binary stream, with the file size
    captured once (the reference's remaining_bytes)."""

    def __init__(self, f):
        self.f = f
        start = f.tell()
        self.file_size = f.seek(0, 2)
        f.seek(start)

    def exact(self, n):
        b = self.f.read(n)
        if len(b) != n:
            _bail("failed to fill whole buffer")
        return b

    def u8(self): return self.exact(1)[0]
    def u32(self): return struct.unpack("<I", self.exact(4))[0]
    def u64(self): return struct.unpack("<Q", self.exact(8))[0]

    def pos(self):
        return self.f.tell()

    def remaining(self):
        return max(0, self.file_size - self.pos())

    def length(self, magic):
        return self.u32() if magic == VersionedMagic.GgufV1 else self.u64()

    def string(self, magic):
        n = self.length(magic)
        if n > GGUF_MAX_STRING_LENGTH:
            _bail(f"gguf: string length {n} exceeds max {GGUF_MAX_STRING_LENGTH}")
        rem = self.remaining()
        if n > rem:
            _bail(f"gguf: string length {n} exceeds remaining file bytes {rem}")
        b = self.exact(n).rstrip(b"\x00")      # trailing NULs occur in practice
        return b.decode("utf-8", errors="replace")

    def value(self, vt, magic, depth):
        if depth > GGUF_MAX_VALUE_DEPTH:
            _bail(f"gguf: value nesting depth exceeds max {GGUF_MAX_VALUE_DEPTH}")
        if vt in _SCALAR:
            fmt = _SCALAR[vt]
            return Value(vt, struct.unpack(fmt, self.exact(struct.calcsize(fmt)))[0])
        if vt == ValueType.Bool:
            b = self.u8()
            if b > 1:
                _bail(f"unexpected bool value {b}")
            return Value(vt, bool(b))
        if vt == ValueType.String:
            return Value(vt, self.string(magic))
        inner = ValueType.from_u32(self.u32())
        n = self.length(magic)
        if n > GGUF_MAX_ARRAY_ELEMENTS:
            _bail(f"gguf: array length {n} exceeds max {GGUF_MAX_ARRAY_ELEMENTS}")
        need = n * inner.min_disk_size(magic.length_prefix_size())
        rem = self.remaining()
        if need > rem:
            _bail(f"gguf: array of {n} elements needs at least {need} bytes, only {rem} remaining")
        return Value(vt, [self.value(inner, magic, depth + 1) for _ in range(n)])


def _read_magic(r):
    m = r.u32()
    if m not in (0x46554747, 0x47475546):
        _bail(f"unknown magic 0x{m:08x}")
    v = r.u32()
    if v not in (1, 2, 3):
        _bail(f"gguf: unsupported magic/version Gguf/{v}")
    return VersionedMagic(v)


class TensorInfo:
    """One tensor of the header: type, shape (row-major, as the reference's
    Shape holds it: the file's dims reversed) and offset from the data start."""

    __slots__ = ("ggml_dtype", "shape", "offset")

    def __init__(self, ggml_dtype, shape, offset):
        self.ggml_dtype = ggml_dtype if isinstance(ggml_dtype, FileType) else FileType(int(ggml_dtype))
        self.shape = tuple(int(d) for d in shape)
        self.offset = int(offset)

    def __repr__(self):
        return f"TensorInfo({self.ggml_dtype!r}, {list(self.shape)}, offset={self.offset})"

    def size_in_bytes(self):
        """Header geometry in u64, checked (gguf_file.rs:88-104)."""
        elems = 1
        for d in self.shape:
            elems *= d
            if elems > _U64_MAX:
                _bail("gguf: tensor element count overflow")
        bs = self.ggml_dtype.block_size()
        if elems % bs:
            _bail(f"the number of elements {elems} is not divisible by the block size {bs}")
        b = (elems // bs) * self.ggml_dtype.type_size()
        if b > _U64_MAX:
            _bail("gguf: tensor byte size overflow")
        return b

    def materialized_size_in_bytes(self):
        """Host limits for a materialised copy (gguf_file.rs:106-120)."""
        elems = 1
        for d in self.shape:
            elems *= d
            if elems > _USIZE_MAX:
                _bail("gguf: host tensor element count overflow")
        b = self.size_in_bytes()
        if b > _USIZE_MAX:
            _bail("gguf: tensor byte size exceeds host usize")
        if b > _ISIZE_MAX:
            _bail(f"gguf: tensor byte size {b} exceeds host allocation limit")
        return b

    def validate_payload(self, f, tensor_data_offset):
        """Type, host size and file extent, reading nothing (gguf_file.rs:125-144).
        Leaves `f` at its end.  Returns (absolute start, byte count)."""
        self.ggml_dtype.validate_file_weight()
        size = self.materialized_size_in_bytes()
        start = tensor_data_offset + self.offset
        if start > _U64_MAX:
            _bail("gguf: tensor start offset overflow")
        file_size = f.seek(0, 2)
        if file_size < start:
            _bail(f"gguf: tensor offset {start} exceeds file size {file_size}, no remaining bytes")
        rem = file_size - start
        if size > rem:
            _bail(f"tensor needs {size} bytes at offset {start}, only {rem} remaining in file")
        return start, size

    def read_bytes(self, f, tensor_data_offset):
        """The tensor's packed bytes as the file holds them (numpy uint8)."""
        start, size = self.validate_payload(f, tensor_data_offset)
        f.seek(start)
        raw = np.empty(size, dtype=np.uint8)
        got = f.readinto(memoryview(raw)) if size else 0
        if got != size:
            _bail("failed to fill whole buffer")
        return raw

    def read(self, f, tensor_data_offset, device="cuda"):
        """TensorInfo::read (gguf_file.rs:146-170): validate, read, upload."""
        raw = self.read_bytes(f, tensor_data_offset)
        return qtensor_from_ggml(self.ggml_dtype, raw, list(self.shape), device)


class Content:
    """A parsed GGUF header (gguf_file.rs:172-178, 532-677)."""

    def __init__(self, magic, metadata, tensor_infos, tensor_data_offset):
        self.magic = magic
        self.metadata = metadata
        self.tensor_infos = tensor_infos
        self.tensor_data_offset = tensor_data_offset

    @staticmethod
    def read(f):
        r = _Reader(f)
        magic = _read_magic(r)
        tensor_count = r.length(magic)
        kv_count = r.length(magic)
        if tensor_count > GGUF_MAX_ARRAY_ELEMENTS:
            _bail(f"gguf: tensor_count {tensor_count} exceeds max {GGUF_MAX_ARRAY_ELEMENTS}")
        if kv_count > GGUF_MAX_ARRAY_ELEMENTS:
            _bail(f"gguf: metadata_kv_count {kv_count} exceeds max {GGUF_MAX_ARRAY_ELEMENTS}")
        prefix = magic.length_prefix_size()
        need = kv_count * (prefix + 4 + 1) + tensor_count * (prefix + 4 + 4 + 8)
        rem = r.remaining()
        if need > rem:
            _bail(f"gguf: header declares {tensor_count} tensors and {kv_count} metadata entries, "
                  f"needs at least {need} bytes, only {rem} remaining")

        metadata = {}
        for _ in range(kv_count):
            key = r.string(magic)
            vt = ValueType.from_u32(r.u32())
            metadata[key] = r.value(vt, magic, 0)

        tensor_infos = {}
        for _ in range(tensor_count):
            name = r.string(magic)
            nd = r.u32()
            if nd > GGUF_MAX_TENSOR_DIMS:
                _bail(f"gguf: tensor '{name}' has {nd} dimensions, max is {GGUF_MAX_TENSOR_DIMS}")
            fmt = "<%d%s" % (nd, "I" if magic == VersionedMagic.GgufV1 else "Q")
            dims = list(struct.unpack(fmt, r.exact(struct.calcsize(fmt))))
            for d in dims:
                if d > _USIZE_MAX:
                    _bail(f"gguf: tensor dimension {d} exceeds host usize")
            dims.reverse()
            dtype = FileType(r.u32())
            offset = r.u64()
            info = TensorInfo(dtype, dims, offset)
            info.size_in_bytes()
            tensor_infos[name] = info

        position = r.pos()
        alignment = DEFAULT_ALIGNMENT
        a = metadata.get("general.alignment")
        if a is not None and a.type in (ValueType.U8, ValueType.U16, ValueType.U32, ValueType.I8,
                                        ValueType.I16, ValueType.I32) and a.v >= 0:
            alignment = a.v
        if alignment == 0:
            _bail("gguf: general.alignment must be nonzero")
        tdo = position + (alignment - position % alignment) % alignment
        if tdo > _U64_MAX:
            _bail("gguf: aligned tensor data offset overflow")
        for info in tensor_infos.values():
            if tdo + info.offset + info.size_in_bytes() > _U64_MAX:
                _bail("gguf: tensor byte range offset overflow")
        return Content(magic, metadata, tensor_infos, tdo)

    def validate_payloads(self, f):
        """Every tensor an eager loader would materialise, unread (gguf_file.rs:656-664)."""
        for info in self.tensor_infos.values():
            info.validate_payload(f, self.tensor_data_offset)

    def tensor(self, f, name, device="cuda"):
        info = self.tensor_infos.get(name)
        if info is None:
            _bail(f"cannot find tensor info for {name}")
        return info.read(f, self.tensor_data_offset, device)


# ------------------------------------------------------------ writing ---

def _write_string(w, s):
    b = s.encode("utf-8")
    w.write(struct.pack("<Q", len(b)))
    w.write(b)


def _pad32(n):
    return 31 - (31 + n) % 32


def packed_offsets(sizes):
    """Offsets `write` gives tensors of these byte sizes: each padded to 32 B
    (gguf_file.rs:696-708)."""
    out, off = [], 0
    for s in sizes:
        out.append(off)
        off += s + _pad32(s)
    return out


class HeaderTensor:
    """A header entry: name, row-major dims, type, offset (gguf_file.rs:684-690)."""

    __slots__ = ("name", "dims", "dtype", "offset")

    def __init__(self, name, dims, dtype, offset):
        self.name, self.dims, self.offset = name, tuple(dims), int(offset)
        self.dtype = dtype if isinstance(dtype, FileType) else FileType(int(dtype))


def write_header(w, metadata, tensors):
    """A version-2 header padded to 32 B; returns where the data starts
    (gguf_file.rs:710-738).  `metadata` is a sequence of (key, Value)."""
    w.write(struct.pack("<IIQQ", 0x46554747, 2, len(tensors), len(metadata)))
    for key, value in metadata:
        _write_string(w, key)
        w.write(struct.pack("<I", int(value.value_type())))
        value.write(w)
    for t in tensors:
        _write_string(w, t.name)
        w.write(struct.pack("<I", len(t.dims)))
        for d in reversed(t.dims):
            w.write(struct.pack("<Q", d))
        w.write(struct.pack("<IQ", int(t.dtype), t.offset))
    w.write(bytes(_pad32(w.tell())))
    return w.tell()


def write(w, metadata, tensors):
    """Header, then each tensor's packed bytes at its offset, 32 B padded
    (gguf_file.rs:740-781).  `tensors` is a sequence of (name, QTensor)."""
    datas = [t.data() for _, t in tensors]
    offsets = packed_offsets(d.size for d in datas)
    start = write_header(w, metadata, [HeaderTensor(name, t.shape, int(t.dtype), off)
                                       for (name, t), off in zip(tensors, offsets)])
    for off, data in zip(offsets, datas):
        pos = w.tell()
        if start + off != pos:
            _bail(f"internal error, unexpected current position {start} {off} {pos}")
        w.write(data.tobytes())
        w.write(bytes(_pad32(data.size)))


# ------------------------------------------------- the upload seam ---

def checked_tensor_bytes(dtype, dims):
    """ggml_file.rs:121-139 (with check_shape, mod.rs:894-906)."""
    dtype.validate_file_weight()
    bs = dtype.block_size()
    if not dims:
        _bail(f"scalar tensor cannot be quantized {list(dims)}")
    if dims[-1] % bs:
        _bail(f"quantized tensor must have their last dim divisible by block size {list(dims)} {bs}")
    elems = 1
    for d in dims:
        elems *= d
        if elems > _USIZE_MAX:
            _bail("ggml: tensor element count overflow")
    b = (elems // bs) * dtype.type_size()
    if b > _USIZE_MAX:
        _bail("ggml: tensor byte size overflow")
    if b > _ISIZE_MAX:
        _bail(f"ggml: tensor byte size {b} exceeds host allocation limit")
    return b


def qtensor_from_ggml(dtype, raw, dims, device="cuda"):
    """Raw file bytes -> a device QTensor (ggml_file.rs:180-228): the first
    size_in_bytes bytes of `raw`, uploaded unchanged."""
    from .quantized import QTensor, GgmlDType

    dtype = dtype if isinstance(dtype, FileType) else FileType(int(dtype))
    dims = [int(d) for d in dims]
    size = checked_tensor_bytes(dtype, dims)
    raw = np.frombuffer(raw, dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.view(np.uint8)
    if raw.size < size:
        _bail(f"ggml: payload length {raw.size} is shorter than expected {size} bytes")
    try:
        gd = GgmlDType(dtype.id)
    except ValueError:
        raise LloomHipError(2, f"quantized type {dtype.name} has no kernel on the HIP arm "
                               f"(Q8_0, Q4K, Q6K, F32, F16, BF16 are uploaded)") from None
    return QTensor.from_data(raw[:size], dims, gd, device=device)
