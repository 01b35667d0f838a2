"""GGUF files: parse a header, write a file, and hand tensors to the device.

The on-disk format follows the public GGUF specification (ggml's
docs/gguf.md): a magic word, a version, two counts, the key/value metadata,
a tensor directory, padding up to the data alignment, then the tensor
payloads.  Versions 2 and 3 store every count and length as u64; version 1
stores them as u32.  All scalars are little endian.

What a file may declare is bounded before anything is allocated:

* counts, string sizes and array lengths are capped at 2^30, and a header
  must be at least as long as the smallest encoding of what it declares;
* a tensor has at most 4 dims and arrays nest at most 64 deep;
* tensor geometry (elements, bytes, file offsets) is computed exactly and
  refused when it leaves the u64 range; a materialised copy is further
  refused above the host's isize limit;
* a payload is checked against the file's extent before it is read.

These are the limits lloom's reader enforces (gguf_file.rs:20-33, 81-171,
532-654), so the same bytes are accepted or refused with the same cause;
the parser here is organised around a small wire cursor and a codec table
of its own, and its messages are its own.

The one device step is the final upload (`QTensor.from_data`), which puts
the packed blocks in HBM with the tail pad the kernels read past.  Q8_0,
Q4_K, Q6_K and the float types F32 / F16 / BF16 are uploaded; other block
types parse (their geometry is known) but are refused at upload, since the
HIP arm has no kernel for them (ggml_file.rs:180-228 is the reference seam).
"""
import enum
import struct

import numpy as np

from .lib import LloomHipError

DEFAULT_ALIGNMENT = 32
CAP_COUNT = 1 << 30            # tensors, metadata entries, array items
CAP_STRING = 1 << 30           # bytes in one string
CAP_RANK = 4                   # dims of one tensor
CAP_NESTING = 64               # array-in-array depth

_TWO64 = 1 << 64
_HOST_ISIZE = (1 << 63) - 1    # 64-bit hosts: usize == u64, isize is the allocation limit
_WRITE_PAD = 32                # the writer pads header and payloads to 32 bytes

GGUF_TYPE_FP8_E4M3 = 1 << 24


class GgufError(LloomHipError):
    """A GGUF file, tensor or value this module refuses; the text names why."""

    def __init__(self, msg):
        super().__init__(3, msg)


def _refuse(msg):
    raise GgufError(msg)


def _fits_u64(v, what):
    if v >= _TWO64:
        _refuse(f"{what} does not fit in 64 bits")
    return v


# ----------------------------------------------------------- block types

class FileType:
    """A GGML block type id as a tensor directory names it, with its geometry
    (elements per block, bytes per block; mod.rs:505-568, 663-713)."""

    # id: (name, elements per block, bytes per block)
    TABLE = {
        0: ("F32", 1, 4), 1: ("F16", 1, 2), 30: ("BF16", 1, 2),
        2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24),
        8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36),
        10: ("Q2K", 256, 84), 11: ("Q3K", 256, 110), 12: ("Q4K", 256, 144), 13: ("Q5K", 256, 176),
        14: ("Q6K", 256, 210), 15: ("Q8K", 256, 292),
        16: ("IQ2XXS", 256, 66), 17: ("IQ2XS", 256, 74), 18: ("IQ3XXS", 256, 98), 20: ("IQ4NL", 32, 18),
        21: ("IQ3S", 256, 110), 22: ("IQ2S", 256, 82), 23: ("IQ4XS", 256, 136),
        39: ("MXFP4", 32, 17), 42: ("Q2_0", 64, 18), GGUF_TYPE_FP8_E4M3: ("FP8E4M3", 32, 34),
    }
    # Activation-side block types: a kernel produces them at run time, a file
    # never holds weights in them (mod.rs:448-475).
    ACTIVATION_ONLY = frozenset((9, 15))

    __slots__ = ("id",)

    def __init__(self, type_id):
        type_id = int(type_id)
        if type_id not in self.TABLE:
            _refuse(f"tensor type id {type_id} is not a known GGML type")
        self.id = type_id

    @property
    def name(self):
        return self.TABLE[self.id][0]

    def block_size(self):
        return self.TABLE[self.id][1]

    def type_size(self):
        return self.TABLE[self.id][2]

    def validate_file_weight(self):
        if self.id in self.ACTIVATION_ONLY:
            _refuse(f"{self.name} is an activation-only block type; no file stores weights in it")

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


def _as_file_type(t):
    return t if isinstance(t, FileType) else FileType(t)


# ------------------------------------------------------- metadata values

class ValueType(enum.IntEnum):
    """Metadata value type ids, as the spec numbers them."""
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
        if v not in ValueType._value2member_map_:
            _refuse(f"metadata type id {v} is unknown")
        return ValueType(v)


# Fixed-width codecs: struct format per scalar type.
_FIXED = {
    ValueType.U8: "<B", ValueType.I8: "<b", ValueType.U16: "<H", ValueType.I16: "<h",
    ValueType.U32: "<I", ValueType.I32: "<i", ValueType.U64: "<Q", ValueType.I64: "<q",
    ValueType.F32: "<f", ValueType.F64: "<d",
}
_INTEGER = {t: t.name[0] == "U" for t in _FIXED if t.name[0] in "UI"}    # type -> unsigned?


def _floor_bytes(vt, len_width):
    """Fewest bytes one value of type `vt` can occupy on disk: a fixed width,
    a bare length for a string, or an element type plus a length for an array."""
    if vt in _FIXED:
        return struct.calcsize(_FIXED[vt])
    if vt == ValueType.Bool:
        return 1
    return len_width if vt == ValueType.String else 4 + len_width


class Value:
    """One metadata value: `type` plus `v`, a Python int / float / bool / str,
    or a list of Value for an array."""

    __slots__ = ("type", "v")

    def __init__(self, vtype, v):
        self.type = ValueType(vtype)
        self.v = v

    def __repr__(self):
        return f"{self.type.name}({self.v!r})"

    def __eq__(self, other):
        return isinstance(other, Value) and (self.type, self.v) == (other.type, other.v)

    def value_type(self):
        return self.type

    def _want(self, vt):
        if self.type != vt:
            _refuse(f"metadata value {self!r} is not of type {vt.name}")
        return self.v

    def to_u8(self): return self._want(ValueType.U8)
    def to_i8(self): return self._want(ValueType.I8)
    def to_u16(self): return self._want(ValueType.U16)
    def to_i16(self): return self._want(ValueType.I16)
    def to_u32(self): return self._want(ValueType.U32)
    def to_i32(self): return self._want(ValueType.I32)
    def to_i64(self): return self._want(ValueType.I64)
    def to_f32(self): return self._want(ValueType.F32)
    def to_f64(self): return self._want(ValueType.F64)
    def to_bool(self): return self._want(ValueType.Bool)
    def to_vec(self): return self._want(ValueType.Array)
    def to_string(self): return self._want(ValueType.String)

    def to_u64(self):
        """Any unsigned width, or a bool as 0/1; signed types are refused
        (gguf_file.rs:321-332)."""
        if _INTEGER.get(self.type) is True:
            return self.v
        if self.type == ValueType.Bool:
            return int(self.v)
        _refuse(f"metadata value {self!r} cannot widen to u64")

    def to_count(self):
        """Any integer width holding a value >= 0 (gguf_file.rs:334-351)."""
        if self.type not in _INTEGER:
            _refuse(f"metadata value {self!r} is not an integer count")
        if self.v < 0:
            _refuse(f"metadata count {self.v} is negative")
        return self.v

    def encode(self):
        """The value's bytes as a version-2+ file holds them (u64 lengths)."""
        t = self.type
        if t in _FIXED:
            return struct.pack(_FIXED[t], self.v)
        if t == ValueType.Bool:
            return b"\x01" if self.v else b"\x00"
        if t == ValueType.String:
            return _encode_string(self.v)
        kinds = {e.type for e in self.v}
        if len(kinds) > 1:
            _refuse(f"array mixes element types {sorted(k.name for k in kinds)}")
        elem = kinds.pop() if kinds else ValueType.U32      # an empty array says U32
        return struct.pack("<IQ", elem, len(self.v)) + b"".join(e.encode() for e in self.v)

    def write(self, w):
        w.write(self.encode())


# ---------------------------------------------------------------- reading

class VersionedMagic(enum.IntEnum):
    GgufV1 = 1
    GgufV2 = 2
    GgufV3 = 3

    def length_prefix_size(self):
        return 4 if self == VersionedMagic.GgufV1 else 8


_MAGIC_WORDS = (0x46554747, 0x47475546)     # "GGUF" read little or big endian


class _Wire:
    """A forward cursor over a seekable binary stream.  `end` is the stream's
    extent, taken once, so every declared size can be checked against what
    the file still holds before anything of that size is read."""

    def __init__(self, stream):
        self.s = stream
        here = stream.tell()
        self.end = stream.seek(0, 2)
        stream.seek(here)
        self.version = None

    def left(self):
        return max(0, self.end - self.s.tell())

    def raw(self, n, what):
        b = self.s.read(n)
        if len(b) != n:
            _refuse(f"file ends inside {what}")
        return b

    def fixed(self, fmt, what):
        return struct.unpack(fmt, self.raw(struct.calcsize(fmt), what))[0]

    def length(self, what):
        """A count or byte length: u32 in version 1, u64 after."""
        return self.fixed("<I" if self.version == VersionedMagic.GgufV1 else "<Q", what)

    def text(self, what):
        n = self.length(what)
        if n > CAP_STRING:
            _refuse(f"{what}: declared string size {n} is above the cap of {CAP_STRING}")
        if n > self.left():
            _refuse(f"{what}: declared string size {n} runs past the end of the file "
                    f"({self.left()} bytes left)")
        # Writers in the wild pad strings with NULs; undecodable bytes become U+FFFD.
        return self.raw(n, what).rstrip(b"\0").decode("utf-8", "replace")


def _decode_value(wire, vt, depth):
    if depth > CAP_NESTING:
        _refuse(f"metadata arrays nested deeper than {CAP_NESTING}")
    if vt in _FIXED:
        return Value(vt, wire.fixed(_FIXED[vt], "a metadata value"))
    if vt == ValueType.Bool:
        b = wire.raw(1, "a metadata value")[0]
        if b not in (0, 1):
            _refuse(f"bool byte {b} (must be 0 or 1)")
        return Value(vt, b == 1)
    if vt == ValueType.String:
        return Value(vt, wire.text("a metadata string"))
    # Array: element type, length, then the elements.
    elem = ValueType.from_u32(wire.fixed("<I", "an array header"))
    n = wire.length("an array header")
    if n > CAP_COUNT:
        _refuse(f"metadata array of {n} items is above the cap of {CAP_COUNT}")
    floor = n * _floor_bytes(elem, wire.version.length_prefix_size())
    if floor > wire.left():
        _refuse(f"metadata array of {n} items needs {floor} bytes or more, "
                f"the file has {wire.left()} left")
    return Value(vt, [_decode_value(wire, elem, depth + 1) for _ in range(n)])


def _read_preamble(wire):
    word = wire.fixed("<I", "the magic word")
    if word not in _MAGIC_WORDS:
        _refuse(f"not a GGUF file (magic word 0x{word:08x})")
    version = wire.fixed("<I", "the version")
    if version not in VersionedMagic._value2member_map_:
        _refuse(f"GGUF version {version} is not supported (1, 2 and 3 are)")
    wire.version = VersionedMagic(version)
    n_tensors = wire.length("the tensor count")
    n_kv = wire.length("the metadata count")
    for n, what in ((n_tensors, "tensor count"), (n_kv, "metadata count")):
        if n > CAP_COUNT:
            _refuse(f"{what} {n} is above the cap of {CAP_COUNT}")
    # Smallest possible entries: a kv is key length + type id + 1 value byte;
    # a directory entry is name length + rank + type id + offset.
    p = wire.version.length_prefix_size()
    floor = n_kv * (p + 4 + 1) + n_tensors * (p + 4 + 4 + 8)
    if floor > wire.left():
        _refuse(f"a header of {n_tensors} tensors and {n_kv} metadata entries takes {floor} "
                f"bytes or more, the file has {wire.left()} left")
    return n_tensors, n_kv


def _read_directory_entry(wire):
    name = wire.text("a tensor name")
    rank = wire.fixed("<I", "a tensor rank")
    if rank > CAP_RANK:
        _refuse(f"tensor '{name}': rank {rank} is above the GGUF limit of {CAP_RANK}")
    dim_fmt = "<I" if wire.version == VersionedMagic.GgufV1 else "<Q"
    file_dims = [wire.fixed(dim_fmt, "tensor dims") for _ in range(rank)]
    ftype = FileType(wire.fixed("<I", "a tensor type"))
    offset = wire.fixed("<Q", "a tensor offset")
    # The file lists the fastest-varying dim first; shapes here are row-major.
    info = TensorInfo(ftype, file_dims[::-1], offset)
    info.size_in_bytes()
    return name, info


def _data_alignment(metadata):
    """general.alignment when it is a non-negative 8/16/32-bit integer,
    otherwise the default (gguf_file.rs:631-639); zero is refused."""
    a = metadata.get("general.alignment")
    ok = (ValueType.U8, ValueType.U16, ValueType.U32, ValueType.I8, ValueType.I16, ValueType.I32)
    align = a.v if a is not None and a.type in ok and a.v >= 0 else DEFAULT_ALIGNMENT
    if align == 0:
        _refuse("general.alignment of 0 is invalid")
    return align


class TensorInfo:
    """One directory entry: block type, row-major shape, and the payload's
    offset from the start of the data section."""

    __slots__ = ("ggml_dtype", "shape", "offset")

    def __init__(self, ggml_dtype, shape, offset):
        self.ggml_dtype = _as_file_type(ggml_dtype)
        self.shape = tuple(int(d) for d in shape)
        self.offset = int(offset)

    def __repr__(self):
        return f"TensorInfo({self.ggml_dtype!r}, {list(self.shape)}, offset={self.offset})"

    def elements(self):
        n = 1
        for d in self.shape:
            n = _fits_u64(n * d, "tensor element count")
        return n

    def size_in_bytes(self):
        """Packed payload bytes, exact in u64."""
        n, per = self.elements(), self.ggml_dtype.block_size()
        if n % per:
            _refuse(f"{n} elements are not a whole number of {self.ggml_dtype.name} blocks ({per} each)")
        return _fits_u64(n // per * self.ggml_dtype.type_size(), "tensor byte size")

    def materialized_size_in_bytes(self):
        """Bytes of a host copy: also bounded by the host's isize."""
        size = self.size_in_bytes()
        if size > _HOST_ISIZE:
            _refuse(f"tensor of {size} bytes is larger than the host can allocate")
        return size

    def validate_payload(self, f, tensor_data_offset):
        """Check type, host size and file extent without reading a byte
        (only the stream's extent is queried).  Returns (start, size)."""
        self.ggml_dtype.validate_file_weight()
        size = self.materialized_size_in_bytes()
        start = tensor_data_offset + self.offset
        if start >= _TWO64:
            _refuse("tensor payload starts beyond 2^64")
        extent = f.seek(0, 2)
        if start > extent:
            _refuse(f"tensor payload starts at {start}, beyond the end of the file ({extent} bytes)")
        if size > extent - start:
            _refuse(f"tensor payload of {size} bytes at {start} runs past the end of the file "
                    f"({extent - start} bytes left)")
        return start, size

    def read_bytes(self, f, tensor_data_offset):
        """The payload, as stored (uint8)."""
        start, size = self.validate_payload(f, tensor_data_offset)
        out = np.empty(size, dtype=np.uint8)
        f.seek(start)
        if size and f.readinto(memoryview(out)) != size:
            _refuse("file ends inside a tensor payload")
        return out

    def read(self, f, tensor_data_offset, device="cuda"):
        """Payload -> device QTensor."""
        return qtensor_from_ggml(self.ggml_dtype, self.read_bytes(f, tensor_data_offset),
                                 list(self.shape), device)


class Content:
    """A parsed header: version, metadata (dict of Value), tensor directory
    (dict of TensorInfo) and the absolute start of the data section."""

    def __init__(self, magic, metadata, tensor_infos, tensor_data_offset):
        self.magic = magic
        self.metadata = metadata
        self.tensor_infos = tensor_infos
        self.tensor_data_offset = tensor_data_offset

    @staticmethod
    def read(f):
        wire = _Wire(f)
        n_tensors, n_kv = _read_preamble(wire)
        metadata = {}
        for _ in range(n_kv):
            key = wire.text("a metadata key")
            metadata[key] = _decode_value(wire, ValueType.from_u32(wire.fixed("<I", "a metadata type")), 0)
        directory = dict(_read_directory_entry(wire) for _ in range(n_tensors))

        align = _data_alignment(metadata)
        data_start = -(-f.tell() // align) * align
        if data_start >= _TWO64:
            _refuse(f"data section would start at {data_start}, beyond 2^64")
        for name, info in directory.items():
            if data_start + info.offset + info.size_in_bytes() >= _TWO64:
                _refuse(f"tensor '{name}': data range ends beyond 2^64")
        return Content(wire.version, metadata, directory, data_start)

    def validate_payloads(self, f):
        """Check every payload an eager loader would read, reading nothing."""
        for info in self.tensor_infos.values():
            info.validate_payload(f, self.tensor_data_offset)

    def tensor(self, f, name, device="cuda"):
        if name not in self.tensor_infos:
            _refuse(f"no tensor named '{name}' in this file")
        return self.tensor_infos[name].read(f, self.tensor_data_offset, device)


# ---------------------------------------------------------------- writing

def _encode_string(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pad_to(n, align=_WRITE_PAD):
    return -n % align


def packed_offsets(sizes):
    """Data-section offsets for payloads of these sizes, each padded to 32 B."""
    out, at = [], 0
    for s in sizes:
        out.append(at)
        at += s + _pad_to(s)
    return out


class HeaderTensor:
    """A directory entry to write: name, row-major dims, block type, offset."""

    __slots__ = ("name", "dims", "dtype", "offset")

    def __init__(self, name, dims, dtype, offset):
        self.name, self.dims, self.offset = name, tuple(dims), int(offset)
        self.dtype = _as_file_type(dtype)


def write_header(w, metadata, tensors):
    """A version-2 header, padded to 32 B; returns the data section's start.
    `metadata` is a sequence of (key, Value), `tensors` of HeaderTensor."""
    parts = [b"GGUF", struct.pack("<IQQ", 2, len(tensors), len(metadata))]
    for key, value in metadata:
        parts += [_encode_string(key), struct.pack("<I", value.value_type()), value.encode()]
    for t in tensors:
        parts += [_encode_string(t.name), struct.pack("<I", len(t.dims))]
        parts += [struct.pack("<Q", d) for d in t.dims[::-1]]
        parts.append(struct.pack("<IQ", int(t.dtype), t.offset))
    blob = b"".join(parts)
    w.write(blob)
    w.write(bytes(_pad_to(w.tell())))
    return w.tell()


def write(w, metadata, tensors):
    """A whole file: header, then each payload at its packed offset.
    `tensors` is a sequence of (name, tensor) where the tensor has `shape`,
    `dtype` and `data()` (its packed bytes, as QTensor does)."""
    payloads = [t.data() for _, t in tensors]
    offsets = packed_offsets(p.size for p in payloads)
    entries = [HeaderTensor(name, t.shape, int(t.dtype), at) for (name, t), at in zip(tensors, offsets)]
    data_start = write_header(w, metadata, entries)
    for entry, p in zip(entries, payloads):
        if w.tell() != data_start + entry.offset:
            _refuse(f"writer out of step at '{entry.name}': at {w.tell()}, "
                    f"expected {data_start + entry.offset}")
        w.write(p.tobytes())
        w.write(bytes(_pad_to(p.size)))


# ------------------------------------------------------- the upload seam

def checked_tensor_bytes(dtype, dims):
    """Bytes a tensor of these dims takes in `dtype` blocks, refusing what the
    upload cannot hold: activation-only types, rank 0, an innermost dim that
    is not whole blocks, and sizes past the host's limits
    (ggml_file.rs:121-139, mod.rs:894-906)."""
    dtype.validate_file_weight()
    per = dtype.block_size()
    if len(dims) == 0:
        _refuse(f"a rank-0 tensor cannot hold {dtype.name} blocks")
    if dims[-1] % per:
        _refuse(f"innermost dim of {list(dims)} is not a multiple of the {dtype.name} block size {per}")
    n = 1
    for d in dims:
        n = _fits_u64(n * d, "tensor element count")
    size = _fits_u64(n // per * dtype.type_size(), "tensor byte size")
    if size > _HOST_ISIZE:
        _refuse(f"tensor of {size} bytes is larger than the host can allocate")
    return size


def qtensor_from_ggml(dtype, raw, dims, device="cuda"):
    """Packed file bytes -> a device QTensor, uploaded unchanged.  `raw` may
    be longer than the tensor; only its first checked_tensor_bytes are used."""
    from .quantized import GgmlDType, QTensor

    dtype = _as_file_type(dtype)
    dims = [int(d) for d in dims]
    size = checked_tensor_bytes(dtype, dims)
    raw = raw.view(np.uint8) if isinstance(raw, np.ndarray) else np.frombuffer(raw, dtype=np.uint8)
    if raw.size < size:
        _refuse(f"payload holds {raw.size} bytes, the tensor needs {size}")
    if dtype.id not in GgmlDType._value2member_map_:
        raise LloomHipError(2, f"quantized type {dtype.name} has no kernel on the HIP arm "
                               f"(Q8_0, Q4K, Q6K, F32, F16, BF16 are uploaded)")
    return QTensor.from_data(raw[:size], dims, GgmlDType(dtype.id), device=device)
