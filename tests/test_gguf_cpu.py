"""GGUF reader / writer on the host (no GPU).

Each test restates one of lloom-tensor/tests/gguf_tests.rs (named in its
docstring) on the same bytes, so the parser refuses and accepts exactly what
the reference does; the write -> read round trip is pinned against byte
layouts written out by hand from the GGUF spec.
"""
import io
import struct

import numpy as np
import pytest

import oracle
from lloom_amd.gguf_file import (Content, FileType, GgufError, HeaderTensor, TensorInfo, Value, ValueType,
                                 VersionedMagic, packed_offsets, qtensor_from_ggml, write, write_header)
from lloom_amd.lib import LloomHipError
from lloom_amd.quantized import GgmlDType

U64_MAX = (1 << 64) - 1
ISIZE_MAX = (1 << 63) - 1


def header(tensor_count, kv_count):
    return b"GGUF" + struct.pack("<IQQ", 3, tensor_count, kv_count)


def lp(s):
    return struct.pack("<Q", len(s)) + s


def rejects(buf, needle):
    with pytest.raises(GgufError) as e:
        Content.read(io.BytesIO(buf))
    assert needle in str(e.value), str(e.value)


def test_empty_header_loads():
    """gguf_tests.rs:38-44"""
    c = Content.read(io.BytesIO(header(0, 0)))
    assert c.metadata == {} and c.tensor_infos == {}
    assert c.magic == VersionedMagic.GgufV3
    assert c.tensor_data_offset == 32          # 24 header bytes, aligned to 32


def test_oversized_counts():
    """gguf_tests.rs:46-54"""
    rejects(header(0, 1 << 31), "metadata count")
    rejects(header(1 << 31, 0), "tensor count")


def test_oversized_string_length():
    """gguf_tests.rs:56-62"""
    rejects(header(1, 0) + struct.pack("<Q", 1 << 31) + bytes(64), "string size")


def test_oversized_array_length():
    """gguf_tests.rs:64-73"""
    buf = header(0, 1) + lp(b"k") + struct.pack("<IIQ", 9, 0, 1 << 31) + bytes(64)
    rejects(buf, "array of")


def test_oversized_n_dimensions():
    """gguf_tests.rs:75-82"""
    rejects(header(1, 0) + lp(b"t") + struct.pack("<I", 0xFFFFFFFF) + bytes(64), "rank")


def test_deeply_nested_arrays():
    """gguf_tests.rs:84-99"""
    buf = header(0, 1) + lp(b"k") + struct.pack("<I", 9)
    buf += struct.pack("<IQ", 9, 1) * 256 + struct.pack("<IQ", 0, 0)
    rejects(buf, "nested deeper")


def test_empty_v1_header_loads():
    """gguf_tests.rs:101-110: version 1 uses u32 lengths."""
    c = Content.read(io.BytesIO(b"GGUF" + struct.pack("<III", 1, 0, 0)))
    assert c.magic == VersionedMagic.GgufV1 and c.tensor_data_offset == 32


def test_v1_tensor_dims_are_u32():
    buf = b"GGUF" + struct.pack("<III", 1, 1, 0) + struct.pack("<I", 1) + b"w"
    buf += struct.pack("<I", 2) + struct.pack("<II", 256, 3) + struct.pack("<IQ", 12, 0)
    c = Content.read(io.BytesIO(buf))
    assert c.tensor_infos["w"].shape == (3, 256) and c.tensor_infos["w"].ggml_dtype == 12


def test_bad_magic_and_version():
    rejects(b"GGUX" + bytes(20), "not a GGUF file")
    rejects(b"GGUF" + struct.pack("<IQQ", 4, 0, 0), "version 4 is not supported")


def test_tensor_size_exceeding_file():
    """gguf_tests.rs:112-136: a 4 GiB F32 tensor with no payload."""
    buf = header(1, 0) + lp(b"t") + struct.pack("<IQIQ", 1, 1 << 30, 0, 0)
    f = io.BytesIO(buf)
    c = Content.read(f)
    with pytest.raises(GgufError, match="end of the file"):
        c.tensor(f, "t", device="cpu")


def test_string_length_above_remaining_file():
    """gguf_tests.rs:138-144"""
    rejects(header(1, 0) + struct.pack("<Q", 1 << 20) + bytes(64), "string size")


def tensor_header(dims, dtype, offset):
    buf = header(1, 0) + lp(b"t") + struct.pack("<I", len(dims))
    for d in reversed(dims):
        buf += struct.pack("<Q", d)
    return buf + struct.pack("<IQ", dtype, offset)


def alignment_header(alignment):
    return header(0, 1) + lp(b"general.alignment") + struct.pack("<II", 4, alignment)


def test_alignment():
    """gguf_tests.rs:230-239: zero refused, any positive alignment kept."""
    rejects(alignment_header(0), "alignment of 0")
    for a in (1, 8, 24, 32):
        buf = alignment_header(a)
        assert Content.read(io.BytesIO(buf)).tensor_data_offset == -(-len(buf) // a) * a


def test_signed_and_negative_alignment():
    """A negative signed alignment falls back to 32 (gguf_file.rs:631-639)."""
    buf = header(0, 1) + lp(b"general.alignment") + struct.pack("<Ii", 5, -8)
    assert Content.read(io.BytesIO(buf)).tensor_data_offset == -(-len(buf) // 32) * 32
    buf = header(0, 1) + lp(b"general.alignment") + struct.pack("<Ih", 3, 24)
    assert Content.read(io.BytesIO(buf)).tensor_data_offset == -(-len(buf) // 24) * 24


def test_tensor_element_and_byte_overflow():
    """gguf_tests.rs:241-258"""
    rejects(tensor_header([U64_MAX, 2], 0, 0), "element count does not fit")
    rejects(tensor_header([U64_MAX // 4 + 1], 0, 0), "byte size does not fit")


def test_large_header_inspectable_materialisation_refused():
    """gguf_tests.rs:260-272"""
    f = io.BytesIO(tensor_header([ISIZE_MAX // 4 + 1], 0, 0))
    c = Content.read(f)
    with pytest.raises(GgufError, match="larger than the host can allocate"):
        c.tensor(f, "t", device="cpu")


def test_scalar_zero_axis_shapes_kept():
    """gguf_tests.rs:274-286"""
    for dims in ([], [0], [2, 0, 3], [1024]):
        c = Content.read(io.BytesIO(tensor_header(dims, 0, 0)))
        assert c.tensor_infos["t"].shape == tuple(dims)


def test_tensor_start_end_overflow():
    """gguf_tests.rs:288-300: the 57-byte header aligns to 64."""
    rejects(tensor_header([1], 0, U64_MAX), "ends beyond 2^64")
    assert len(tensor_header([1], 0, 0)) == 57
    rejects(tensor_header([1], 0, U64_MAX - 66), "ends beyond 2^64")
    # two bytes lower and the F32 payload ends at u64::MAX exactly
    Content.read(io.BytesIO(tensor_header([1], 0, U64_MAX - 68)))


def test_direct_tensor_info_read():
    """gguf_tests.rs:302-323"""
    for dims, offset, base, want in [([U64_MAX, 2], 0, 0, "element count does not fit"),
                                     ([U64_MAX // 4 + 1], 0, 0, "byte size does not fit"),
                                     ([1], U64_MAX, 1, "starts beyond 2^64"),
                                     ([0], 1, 0, "beyond the end of the file"),
                                     ([1], 0, 0, "past the end")]:
        info = TensorInfo(FileType(0), dims, offset)
        with pytest.raises(GgufError) as e:
            info.read(io.BytesIO(b""), base, device="cpu")
        assert want in str(e.value), (want, str(e.value))


class _Positioned(io.RawIOBase):
    """A reader whose positions start near u64::MAX (gguf_tests.rs:326-358)."""

    def __init__(self, data, base):
        self.b, self.base = io.BytesIO(data), base

    def readable(self):
        return True

    def read(self, n=-1):
        return self.b.read(n)

    def tell(self):
        return self.b.tell() + self.base

    def seek(self, off, whence=0):
        if whence == 0:
            off -= self.base
        return self.b.seek(off, whence) + self.base


def test_alignment_roundup_overflow():
    """gguf_tests.rs:325-359"""
    with pytest.raises(GgufError, match="data section would start"):
        Content.read(_Positioned(header(0, 0), U64_MAX - 31))


class _Extent:
    """Only the extent is observable (gguf_tests.rs:370-377)."""

    def __init__(self, n):
        self.n = n

    def seek(self, off, whence=0):
        assert (off, whence) == (0, 2), "preflight only observes extent"
        return self.n


def test_eager_payload_preflight():
    """gguf_tests.rs:362-459"""
    c = Content(VersionedMagic.GgufV3, {}, {"required": TensorInfo(FileType(0), [4], 0),
                                           "extra": TensorInfo(FileType(0), [4], 48)}, 0)
    c.validate_payloads(_Extent(64))
    for dt in (9, 15):
        ft = FileType(dt)
        c.tensor_infos["extra"] = TensorInfo(ft, [ft.block_size()], 48)
        with pytest.raises(GgufError, match="activation-only"):
            c.validate_payloads(_Extent(U64_MAX))
        with pytest.raises(GgufError, match="activation-only"):
            qtensor_from_ggml(dt, b"", [ft.block_size()], device="cpu")
    c.tensor_infos["extra"] = TensorInfo(FileType(0), [4], 48)
    with pytest.raises(GgufError, match="15 bytes left"):
        c.validate_payloads(_Extent(63))
    c.tensor_infos["extra"] = TensorInfo(FileType(0), [0], 64)
    c.validate_payloads(_Extent(64))
    c.tensor_data_offset = 1
    c.tensor_infos["extra"].offset = U64_MAX
    with pytest.raises(GgufError, match="starts beyond 2"):
        c.validate_payloads(_Extent(U64_MAX))
    c.tensor_data_offset = 0
    c.tensor_infos["extra"] = TensorInfo(FileType(2), [31], 0)
    with pytest.raises(GgufError, match="whole number of"):
        c.validate_payloads(_Extent(64))
    c.tensor_infos["extra"] = TensorInfo(FileType(0), [ISIZE_MAX // 4 + 1], 0)
    with pytest.raises(GgufError, match="larger than the host can allocate"):
        c.validate_payloads(_Extent(U64_MAX))


def test_a_count_is_any_non_negative_integer():
    """gguf_tests.rs:465-486"""
    for v, want in [(Value(ValueType.U8, 7), 7), (Value(ValueType.U32, 8), 8), (Value(ValueType.U64, U64_MAX), U64_MAX),
                    (Value(ValueType.I8, 0), 0), (Value(ValueType.I32, 8), 8),
                    (Value(ValueType.I64, (1 << 63) - 1), (1 << 63) - 1)]:
        assert v.to_count() == want
    for v in [Value(ValueType.I32, -1), Value(ValueType.I64, -(1 << 63)), Value(ValueType.Bool, True),
              Value(ValueType.F32, 2.0)]:
        with pytest.raises(GgufError):
            v.to_count()
    assert Value(ValueType.Bool, True).to_u64() == 1
    with pytest.raises(GgufError):
        Value(ValueType.I8, 1).to_u64()


def test_unknown_tensor_dtype_and_bad_bool():
    rejects(tensor_header([4], 5, 0), "type id 5 is not")
    rejects(header(0, 1) + lp(b"b") + struct.pack("<IB", 7, 2) + bytes(16), "bool byte 2")
    rejects(header(0, 1) + lp(b"x") + struct.pack("<I", 13) + bytes(16), "metadata type id 13")


def test_strings_strip_trailing_nuls_and_decode_lossy():
    buf = header(0, 2) + lp(b"a") + struct.pack("<I", 8) + lp(b"llama\x00\x00")
    buf += lp(b"b") + struct.pack("<I", 8) + lp(b"\xffok")
    c = Content.read(io.BytesIO(buf))
    assert c.metadata["a"].to_string() == "llama"
    assert c.metadata["b"].to_string() == "�ok"


class _HostQ:
    """A host-side stand-in with QTensor's writer-facing surface (shape, dtype, data())."""

    def __init__(self, shape, dtype, data):
        self.shape, self.dtype, self._d = tuple(shape), dtype, np.frombuffer(bytes(data), np.uint8)

    def data(self):
        return self._d


def test_write_is_header_then_each_tensor_at_its_offset():
    """gguf_tests.rs:146-207, with the expected bytes spelled out from the spec."""
    a = _HostQ((3, 5), GgmlDType.F32, np.arange(15, dtype=np.float32).tobytes())
    xb = (np.arange(128, dtype=np.float32) / np.float32(7.0)).astype(np.float32)
    qb = oracle.quantize(GgmlDType.Q8_0, xb)
    b = _HostQ((2, 64), GgmlDType.Q8_0, qb)
    md = [("general.test", Value(ValueType.U32, 7))]
    whole = io.BytesIO()
    write(whole, md, [("a", a), ("b", b)])
    whole = whole.getvalue()

    offsets = packed_offsets([60, b.data().size])
    assert offsets == [0, 64]                   # 15 f32 = 60 B, padded to 64
    split = io.BytesIO()
    start = write_header(split, md, [HeaderTensor("a", a.shape, 0, 0), HeaderTensor("b", b.shape, 8, 64)])
    for t, off in zip((a, b), offsets):
        split.seek(start + off)
        split.write(t.data().tobytes())
    sp = split.getvalue()
    assert sp + bytes(len(whole) - len(sp)) == whole

    # spelled out: magic, v2, counts, the kv, two tensor entries (dims reversed), pad to 32
    hdr = b"GGUF" + struct.pack("<IQQ", 2, 2, 1) + lp(b"general.test") + struct.pack("<II", 4, 7)
    hdr += lp(b"a") + struct.pack("<IQQ", 2, 5, 3) + struct.pack("<IQ", 0, 0)
    hdr += lp(b"b") + struct.pack("<IQQ", 2, 64, 2) + struct.pack("<IQ", 8, 64)
    hdr += bytes(-len(hdr) % 32)
    assert start == len(hdr) and whole[:start] == hdr
    assert whole[start:start + 60] == a.data().tobytes() and whole[start + 60:start + 64] == bytes(4)
    assert whole[start + 64:start + 64 + 136] == qb.tobytes() and len(whole) == start + 64 + 160

    f = io.BytesIO(whole)
    c = Content.read(f)
    assert c.tensor_data_offset == start
    assert c.metadata == {"general.test": Value(ValueType.U32, 7)}
    assert c.tensor_infos["b"].offset == 64 and c.tensor_infos["b"].shape == (2, 64)
    assert c.tensor_infos["a"].ggml_dtype == 0 and c.tensor_infos["a"].shape == (3, 5)
    assert c.tensor_infos["b"].read_bytes(f, c.tensor_data_offset).tobytes() == qb.tobytes()
    assert c.tensor_infos["a"].read_bytes(f, c.tensor_data_offset).tobytes() == a.data().tobytes()


def test_metadata_values_round_trip():
    vals = [("u8", Value(ValueType.U8, 255)), ("i8", Value(ValueType.I8, -128)), ("u16", Value(ValueType.U16, 65535)),
            ("i16", Value(ValueType.I16, -2)), ("i32", Value(ValueType.I32, -7)), ("u64", Value(ValueType.U64, U64_MAX)),
            ("i64", Value(ValueType.I64, -(1 << 63))), ("f32", Value(ValueType.F32, 0.5)),
            ("f64", Value(ValueType.F64, -1e300)), ("t", Value(ValueType.Bool, True)),
            ("s", Value(ValueType.String, "ök")), ("empty", Value(ValueType.Array, [])),
            ("arr", Value(ValueType.Array, [Value(ValueType.Array, [Value(ValueType.String, "x")]),
                                            Value(ValueType.Array, [])]))]
    f = io.BytesIO()
    write(f, vals, [])
    c = Content.read(io.BytesIO(f.getvalue()))
    for k, v in vals:
        if k == "empty":                        # an empty array is written with element type U32
            assert c.metadata[k] == v
        else:
            assert c.metadata[k] == v, k
    with pytest.raises(GgufError, match="mixes element types"):
        write(io.BytesIO(), [("m", Value(ValueType.Array, [Value(ValueType.U8, 1), Value(ValueType.I8, 1)]))], [])


def test_file_type_geometry():
    """Block geometry for every id the reference reads (mod.rs:505-713)."""
    want = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 14: (256, 210), 15: (256, 292), 30: (1, 2),
            2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 10: (256, 84), 11: (256, 110), 13: (256, 176),
            20: (32, 18), 23: (256, 136), 39: (32, 17), 42: (64, 18), 1 << 24: (32, 34)}
    for i, (bs, ts) in want.items():
        ft = FileType(i)
        assert (ft.block_size(), ft.type_size()) == (bs, ts), ft
    for d in (GgmlDType.Q8_0, GgmlDType.Q4K, GgmlDType.Q6K, GgmlDType.F32, GgmlDType.F16, GgmlDType.BF16):
        assert (FileType(int(d)).block_size(), FileType(int(d)).type_size()) == (d.block_size(), d.type_size())


def test_upload_refusals_before_any_device_work():
    with pytest.raises(GgufError, match="the tensor needs"):
        qtensor_from_ggml(12, bytes(100), [1, 256], device="cpu")
    with pytest.raises(GgufError, match="rank-0"):
        qtensor_from_ggml(0, bytes(4), [], device="cpu")
    with pytest.raises(GgufError, match="innermost dim"):
        qtensor_from_ggml(8, bytes(68), [2, 34], device="cpu")
    with pytest.raises(LloomHipError, match="no kernel on the HIP arm"):
        qtensor_from_ggml(13, bytes(176), [1, 256], device="cpu")
    with pytest.raises(GgufError, match="no tensor named 'w'"):
        Content.read(io.BytesIO(header(0, 0))).tensor(io.BytesIO(header(0, 0)), "w", device="cpu")
