"""GGUF directory reader and the ingestion of its quantized tensors straight
into HBM.

``GgufReader.read`` mirrors crates/bridge-gguf/src/reader.rs:194-341: magic
(``GGUF`` little-endian or ``FUGG`` big-endian), version 2 or 3, counts checked
against ``ReaderLimits``, typed metadata with duplicate-key and budget checks,
``general.alignment``, tensor records (rank 1..4, block-aligned first
dimension, known GGML type) whose payload offsets must be the running padded
extent, and a data section that fits the file.  Errors are ``GgufError`` with
the reference variant and, where the reference's tests compare them, its
message.  Tensor descriptors follow crates/bridge-core/src/tensor.rs:21-97
and the GGML type table crates/bridge-core/src/ggml_type.rs.

``ingest`` uploads chosen tensors of a file with ``lbh_matrix_create_streamed``:
each tensor's payload is read with positioned reads into the library's pinned
chunks and repacked on the device, with no host copy of the tensor.
``write_gguf`` writes little-endian v3 files for tests and benchmarks.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os
import struct

DEFAULT_ALIGNMENT = 32
GGML_MAX_DIMENSIONS = 4

# GgmlType: discriminant -> (name, block elements, block bytes)  (ggml_type.rs)
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 19: ("IQ1_S", 256, 50),
    20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8),
    29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66),
    39: ("MXFP4", 32, 17), 40: ("NVFP4", 64, 36), 41: ("Q1_0", 128, 18), 42: ("Q2_0", 64, 18),
}

# GgufValueType (value.rs): code -> (name, struct format or None)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "B", I8: "b", U16: "H", I16: "h", U32: "I", I32: "i", F32: "f", U64: "Q", I64: "q", F64: "d"}
_MIN_BYTES = {U8: 1, I8: 1, BOOL: 1, U16: 2, I16: 2, U32: 4, I32: 4, F32: 4, STRING: 8, U64: 8, I64: 8, F64: 8}
_U64 = 1 << 64


class GgufError(Exception):
    """GgufError / CoreError (crates/bridge-gguf/src/error.rs, bridge-core/src/error.rs)."""

    def __init__(self, variant: str, message: str = "", **fields):
        self.variant, self.fields = variant, fields
        super().__init__(message or (f"{variant} {fields}" if fields else variant))


@dataclasses.dataclass(frozen=True)
class ReaderLimits:
    """ReaderLimits::default (reader.rs:22-43)."""
    max_dimensions: int = GGML_MAX_DIMENSIONS
    max_string_bytes: int = 1024 * 1024
    max_array_elements: int = 1_000_000
    max_tensors: int = 4_000_000
    max_metadata_entries: int = 1_000_000
    max_metadata_bytes: int = 64 * 1024 * 1024


@dataclasses.dataclass
class TensorDesc:
    """TensorDesc (tensor.rs:21-97): name, shape (ne, innermost first), type, payload offset."""
    name: str
    shape: tuple
    ggml_type: int
    relative_offset: int

    @property
    def type_name(self) -> str:
        return GGML_TYPES[self.ggml_type][0]

    def row_bytes(self) -> int:
        _, block, size = GGML_TYPES[self.ggml_type]
        return self.shape[0] // block * size

    def encoded_bytes(self) -> int:
        n = self.row_bytes()
        for d in self.shape[1:]:
            n *= d
        return n


@dataclasses.dataclass
class GgufFile:
    version: int
    endianness: str
    metadata: list          # [(key, (value_type, value))]
    tensors: list           # [TensorDesc]
    alignment: int
    data_offset: int
    file_len: int

    def get(self, key: str):
        for k, v in self.metadata:
            if k == key:
                return v[1]
        raise GgufError("Missing", f"missing GGUF metadata key {key!r}", key=key)

    def tensor(self, name: str) -> TensorDesc:
        for t in self.tensors:
            if t.name == name:
                return t
        raise GgufError("MissingTensor", f"no tensor {name!r}", name=name)

    def absolute_range(self, t: TensorDesc) -> range:
        start = self.data_offset + t.relative_offset
        return range(start, start + t.encoded_bytes())


class GgufReader:
    def __init__(self, f, limits: ReaderLimits = ReaderLimits()):
        self.f, self.limits = f, limits
        self.order = "<"
        self.metadata_bytes = 0
        self.array_elements = 0
        self.account = False

    # -- primitives ------------------------------------------------------------
    def _exact(self, n: int, context: str) -> bytes:
        if self.account:
            nxt = self.metadata_bytes + n
            if nxt > self.limits.max_metadata_bytes:
                raise GgufError("LimitExceeded", f"metadata bytes count {nxt} exceeds configured limit "
                                f"{self.limits.max_metadata_bytes}", kind="metadata bytes",
                                limit=self.limits.max_metadata_bytes, actual=nxt)
            self.metadata_bytes = nxt
        b = self.f.read(n)
        if len(b) != n:
            raise GgufError("Truncated", f"GGUF is truncated while reading {context}", context=context)
        return b

    def _u(self, fmt: str, context: str):
        return struct.unpack(self.order + fmt, self._exact(struct.calcsize(fmt), context))[0]

    def _count(self, actual: int, limit: int, kind: str) -> int:
        if actual > limit:
            raise GgufError("LimitExceeded", f"{kind} count {actual} exceeds configured limit {limit}",
                            kind=kind, limit=limit, actual=actual)
        return actual

    def _string(self, context: str) -> str:
        n = self._u("Q", "string length")
        if n > self.limits.max_string_bytes:
            raise GgufError("LimitExceeded", f"string bytes count {n} exceeds configured limit "
                            f"{self.limits.max_string_bytes}", kind="string bytes",
                            limit=self.limits.max_string_bytes, actual=n)
        raw = self._exact(n, context)
        try:
            return raw.decode("utf-8")
        except UnicodeDecodeError as e:
            raise GgufError("InvalidUtf8", f"invalid UTF-8 in {context}: {e}", context=context) from e

    def _value_type(self, code: int) -> int:
        if not 0 <= code <= 12:
            raise GgufError("UnknownValueType", f"unknown GGUF metadata value type {code}", code=code)
        return code

    def _value(self, ty: int):
        if ty == ARRAY:
            et = self._value_type(self._u("I", "array element type"))
            if et == ARRAY:
                raise GgufError("NestedArray", "GGUF arrays may not contain arrays")
            count = self._u("Q", "array element count")
            agg = self.array_elements + count
            if agg > self.limits.max_array_elements:
                raise GgufError("LimitExceeded", f"array elements count {agg} exceeds configured limit "
                                f"{self.limits.max_array_elements}", kind="array elements",
                                limit=self.limits.max_array_elements, actual=agg)
            floor = self.metadata_bytes + count * _MIN_BYTES[et]
            if floor > self.limits.max_metadata_bytes:
                raise GgufError("LimitExceeded", f"metadata bytes count {floor} exceeds configured limit "
                                f"{self.limits.max_metadata_bytes}", kind="metadata bytes",
                                limit=self.limits.max_metadata_bytes, actual=floor)
            self.array_elements = agg
            return (et, [self._value(et) for _ in range(count)])
        if ty == BOOL:
            b = self._u("B", "boolean metadata value")
            if b > 1:
                raise GgufError("InvalidBoolean", f"invalid GGUF boolean byte {b}", byte=b)
            return bool(b)
        if ty == STRING:
            return self._string("string metadata value")
        return self._u(_SCALAR[ty], f"{['u8','i8','u16','i16','u32','i32','f32','bool','string','array','u64','i64','f64'][ty]} metadata value")

    # -- the file ----------------------------------------------------------------
    def read(self) -> GgufFile:
        """GgufReader::read (reader.rs:194-341)."""
        if self.limits.max_dimensions > GGML_MAX_DIMENSIONS:
            raise GgufError("InvalidDimensionLimit", value=self.limits.max_dimensions)
        magic = self._exact(4, "magic")
        if magic == b"GGUF":
            self.order = "<"
        elif magic == b"FUGG":
            self.order = ">"
        else:
            raise GgufError("BadMagic", f"bad GGUF magic bytes {list(magic)}", magic=magic)
        version = self._u("I", "version")
        if version not in (2, 3):
            raise GgufError("UnsupportedVersion", f"unsupported GGUF version {version}", version=version)
        n_tensors = self._count(self._u("Q", "tensor count"), self.limits.max_tensors, "tensors")
        n_meta = self._count(self._u("Q", "metadata count"), self.limits.max_metadata_entries, "metadata entries")
        metadata, keys = [], set()
        self.account = True
        for _ in range(n_meta):
            key = self._string("metadata key")
            ty = self._value_type(self._u("I", "metadata value type"))
            value = self._value(ty)
            if key in keys:
                raise GgufError("DuplicateMetadataKey", f"duplicate GGUF metadata key {key!r}", key=key)
            keys.add(key)
            metadata.append((key, (ty, value)))
        self.account = False
        alignment = DEFAULT_ALIGNMENT
        for key, (ty, value) in metadata:
            if key == "general.alignment":
                if ty != U32:
                    raise GgufError("AlignmentWrongType", value_type=ty)
                if value == 0 or value & (value - 1):
                    raise GgufError("InvalidAlignment", f"general.alignment must be a positive u32 power of two, "
                                    f"got {value}", value=value)
                alignment = value
                break
        tensors = []
        for _ in range(n_tensors):
            self.account = True
            name = self._string("tensor name")
            self.account = False
            n_dims = self._u("I", "tensor dimension count")
            if not 1 <= n_dims <= GGML_MAX_DIMENSIONS:
                raise GgufError("InvalidDimensionCount", f"tensor dimension count {n_dims} is outside GGML's "
                                "supported 1..=4 dimensions", n_dims=n_dims)
            if n_dims > self.limits.max_dimensions:
                raise GgufError("LimitExceeded", kind="dimensions", limit=self.limits.max_dimensions, actual=n_dims)
            shape = tuple(self._u("Q", "tensor dimension") for _ in range(n_dims))
            code = self._u("I", "GGML type")
            if code not in GGML_TYPES:
                raise GgufError("UnknownGgmlType", value=code)
            offset = self._u("Q", "tensor payload offset")
            for i, d in enumerate(shape):
                if d == 0:
                    raise GgufError("ZeroTensorDimension", dimension=i)
            _, block, size = GGML_TYPES[code]
            if shape[0] % block:
                raise GgufError("NotBlockAligned", ne=shape[0], block=block, ty=GGML_TYPES[code][0])
            tensors.append(TensorDesc(name, shape, code, offset))
        directory_end = self.f.tell()
        data_offset = (directory_end + alignment - 1) // alignment * alignment
        self.f.seek(0, os.SEEK_END)
        file_len = self.f.tell()
        if data_offset > file_len:
            raise GgufError("DataOffsetBeyondFile", f"GGUF data offset {data_offset} exceeds physical file length "
                            f"{file_len}", data_offset=data_offset, file_len=file_len)
        extent = 0
        for t in tensors:
            if t.relative_offset != extent:
                raise GgufError("TensorOffsetMismatch", f"tensor {t.name!r}".replace("'", '"') +
                                f" has relative payload offset {t.relative_offset}, expected {extent} for "
                                f"{alignment}-byte alignment", name=t.name, actual_offset=t.relative_offset,
                                expected_offset=extent, alignment=alignment)
            enc = t.encoded_bytes()
            if enc >= _U64:
                raise GgufError("ArithmeticOverflow", what="tensor encoded byte length")
            padded = (enc + alignment - 1) // alignment * alignment
            if padded >= _U64:
                raise GgufError("TensorPaddingOverflow", f"tensor {t.name!r}".replace("'", '"') +
                                f" encoded byte length {enc} overflows {alignment}-byte padding",
                                name=t.name, encoded_bytes=enc, alignment=alignment)
            extent += padded
            if extent >= _U64:
                raise GgufError("TensorExtentOverflow", name=t.name)
            start = data_offset + t.relative_offset
            if start >= _U64 or start + enc >= _U64:
                raise GgufError("ArithmeticOverflow", what="tensor absolute offset")
            if start + enc > file_len:
                raise GgufError("TensorOutOfBounds", start=start, end=start + enc, file_len=file_len)
        required_end = data_offset + extent
        if required_end >= _U64:
            raise GgufError("TensorDataEndOverflow", data_offset=data_offset, padded_extent=extent)
        if required_end > file_len:
            raise GgufError("TensorDataSectionTruncated", f"GGUF tensor data section requires padded range "
                            f"{data_offset}..{required_end}, but physical file length is {file_len}",
                            data_offset=data_offset, required_end=required_end, file_len=file_len)
        return GgufFile(version, "little" if self.order == "<" else "big", metadata, tensors, alignment,
                        data_offset, file_len)


def open_gguf(path, limits: ReaderLimits = ReaderLimits()) -> GgufFile:
    """reader.rs:528-530."""
    with open(path, "rb") as f:
        return GgufReader(f, limits).read()


def write_gguf(path, metadata, tensors, alignment: int = DEFAULT_ALIGNMENT, version: int = 3) -> None:
    """Little-endian GGUF: `metadata` [(key, value_type, value)], `tensors`
    [(name, shape (ne, innermost first), ggml_type, payload bytes)] in payload order."""
    def s(x: str) -> bytes:
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    def val(ty, v) -> bytes:
        if ty == STRING:
            return s(v)
        if ty == BOOL:
            return struct.pack("<B", 1 if v else 0)
        if ty == ARRAY:
            et, items = v
            return struct.pack("<IQ", et, len(items)) + b"".join(val(et, x) for x in items)
        return struct.pack("<" + _SCALAR[ty], v)

    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata)))
    if alignment != DEFAULT_ALIGNMENT and not any(k == "general.alignment" for k, _, _ in metadata):
        metadata = list(metadata) + [("general.alignment", U32, alignment)]
        out[16:24] = struct.pack("<Q", len(metadata))
    for k, ty, v in metadata:
        out += s(k) + struct.pack("<I", ty) + val(ty, v)
    offset = 0
    payloads = []
    for name, shape, ty, data in tensors:
        out += s(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", ty, offset)
        payloads.append((offset, bytes(data)))
        offset += (len(data) + alignment - 1) // alignment * alignment
    data_offset = (len(out) + alignment - 1) // alignment * alignment
    out += b"\0" * (data_offset - len(out))
    with open(path, "wb") as f:
        f.write(out)
        for off, data in payloads:
            f.write(data)
            pad = (len(data) + alignment - 1) // alignment * alignment - len(data)
            f.write(b"\0" * pad)


_READER = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_uint64, C.POINTER(C.c_uint8), C.c_size_t)


def ingest(be, path, names=None) -> dict:
    """Upload the named 2-D dot-typed tensors of a GGUF file straight to HBM
    (lbh_matrix_create_streamed); returns {name: DeviceMatrix}."""
    from . import DeviceMatrix
    gf = open_gguf(path)
    fd = os.open(path, os.O_RDONLY)
    out = {}
    try:
        for t in gf.tensors:
            if names is not None and t.name not in names:
                continue
            if len(t.shape) != 2 or t.ggml_type not in (12, 13, 21, 22):
                continue
            base = gf.data_offset + t.relative_offset
            box: list = []

            def read(user, off, dst, n, base=base, box=box):
                try:
                    view = memoryview((C.c_uint8 * n).from_address(C.cast(dst, C.c_void_p).value)).cast("B")
                    got = os.preadv(fd, [view], base + off)
                    return 0 if got == n else 2
                except Exception as e:   # reported as SourceReadFailed
                    box.append(e)
                    return 1

            out[t.name] = DeviceMatrix.streamed(be, t.ggml_type, t.shape[1], t.shape[0], _READER(read))
    finally:
        os.close(fd)
    return out
