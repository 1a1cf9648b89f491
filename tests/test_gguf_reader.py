"""The GGUF directory reader on the CPU (lbhip.gguf, mirror of
crates/bridge-gguf/src/reader.rs): the reference's reader tests
(crates/bridge-gguf/tests/reader.rs) restated with an equivalent byte-level
fixture builder, plus write_gguf -> open_gguf round trips."""
import struct

import numpy as np
import pytest

from lbhip import gguf as gg
from lbhip import synth


class Fixture:
    """GGUF bytes: header, metadata records, tensor records, padding to 32, payload."""

    def __init__(self, version=3, order="<"):
        self.version, self.order, self.meta, self.tens, self.payload = version, order, [], [], b""

    def _s(self, b: bytes) -> bytes:
        return struct.pack(self.order + "Q", len(b)) + b

    def metadata(self, key: bytes, ty: int, value: bytes):
        self.meta.append(self._s(key) + struct.pack(self.order + "I", ty) + value)
        return self

    def tensor(self, name: bytes, dims, ty: int, offset: int):
        rec = self._s(name) + struct.pack(self.order + "I", len(dims))
        rec += b"".join(struct.pack(self.order + "Q", d) for d in dims) + struct.pack(self.order + "IQ", ty, offset)
        self.tens.append(rec)
        return self

    def with_payload(self, b: bytes):
        self.payload += b
        return self

    def bytes(self) -> bytes:
        magic = b"GGUF" if self.order == "<" else b"FUGG"
        out = magic + struct.pack(self.order + "IQQ", self.version, len(self.tens), len(self.meta))
        out += b"".join(self.meta) + b"".join(self.tens)
        out += b"\0" * ((-len(out)) % 32)
        return out + self.payload


def read(data: bytes, limits=gg.ReaderLimits()):
    import io
    return gg.GgufReader(io.BytesIO(data), limits).read()


def test_reads_minimal_little_endian_v3():
    f = read(Fixture().tensor(b"x", [1], 0, 0).with_payload(bytes(32)).bytes())
    assert (f.version, f.endianness, f.alignment, f.data_offset, f.file_len) == (3, "little", 32, 64, 96)
    assert [t.name for t in f.tensors] == ["x"] and f.tensors[0].shape == (1,)


def test_reads_exactly_aligned_tensor_directory():
    f = read(Fixture().tensor(b"12345678", [1], 0, 0).with_payload(bytes(32)).bytes())
    assert f.data_offset == 64 and f.file_len == 96 and f.tensors[0].name == "12345678"


@pytest.mark.parametrize("records,payload,message", [
    ([(b"first", [1], 0), (b"alias", [1], 0)], 64,
     'tensor "alias" has relative payload offset 0, expected 32 for 32-byte alignment'),
    ([(b"wide", [9], 0), (b"overlap", [1], 32)], 96,
     'tensor "overlap" has relative payload offset 32, expected 64 for 32-byte alignment'),
    ([(b"first", [1], 0), (b"after-gap", [1], 64)], 96,
     'tensor "after-gap" has relative payload offset 64, expected 32 for 32-byte alignment'),
    ([(b"first", [1], 32)], 64, 'tensor "first" has relative payload offset 32, expected 0 for 32-byte alignment'),
    ([(b"second", [1], 32), (b"first", [1], 0)], 64,
     'tensor "second" has relative payload offset 32, expected 0 for 32-byte alignment'),
])
def test_rejects_payload_offsets_off_the_padded_extent(records, payload, message):
    fx = Fixture()
    for name, dims, off in records:
        fx.tensor(name, dims, 0, off)
    with pytest.raises(gg.GgufError) as e:
        read(fx.with_payload(bytes(payload)).bytes())
    assert e.value.variant == "TensorOffsetMismatch" and str(e.value) == message


def test_rejects_truncated_final_tensor_padding():
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().tensor(b"x", [1], 0, 0).with_payload(bytes(4)).bytes())
    assert str(e.value) == "GGUF tensor data section requires padded range 64..96, but physical file length is 68"


def test_rejects_overflow_while_padding_a_tensor_extent():
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().tensor(b"huge", [2**64 - 1], 24, 0).bytes())
    assert str(e.value) == 'tensor "huge" encoded byte length 18446744073709551615 overflows 32-byte padding'


def test_accepts_mixed_types_at_exact_padded_offsets_and_trailing_bytes():
    f = read(Fixture().tensor(b"float", [1], 0, 0).tensor(b"quant", [256], 12, 32).tensor(b"bytes", [7], 24, 192)
             .with_payload(bytes(231)).bytes())
    assert [t.encoded_bytes() for t in f.tensors] == [4, 144, 7]
    assert f.file_len == f.data_offset + 224 + 7


def test_reads_minimal_v2_and_big_endian():
    f = read(Fixture(2).bytes())
    assert f.version == 2 and f.endianness == "little"
    f = read(Fixture(3, ">").metadata(b"answer", 4, struct.pack(">I", 42)).bytes())
    assert f.endianness == "big" and f.get("answer") == 42


def test_rejects_bad_magic_and_unsupported_versions():
    b = bytearray(Fixture().bytes())
    b[:4] = b"NOPE"
    with pytest.raises(gg.GgufError, match="bad GGUF magic"):
        read(bytes(b))
    for v in (1, 4):
        with pytest.raises(gg.GgufError) as e:
            read(Fixture(v).bytes())
        assert e.value.variant == "UnsupportedVersion" and e.value.fields["version"] == v


def test_rejects_truncated_scalars_strings_arrays_and_tensor_records():
    cases = [Fixture().metadata(b"k", 10, bytes(7)).bytes()[:44],
             Fixture().metadata(b"k", 8, struct.pack("<Q", 4) + b"abc").bytes()[:48],
             Fixture().metadata(b"k", 9, struct.pack("<IQ", 4, 1) + bytes(3)).bytes()[:52],
             Fixture().tensor(b"x", [1], 0, 0).bytes()[:56]]
    for data in cases:
        with pytest.raises(gg.GgufError) as e:
            read(data)
        assert e.value.variant == "Truncated"


def test_limits_utf8_booleans_types_and_dimensions():
    with pytest.raises(gg.GgufError, match="LimitExceeded|exceeds"):
        read(Fixture().tensor(b"a", [1], 0, 0).tensor(b"b", [1], 0, 32).with_payload(bytes(64)).bytes(),
             gg.ReaderLimits(max_tensors=1))
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().metadata(b"k", 8, struct.pack("<Q", 2) + b"\xff\xfe").bytes())
    assert e.value.variant == "InvalidUtf8"
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().metadata(b"k", 7, b"\x02").bytes())
    assert e.value.variant == "InvalidBoolean"
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().metadata(b"k", 13, b"").bytes())
    assert e.value.variant == "UnknownValueType"
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().metadata(b"k", 9, struct.pack("<IQ", 9, 0)).bytes())
    assert e.value.variant == "NestedArray"
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().tensor(b"x", [1], 31, 0).bytes())
    assert e.value.variant == "UnknownGgmlType"
    for dims in ([], [1, 1, 1, 1, 1]):
        with pytest.raises(gg.GgufError) as e:
            read(Fixture().tensor(b"x", dims, 0, 0).bytes())
        assert e.value.variant == "InvalidDimensionCount"
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().tensor(b"q", [255, 2], 12, 0).bytes())
    assert e.value.variant == "NotBlockAligned"
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().metadata(b"k", 4, struct.pack("<I", 1)).metadata(b"k", 4, struct.pack("<I", 2)).bytes())
    assert e.value.variant == "DuplicateMetadataKey"
    with pytest.raises(gg.GgufError) as e:
        read(Fixture().metadata(b"general.alignment", 4, struct.pack("<I", 48)).bytes())
    assert e.value.variant == "InvalidAlignment"


def test_metadata_budget_counts_keys_and_values():
    limits = gg.ReaderLimits(max_metadata_bytes=40)
    ok = Fixture().metadata(b"k", 8, struct.pack("<Q", 8) + b"12345678").bytes()   # 8+1+4+8+8 = 29 bytes
    read(ok, limits)
    big = Fixture().metadata(b"k", 8, struct.pack("<Q", 20) + b"x" * 20).bytes()   # 41 bytes
    with pytest.raises(gg.GgufError) as e:
        read(big, limits)
    assert e.value.variant == "LimitExceeded" and e.value.fields["kind"] == "metadata bytes"


def test_write_then_open_round_trip(tmp_path):
    q4 = synth.random_matrix(synth.Q4_K, 64, 512, 3)
    iq = synth.random_matrix(synth.IQ2_S, 32, 1024, 4)
    meta = [("general.architecture", gg.STRING, "hy3"), ("hy3.expert_count", gg.U32, 192),
            ("tokens", gg.ARRAY, (gg.STRING, ["a", "bc"])), ("scale", gg.F32, 2.5)]
    gg.write_gguf(tmp_path / "m.gguf", meta, [("blk.0.attn_v.weight", (512, 64), synth.Q4_K, q4.tobytes()),
                                              ("blk.0.ffn_gate.weight", (1024, 32), synth.IQ2_S, iq.tobytes())],
                  alignment=64)
    f = gg.open_gguf(tmp_path / "m.gguf")
    assert f.alignment == 64 and f.get("hy3.expert_count") == 192 and f.get("tokens") == (gg.STRING, ["a", "bc"])
    data = (tmp_path / "m.gguf").read_bytes()
    for t, want in zip(f.tensors, (q4, iq)):
        r = f.absolute_range(t)
        assert np.array_equal(np.frombuffer(data[r.start:r.stop], np.uint8), want.reshape(-1))
