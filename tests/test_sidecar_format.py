"""The expert-major sidecar format on the CPU (lbhip.sidecar, mirror of
crates/bridge-format/src/lib.rs): the reference's own manifest tests
(crates/bridge-format/tests/manifest.rs) restated, plus a write -> open ->
read_expert / read_into round trip of synthetic experts in both layouts."""
import copy

import numpy as np
import pytest

from lbhip import sidecar as sc
from lbhip import synth

SHA = "a" * 64


def manifest(layout):
    """The fixture of manifest.rs:11-57."""
    up_off, down_off = (96, 128) if layout == sc.SEQUENTIAL else (80, 128)
    rec = sc.ExpertRecord(sc.ExpertKey(1, 0), 64, 96, sc.Segment(64, 16, "IQ2_S"), sc.Segment(up_off, 16, "IQ2_S"),
                          sc.Segment(down_off, 16, "IQ3_S"))
    return sc.SidecarManifest(sc.SIDECAR_FORMAT, sc.SIDECAR_FORMAT_VERSION, "0.1.0", sc.QUANT_ABI_VERSION, 32, layout,
                              [{"ordinal": 0, "path": "model.gguf", "length": 1024, "sha256": SHA}], SHA,
                              {"length": 160, "sha256": SHA}, [rec])


def test_validates_both_supported_layouts():
    manifest(sc.SEQUENTIAL).validate()
    manifest(sc.FUSED_GATE_UP).validate()


def test_header_round_trips_and_rejects_reserved_bytes():
    h = sc.SidecarHeader(sc.FUSED_GATE_UP, 4096, 15_168)
    assert sc.SidecarHeader.decode(h.encode()) == h
    b = bytearray(h.encode())
    b[63] = 1
    with pytest.raises(sc.FormatError) as e:
        sc.SidecarHeader.decode(bytes(b))
    assert e.value.variant == "NonZeroReservedHeader"


def test_header_bytes_are_the_documented_layout():
    raw = sc.SidecarHeader(sc.SEQUENTIAL, 64, 3).encode()
    assert len(raw) == 64 and raw[:16] == b"LIGHTBRIDGE.EXP\0"
    assert raw[16:20] == (1).to_bytes(4, "little") and raw[20:24] == (0).to_bytes(4, "little")
    assert raw[24:32] == (64).to_bytes(8, "little") and raw[32:40] == (3).to_bytes(8, "little")
    with pytest.raises(sc.FormatError, match="BadMagic"):
        sc.SidecarHeader.decode(b"X" + raw[1:])


def test_manifest_rejects_overlap_and_bad_hashes():
    bad = manifest(sc.SEQUENTIAL)
    bad.records[0].up.offset = 64
    with pytest.raises(sc.FormatError) as e:
        bad.validate()
    assert e.value.variant == "OverlappingSegments"
    bad = manifest(sc.SEQUENTIAL)
    bad.tensor_directory_sha256 = "ABC"
    with pytest.raises(sc.FormatError) as e:
        bad.validate()
    assert e.value.variant == "InvalidSha256"


@pytest.mark.parametrize("mutate,variant", [
    (lambda m: setattr(m, "format", "other"), "WrongFormat"),
    (lambda m: setattr(m, "format_version", 2), "WrongVersion"),
    (lambda m: setattr(m, "quant_abi_version", 9), "WrongQuantAbi"),
    (lambda m: setattr(m, "alignment", 48), "InvalidAlignment"),
    (lambda m: setattr(m, "source_files", []), "NoSourceFiles"),
    (lambda m: m.sidecar.update(length=63), "SidecarTooShort"),
    (lambda m: m.records.append(copy.deepcopy(m.records[0])), "RecordsNotStrictlyOrdered"),
    (lambda m: setattr(m.records[0], "offset", 65), "UnalignedRecord"),
    (lambda m: setattr(m.records[0], "length", 200), "RecordOutOfBounds"),
    (lambda m: setattr(m.records[0].down, "length", 0), "SegmentOutOfBounds"),
    (lambda m: setattr(m.records[0].up, "offset", 97), "UnalignedSegment"),
])
def test_manifest_validation_variants(mutate, variant):
    m = manifest(sc.SEQUENTIAL)
    mutate(m)
    with pytest.raises(sc.FormatError) as e:
        m.validate()
    assert e.value.variant == variant


def test_fused_layout_requires_adjacent_gate_and_up():
    m = manifest(sc.FUSED_GATE_UP)
    m.records[0].up.offset = 96
    with pytest.raises(sc.FormatError) as e:
        m.validate()
    assert e.value.variant == "InvalidFusedLayout"


def test_checked_alignment():
    assert sc.align_up(64, 4096) == 4096
    with pytest.raises(sc.FormatError, match="InvalidAlignment"):
        sc.align_up(1, 3)
    with pytest.raises(sc.FormatError, match="ArithmeticOverflow"):
        sc.align_up(2**64 - 1, 4096)


def _experts(n, hidden=512, ffn=256, seed=0):
    out = []
    for e in range(n):
        g = synth.random_matrix(synth.IQ2_S, ffn, hidden, seed + 3 * e)
        u = synth.random_matrix(synth.IQ2_S, ffn, hidden, seed + 3 * e + 1)
        d = synth.random_matrix(synth.IQ3_S, hidden, ffn, seed + 3 * e + 2)
        out.append((sc.ExpertKey(3, e), (g.tobytes(), u.tobytes(), d.tobytes()), ("IQ2_S", "IQ2_S", "IQ3_S")))
    return out


@pytest.mark.parametrize("layout,alignment", [(sc.SEQUENTIAL, 64), (sc.FUSED_GATE_UP, 4096)])
def test_write_open_read_round_trip(tmp_path, layout, alignment):
    experts = _experts(5)
    m = sc.write_sidecar(tmp_path / "x.sidecar", tmp_path / "x.json", list(reversed(experts)), layout, alignment)
    assert [r.key for r in m.records] == [e[0] for e in experts]
    s = sc.Sidecar(tmp_path / "x.sidecar", tmp_path / "x.json")
    s.verify_data_hash()
    for key, (g, u, d), _ in experts:
        eb = s.read_expert(key)
        assert bytes(eb.gate) == g and bytes(eb.up) == u and bytes(eb.down) == d
        tight = s.tight_record(key)
        assert tight == g + u + d
        buf = bytearray(len(tight))
        assert s.read_into(key, memoryview(buf)) == len(tight) and bytes(buf) == tight
        assert s.read_into(key, memoryview(bytearray(10))) == len(tight)   # too small: nothing written
    with pytest.raises(sc.SidecarError, match="MissingExpert"):
        s.read_expert(sc.ExpertKey(3, 99))
    s.close()


def test_open_detects_tampering(tmp_path):
    sc.write_sidecar(tmp_path / "x.sidecar", tmp_path / "x.json", _experts(2), sc.FUSED_GATE_UP, 256)
    data = bytearray((tmp_path / "x.sidecar").read_bytes())
    data[300] ^= 1
    (tmp_path / "x.sidecar").write_bytes(bytes(data))
    s = sc.Sidecar(tmp_path / "x.sidecar", tmp_path / "x.json")
    with pytest.raises(sc.SidecarError, match="DataHash"):
        s.verify_data_hash()
    (tmp_path / "x.sidecar").write_bytes(bytes(data) + b"\0")
    with pytest.raises(sc.SidecarError, match="DataLength"):
        sc.Sidecar(tmp_path / "x.sidecar", tmp_path / "x.json")
    hdr = bytearray(data)
    hdr[32] = 7   # record count disagrees with the manifest
    (tmp_path / "x.sidecar").write_bytes(bytes(hdr))
    with pytest.raises(sc.SidecarError, match="HeaderManifestMismatch"):
        sc.Sidecar(tmp_path / "x.sidecar", tmp_path / "x.json")
