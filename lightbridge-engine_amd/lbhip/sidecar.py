"""Expert-major sidecar files: the on-disk format that feeds routed experts to
the HBM expert cache.

Mirror of crates/bridge-format/src/lib.rs (format version 1): a data file that
starts with a 64-byte header (magic ``LIGHTBRIDGE.EXP\\0``, format version,
layout code, alignment, record count; the rest zero, lib.rs:186-236) followed by
one aligned record per (layer, expert) holding that expert's gate, up and down
GGML bytes, and a JSON manifest (SidecarManifest, lib.rs:100-184) that binds
the records to their source files.  ``Sidecar.open`` / ``read_expert`` /
``verify_data_hash`` follow lib.rs:238-329; ``tight_record`` is the runtime's
read_tight (crates/bridge-runtime/src/hy3_scalar.rs:1040-1064): gate | up | down
back to back, the record an ``ExpertCache`` loader hands over.

``write_sidecar`` produces the layout bridge-prepare writes (records in key
order at aligned offsets; FusedGateUp keeps gate and up adjacent), so tests and
benchmarks can build sidecars from synthetic experts.
"""
from __future__ import annotations

import dataclasses
import hashlib
import json
import os
import re
from pathlib import Path

SIDECAR_FORMAT = "lightbridge-expert-sidecar"
SIDECAR_FORMAT_VERSION = 1
QUANT_ABI_VERSION = 1
SIDECAR_HEADER_BYTES = 64
MAX_MANIFEST_BYTES = 32 * 1024 * 1024
SIDECAR_MAGIC = b"LIGHTBRIDGE.EXP\0"

SEQUENTIAL, FUSED_GATE_UP = "sequential", "fused-gate-up"
LAYOUT_CODES = {SEQUENTIAL: 0, FUSED_GATE_UP: 1}
_SHA256 = re.compile(r"[0-9a-f]{64}")


class FormatError(Exception):
    """FormatError (lib.rs:454-504): ``variant`` names the reference variant."""

    def __init__(self, variant: str, **fields):
        self.variant, self.fields = variant, fields
        super().__init__(f"{variant} {fields}" if fields else variant)


class SidecarError(Exception):
    """SidecarError (lib.rs:506-534)."""

    def __init__(self, variant: str, **fields):
        self.variant, self.fields = variant, fields
        super().__init__(f"{variant} {fields}" if fields else variant)


def align_up(value: int, alignment: int) -> int:
    """lib.rs:352-362: checked power-of-two round-up."""
    if alignment <= 0 or alignment & (alignment - 1):
        raise FormatError("InvalidAlignment", alignment=alignment)
    out = (value + alignment - 1) & ~(alignment - 1)
    if out >= 1 << 64:
        raise FormatError("ArithmeticOverflow")
    return out


@dataclasses.dataclass(frozen=True, order=True)
class ExpertKey:
    layer: int
    expert: int


@dataclasses.dataclass
class Segment:
    offset: int
    length: int
    ggml_type: str

    def range(self) -> range:
        return range(self.offset, self.offset + self.length)


@dataclasses.dataclass
class ExpertRecord:
    key: ExpertKey
    offset: int
    length: int
    gate: Segment
    up: Segment
    down: Segment


@dataclasses.dataclass
class SidecarHeader:
    """SidecarHeader (lib.rs:186-236): 64 little-endian bytes."""

    layout: str
    alignment: int
    record_count: int
    format_version: int = SIDECAR_FORMAT_VERSION

    def encode(self) -> bytes:
        out = bytearray(SIDECAR_HEADER_BYTES)
        out[0:16] = SIDECAR_MAGIC
        out[16:20] = self.format_version.to_bytes(4, "little")
        out[20:24] = LAYOUT_CODES[self.layout].to_bytes(4, "little")
        out[24:32] = self.alignment.to_bytes(8, "little")
        out[32:40] = self.record_count.to_bytes(8, "little")
        return bytes(out)

    @staticmethod
    def decode(data: bytes) -> "SidecarHeader":
        if len(data) != SIDECAR_HEADER_BYTES:
            raise FormatError("HeaderLength", expected=SIDECAR_HEADER_BYTES, actual=len(data))
        if data[:16] != SIDECAR_MAGIC:
            raise FormatError("BadMagic")
        if any(data[40:]):
            raise FormatError("NonZeroReservedHeader")
        code = int.from_bytes(data[20:24], "little")
        layouts = {v: k for k, v in LAYOUT_CODES.items()}
        if code not in layouts:
            raise FormatError("UnknownLayout", code=code)
        return SidecarHeader(layout=layouts[code], alignment=int.from_bytes(data[24:32], "little"),
                             record_count=int.from_bytes(data[32:40], "little"),
                             format_version=int.from_bytes(data[16:20], "little"))


def _sha_ok(value: str, context: str) -> None:
    if not isinstance(value, str) or not _SHA256.fullmatch(value):
        raise FormatError("InvalidSha256", context=context, value=value)


@dataclasses.dataclass
class SidecarManifest:
    format: str
    format_version: int
    engine_version: str
    quant_abi_version: int
    alignment: int
    layout: str
    source_files: list          # [{"ordinal", "path", "length", "sha256"}]
    tensor_directory_sha256: str
    sidecar: dict               # {"length", "sha256"}
    records: list               # [ExpertRecord]

    def validate(self) -> None:
        """SidecarManifest::validate (lib.rs:114-178), in the reference's order."""
        if self.format != SIDECAR_FORMAT:
            raise FormatError("WrongFormat", format=self.format)
        if self.format_version != SIDECAR_FORMAT_VERSION:
            raise FormatError("WrongVersion", expected=SIDECAR_FORMAT_VERSION, actual=self.format_version)
        if self.quant_abi_version != QUANT_ABI_VERSION:
            raise FormatError("WrongQuantAbi", expected=QUANT_ABI_VERSION, actual=self.quant_abi_version)
        a = self.alignment
        if a < 32 or a & (a - 1):
            raise FormatError("InvalidAlignment", alignment=a)
        _sha_ok(self.tensor_directory_sha256, "tensor directory")
        _sha_ok(self.sidecar["sha256"], "sidecar")
        if self.sidecar["length"] < SIDECAR_HEADER_BYTES:
            raise FormatError("SidecarTooShort", length=self.sidecar["length"])
        if not self.source_files:
            raise FormatError("NoSourceFiles")
        for index, source in enumerate(self.source_files):
            if source["ordinal"] != index:
                raise FormatError("SourceOrdinal", index=index, actual=source["ordinal"])
            _sha_ok(source["sha256"], "source file")
        previous_key, previous_end = None, align_up(SIDECAR_HEADER_BYTES, a)
        for r in self.records:
            if previous_key is not None and previous_key >= r.key:
                raise FormatError("RecordsNotStrictlyOrdered", key=r.key)
            if r.offset % a:
                raise FormatError("UnalignedRecord", key=r.key, offset=r.offset, alignment=a)
            end = r.offset + r.length
            if r.offset < previous_end or end > self.sidecar["length"]:
                raise FormatError("RecordOutOfBounds", key=r.key, start=r.offset, end=end, minimum=previous_end,
                                  sidecar_length=self.sidecar["length"])
            _validate_segments(r, self.layout, a)
            previous_key, previous_end = r.key, end

    def record(self, key: ExpertKey) -> ExpertRecord | None:
        for r in self.records:   # records are strictly ordered; a scan is enough at these sizes
            if r.key == key:
                return r
        return None

    def to_json(self) -> bytes:
        def seg(s):
            return {"offset": s.offset, "length": s.length, "ggml_type": s.ggml_type}
        doc = {"format": self.format, "format_version": self.format_version, "engine_version": self.engine_version,
               "quant_abi_version": self.quant_abi_version, "alignment": self.alignment, "layout": self.layout,
               "source_files": self.source_files, "tensor_directory_sha256": self.tensor_directory_sha256,
               "sidecar": self.sidecar,
               "records": [{"key": {"layer": r.key.layer, "expert": r.key.expert}, "offset": r.offset,
                            "length": r.length, "gate": seg(r.gate), "up": seg(r.up), "down": seg(r.down)}
                           for r in self.records]}
        return json.dumps(doc, indent=2).encode()

    @staticmethod
    def from_json(data: bytes) -> "SidecarManifest":
        try:
            d = json.loads(data)
            seg = lambda s: Segment(int(s["offset"]), int(s["length"]), str(s["ggml_type"]))  # noqa: E731
            recs = [ExpertRecord(ExpertKey(int(r["key"]["layer"]), int(r["key"]["expert"])), int(r["offset"]),
                                 int(r["length"]), seg(r["gate"]), seg(r["up"]), seg(r["down"])) for r in d["records"]]
            if d["layout"] not in LAYOUT_CODES:
                raise ValueError(f"unknown layout {d['layout']!r}")
            return SidecarManifest(d["format"], int(d["format_version"]), d["engine_version"],
                                   int(d["quant_abi_version"]), int(d["alignment"]), d["layout"], d["source_files"],
                                   d["tensor_directory_sha256"], d["sidecar"], recs)
        except (ValueError, KeyError, TypeError) as e:
            raise SidecarError("ManifestJson", detail=str(e)) from e


def _validate_segments(r: ExpertRecord, layout: str, alignment: int) -> None:
    """validate_record_segments (lib.rs:364-424)."""
    lo, hi = r.offset, r.offset + r.length
    for name, s in (("gate", r.gate), ("up", r.up), ("down", r.down)):
        if s.length == 0 or s.offset < lo or s.offset + s.length > hi:
            raise FormatError("SegmentOutOfBounds", key=r.key, segment=name)
    if not (r.gate.offset + r.gate.length <= r.up.offset and r.up.offset + r.up.length <= r.down.offset):
        raise FormatError("OverlappingSegments", key=r.key)
    if layout == SEQUENTIAL:
        if any(s.offset % alignment for s in (r.gate, r.up, r.down)):
            raise FormatError("UnalignedSegment", key=r.key)
    elif (r.gate.offset != r.offset or r.up.offset != r.gate.offset + r.gate.length
          or r.down.offset % alignment):
        raise FormatError("InvalidFusedLayout", key=r.key)


@dataclasses.dataclass
class ExpertBytes:
    """ExpertBytes (lib.rs:331-350): the record and its three segments."""
    record: bytes
    gate: memoryview
    up: memoryview
    down: memoryview


class Sidecar:
    """Sidecar::open / read_expert / verify_data_hash (lib.rs:238-329)."""

    def __init__(self, data_path, manifest_path):
        manifest_path = Path(manifest_path)
        if not manifest_path.is_file():
            raise SidecarError("ManifestNotAFile", path=str(manifest_path))
        size = manifest_path.stat().st_size
        if size > MAX_MANIFEST_BYTES:
            raise SidecarError("ManifestTooLarge", actual=size, maximum=MAX_MANIFEST_BYTES)
        self.manifest = SidecarManifest.from_json(manifest_path.read_bytes())
        self.manifest.validate()
        self.path = Path(data_path)
        length = self.path.stat().st_size
        if length != self.manifest.sidecar["length"]:
            raise SidecarError("DataLength", expected=self.manifest.sidecar["length"], actual=length)
        self._f = open(self.path, "rb")
        header = SidecarHeader.decode(os.pread(self._f.fileno(), SIDECAR_HEADER_BYTES, 0))
        m = self.manifest
        if (header.format_version != m.format_version or header.layout != m.layout or header.alignment != m.alignment
                or header.record_count != len(m.records)):
            raise SidecarError("HeaderManifestMismatch")

    def read_expert(self, key: ExpertKey) -> ExpertBytes:
        r = self.manifest.record(key)
        if r is None:
            raise SidecarError("MissingExpert", key=key)
        data = os.pread(self._f.fileno(), r.length, r.offset)
        if len(data) != r.length:
            raise SidecarError("Read", detail=f"short read of {key}")
        mv = memoryview(data)
        cut = lambda s: mv[s.offset - r.offset:s.offset - r.offset + s.length]  # noqa: E731
        return ExpertBytes(data, cut(r.gate), cut(r.up), cut(r.down))

    def read_into(self, key: ExpertKey, dst: memoryview) -> int:
        """The tight record of `key` (gate | up | down) written into `dst`, read
        straight from the file (one positioned read per segment); returns its length."""
        r = self.manifest.record(key)
        if r is None:
            raise SidecarError("MissingExpert", key=key)
        total = r.gate.length + r.up.length + r.down.length
        if total > len(dst):
            return total   # the caller reports the length mismatch; nothing written
        pos = 0
        for s in (r.gate, r.up, r.down):
            n = os.preadv(self._f.fileno(), [dst[pos:pos + s.length]], s.offset)
            if n != s.length:
                raise SidecarError("Read", detail=f"short read of {key}")
            pos += s.length
        return pos

    def tight_record(self, key: ExpertKey) -> bytes:
        e = self.read_expert(key)
        return bytes(e.gate) + bytes(e.up) + bytes(e.down)

    def verify_data_hash(self) -> None:
        h = hashlib.sha256()
        with open(self.path, "rb") as f:
            for chunk in iter(lambda: f.read(8 << 20), b""):
                h.update(chunk)
        if h.hexdigest() != self.manifest.sidecar["sha256"]:
            raise SidecarError("DataHash", expected=self.manifest.sidecar["sha256"], actual=h.hexdigest())

    def close(self) -> None:
        if self._f:
            self._f.close()
            self._f = None


def write_sidecar(data_path, manifest_path, experts, layout: str = FUSED_GATE_UP, alignment: int = 4096,
                  source_files=None, engine_version: str = "lightbridge-engine-amd") -> SidecarManifest:
    """Write a sidecar: `experts` is a list of (ExpertKey, (gate, up, down) bytes,
    (gate_type, up_type, down_type) names) in any order; records go in key order."""
    experts = sorted(experts, key=lambda e: e[0])
    records, pos = [], align_up(SIDECAR_HEADER_BYTES, alignment)
    body = []
    for key, (g, u, d), (tg, tu, td) in experts:
        start = align_up(pos, alignment)
        if layout == SEQUENTIAL:
            og = start
            ou = align_up(og + len(g), alignment)
        else:
            og = start
            ou = og + len(g)
        od = align_up(ou + len(u), alignment)
        end = od + len(d)
        records.append(ExpertRecord(key, start, end - start, Segment(og, len(g), tg), Segment(ou, len(u), tu),
                                    Segment(od, len(d), td)))
        body.append(((og, g), (ou, u), (od, d)))
        pos = end
    header = SidecarHeader(layout, alignment, len(records)).encode()
    h = hashlib.sha256()
    with open(data_path, "wb") as f:
        f.write(header)
        cur = SIDECAR_HEADER_BYTES
        for segs in body:
            for off, blob in segs:
                if off > cur:
                    pad = b"\0" * (off - cur)
                    f.write(pad)
                f.write(bytes(blob))
                cur = off + len(blob)
    with open(data_path, "rb") as f:
        for chunk in iter(lambda: f.read(8 << 20), b""):
            h.update(chunk)
    sources = source_files or [{"ordinal": 0, "path": "synthetic.gguf", "length": 0, "sha256": "0" * 64}]
    m = SidecarManifest(SIDECAR_FORMAT, SIDECAR_FORMAT_VERSION, engine_version, QUANT_ABI_VERSION, alignment, layout,
                        sources, "0" * 64, {"length": cur, "sha256": h.hexdigest()}, records)
    m.validate()
    Path(manifest_path).write_bytes(m.to_json())
    return m
