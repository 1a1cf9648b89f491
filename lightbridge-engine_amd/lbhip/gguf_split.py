"""GGUF split-shard sets and their ingestion straight into HBM.

``open_set`` mirrors crates/bridge-gguf-split/src/lib.rs:155-159: shard
discovery from any member's path (discovery.rs) and one tensor directory over
every shard (directory.rs), with the reference's checks and error variants:

* discovery: the entry must be a regular file whose canonical path stays in its
  lexical parent (symlinks may not escape); ``<prefix>-NNNNN-of-TTTTT.gguf``
  (exactly five digits each, 1 <= N <= T <= 65535) names a numbered set whose
  members are all looked up beside it, canonicalised, parsed and checked
  against their required ``split.no`` / ``split.count`` (u16) metadata; any
  other name is a single file whose optional split metadata must say 0 of 1;
* directory: every shard shares the primary's version, endianness and
  alignment; an optional ``split.tensors.count`` (i32, non-negative) must agree
  between shards and with the number of tensors; tensor names are unique across
  shards; the directory keeps shard order, then each shard's tensor order.

``ingest_set`` streams the chosen dot-typed 2-D tensors of a set to HBM with
``lbh_matrix_create_streamed``, each read with positioned reads from the shard
that holds it (crates/bridge-gguf-split/src/lib.rs: TensorLocation's shard
index and absolute range).
"""
from __future__ import annotations

import dataclasses
import os

from .gguf import _READER, GgufError, GgufFile, I32, U16, open_gguf

_VALUE_TYPE_NAMES = ["U8", "I8", "U16", "I16", "U32", "I32", "F32", "Bool", "String", "Array", "U64", "I64", "F64"]


class SplitError(Exception):
    """SplitError (crates/bridge-gguf-split/src/lib.rs:88-153): ``variant`` and its fields."""

    def __init__(self, variant: str, message: str = "", **fields):
        self.variant, self.fields = variant, fields
        super().__init__(message or (f"{variant} {fields}" if fields else variant))


def _debug_path(p) -> str:
    """A path as Rust's Debug formatting prints it (quoted, backslashes and quotes escaped)."""
    return '"' + str(p).replace("\\", "\\\\").replace('"', '\\"') + '"'


def get_typed(parsed: GgufFile, key: str, expected: int):
    """GgufFile::get_u16 / get_i32 / ... (crates/bridge-gguf/src/reader.rs:77-145):
    MetadataError::Missing or WrongType { key, expected, actual }."""
    for k, (ty, value) in parsed.metadata:
        if k == key:
            if ty != expected:
                raise GgufError("WrongType", f"GGUF metadata key {key!r} has type {_VALUE_TYPE_NAMES[ty]}, expected "
                                f"{_VALUE_TYPE_NAMES[expected]}", key=key, expected=expected, actual=ty)
            return value
    raise GgufError("Missing", f"missing GGUF metadata key {key!r}", key=key)


def _metadata_error(e: GgufError) -> SplitError:
    return SplitError("Metadata", str(e), error=e)


@dataclasses.dataclass
class GgufShard:
    path: str
    parsed: GgufFile
    ordinal: int
    count: int


@dataclasses.dataclass
class TensorLocation:
    shard_index: int
    descriptor: object
    absolute_range: range


class TensorDirectory:
    def __init__(self, ordered, by_name):
        self.ordered, self.by_name = ordered, by_name

    def get(self, name: str):
        i = self.by_name.get(name)
        return None if i is None else self.ordered[i]


@dataclasses.dataclass
class GgufSet:
    files: list
    tensors: TensorDirectory


# ----------------------------------------------------------------- discovery

def _parse_numbered(path: str):
    """NumberedName::parse (discovery.rs:150-180): (prefix, total) or None."""
    filename = os.path.basename(path)
    if not filename.endswith(".gguf"):
        return None
    stem = filename[: -len(".gguf")]
    if "-of-" not in stem:
        return None
    before_total, total_text = stem.rsplit("-of-", 1)
    if "-" not in before_total:
        return None
    prefix, ordinal_text = before_total.rsplit("-", 1)
    digits = set("0123456789")
    if len(ordinal_text) != 5 or len(total_text) != 5 or not set(ordinal_text) <= digits or \
            not set(total_text) <= digits:
        return None
    ordinal, total = int(ordinal_text), int(total_text)
    if ordinal == 0 or total == 0 or ordinal > total or total > 0xFFFF:
        raise SplitError("InvalidNumberedFilename", f"invalid numbered GGUF filename {filename!r}", name=filename)
    return prefix, total


def _numbered_filename(prefix: str, ordinal: int, total: int) -> str:
    return f"{prefix}-{ordinal:05d}-of-{total:05d}.gguf"


def _required_u16(path, parsed, key):
    try:
        return get_typed(parsed, key, U16)
    except GgufError as e:
        if e.variant == "Missing":
            raise SplitError("MissingSplitMetadata", f"numbered GGUF shard {_debug_path(path)} is missing required "
                             f"metadata {key!r}", path=path, key=key) from e
        raise _metadata_error(e) from e


def _optional_u16(parsed, key):
    try:
        return get_typed(parsed, key, U16)
    except GgufError as e:
        if e.variant == "Missing":
            return None
        raise _metadata_error(e) from e


def _disagreement(path, key):
    return SplitError("SplitMetadataDisagreement", f"numbered GGUF shard {_debug_path(path)} metadata {key!r} "
                      "does not match its filename", path=path, key=key)


def validate_required_split_metadata(path, parsed, ordinal: int, count: int) -> None:
    """discovery.rs:71-98."""
    no = _required_u16(path, parsed, "split.no")
    cnt = _required_u16(path, parsed, "split.count")
    if count == 1:
        raise SplitError("NumberedSingleShard", f"numbered GGUF shard {_debug_path(path)} declares only one shard",
                         path=path)
    if no != ordinal:
        raise _disagreement(path, "split.no")
    if cnt != count:
        raise _disagreement(path, "split.count")


def validate_optional_split_metadata(path, parsed, ordinal: int, count: int) -> None:
    """discovery.rs:100-124."""
    no = _optional_u16(parsed, "split.no")
    if no is not None and no != ordinal:
        raise _disagreement(path, "split.no")
    cnt = _optional_u16(parsed, "split.count")
    if cnt is not None and cnt != count:
        raise _disagreement(path, "split.count")


def discover(entry) -> list:
    """discovery::discover (discovery.rs:7-25)."""
    entry = os.fspath(entry)
    if not os.path.isfile(entry):
        raise SplitError("NotAFile", f"input path is not a regular file: {_debug_path(entry)}", path=entry)
    lexical_parent = os.path.realpath(os.path.dirname(entry) or ".")
    canonical = os.path.realpath(entry)
    if os.path.dirname(canonical) != lexical_parent:
        raise SplitError("ShardEscapesParent", f"canonical GGUF shard escapes its input parent directory: "
                         f"{_debug_path(canonical)}", path=canonical)
    numbered = _parse_numbered(canonical)
    if numbered is None:
        parsed = open_gguf(canonical)
        validate_optional_split_metadata(canonical, parsed, 0, 1)
        return [GgufShard(canonical, parsed, 0, 1)]
    prefix, total = numbered
    files = []
    for one_based in range(1, total + 1):
        expected = os.path.join(lexical_parent, _numbered_filename(prefix, one_based, total))
        if not os.path.isfile(expected):
            raise SplitError("MissingShard", f"expected GGUF shard is missing or is not a regular file: "
                             f"{_debug_path(expected)}", path=expected)
        path = os.path.realpath(expected)
        if os.path.dirname(path) != lexical_parent:
            raise SplitError("ShardEscapesParent", f"canonical GGUF shard escapes its input parent directory: "
                             f"{_debug_path(path)}", path=path)
        parsed = open_gguf(path)
        validate_required_split_metadata(path, parsed, one_based - 1, total)
        files.append(GgufShard(path, parsed, one_based - 1, total))
    return files


# ----------------------------------------------------------------- directory

_ENDIANNESS = {"little": "Little", "big": "Big"}


def _validate_common_fields(files) -> None:
    """directory.rs:60-88: every shard shares the primary's version, endianness and alignment."""
    if not files:
        return
    p = files[0].parsed
    for s in files[1:]:
        q = s.parsed
        if q.version != p.version:
            raise SplitError("HeterogeneousVersion", f"GGUF shard {_debug_path(s.path)} has version {q.version}, "
                             f"expected common version {p.version}", path=s.path, expected=p.version, actual=q.version)
        if q.endianness != p.endianness:
            raise SplitError("HeterogeneousEndianness", f"GGUF shard {_debug_path(s.path)} has endianness "
                             f"{_ENDIANNESS[q.endianness]}, expected common endianness {_ENDIANNESS[p.endianness]}",
                             path=s.path, expected=p.endianness, actual=q.endianness)
        if q.alignment != p.alignment:
            raise SplitError("HeterogeneousAlignment", f"GGUF shard {_debug_path(s.path)} has alignment "
                             f"{q.alignment}, expected common alignment {p.alignment}", path=s.path,
                             expected=p.alignment, actual=q.alignment)


def _optional_aggregate_count(shard):
    """directory.rs:90-97."""
    try:
        v = get_typed(shard.parsed, "split.tensors.count", I32)
    except GgufError as e:
        if e.variant == "Missing":
            return None
        raise _metadata_error(e) from e
    if v < 0:
        raise SplitError("NegativeAggregateTensorCount", f"aggregate split.tensors.count is negative in "
                         f"{_debug_path(shard.path)}", path=shard.path)
    return v


def build_directory(files) -> TensorDirectory:
    """directory::build (directory.rs:7-58)."""
    _validate_common_fields(files)
    ordered, by_name = [], {}
    declared = None
    for shard_index, shard in enumerate(files):
        count = _optional_aggregate_count(shard)
        if count is not None:
            if declared is not None and declared != count:
                raise SplitError("AggregateTensorCountDisagreement",
                                 "split.tensors.count disagrees between GGUF shards")
            declared = count if declared is None else declared
        g = shard.parsed
        for t in g.tensors:
            if t.relative_offset % g.alignment:
                raise SplitError("UnalignedTensorOffset", f"tensor {t.name!r} in {_debug_path(shard.path)} has "
                                 f"offset {t.relative_offset} not aligned to {g.alignment}", path=shard.path,
                                 name=t.name, offset=t.relative_offset, alignment=g.alignment)
            start = g.data_offset + t.relative_offset
            end = start + t.encoded_bytes()
            if end > g.file_len:   # TensorDesc::checked_absolute_range (bridge-core/src/tensor.rs)
                raise SplitError("Core", f"tensor {t.name!r} range {start}..{end} exceeds file length {g.file_len}",
                                 name=t.name)
            if t.name in by_name:
                raise SplitError("DuplicateTensorName", f"duplicate tensor name {t.name!r} across GGUF shards",
                                 name=t.name)
            by_name[t.name] = len(ordered)
            ordered.append(TensorLocation(shard_index, t, range(start, end)))
    if declared is not None and declared != len(ordered):
        raise SplitError("AggregateTensorDirectoryDisagreement",
                         "split.tensors.count does not match the aggregate tensor directory")
    return TensorDirectory(ordered, by_name)


def open_set(entry) -> GgufSet:
    """open_set (crates/bridge-gguf-split/src/lib.rs:155-159)."""
    try:
        files = discover(entry)
    except GgufError as e:
        raise SplitError("Gguf", str(e), error=e) from e
    return GgufSet(files, build_directory(files))


# ----------------------------------------------------------------- ingestion

def ingest_set(be, gset: GgufSet, names=None) -> dict:
    """Upload the named 2-D dot-typed tensors of a split set straight to HBM
    (lbh_matrix_create_streamed); each tensor's bytes are read from its shard
    with positioned reads.  Returns {name: DeviceMatrix}."""
    from . import DeviceMatrix
    fds = {}
    out = {}
    try:
        for loc in gset.tensors.ordered:
            t = loc.descriptor
            if names is not None and t.name not in names:
                continue
            if len(t.shape) != 2 or t.ggml_type not in (12, 13, 21, 22):
                continue
            path = gset.files[loc.shard_index].path
            if path not in fds:
                fds[path] = os.open(path, os.O_RDONLY)
            fd, base = fds[path], loc.absolute_range.start

            def read(user, off, dst, n, fd=fd, base=base):
                import ctypes as C
                try:
                    view = memoryview((C.c_uint8 * n).from_address(C.cast(dst, C.c_void_p).value)).cast("B")
                    return 0 if os.preadv(fd, [view], base + off) == n else 2
                except Exception:   # reported as SourceReadFailed
                    return 1

            out[t.name] = DeviceMatrix.streamed(be, t.ggml_type, t.shape[1], t.shape[0], _READER(read))
    finally:
        for fd in fds.values():
            os.close(fd)
    return out
