"""GGUF split-shard sets on the CPU (lbhip.gguf_split, mirror of
crates/bridge-gguf-split): the reference's tests (crates/bridge-gguf-split/
tests/splits.rs and the testing helpers' unit tests) restated with an
equivalent byte-level fixture writer: discovery from any member, ordering by
ordinal, missing / misnamed / contradictory shards, symlinks that escape the
entry's directory, the aggregate tensor count, duplicate names across shards,
and the heterogeneous version / endianness / alignment messages."""
import os
import struct

import pytest

from lbhip import gguf as gg
from lbhip import gguf_split as gs


class Fixture:
    """Fixture of splits.rs:80-181: metadata records (key, value type, raw value
    bytes), rank-1 F32 tensor records at given payload offsets, zero padding to
    the alignment and `payload_bytes` of zero payload."""

    def __init__(self):
        self.order, self.version, self.meta, self.tensors = "<", 3, [], []
        self.payload, self.align = 0, 32

    def _u(self, fmt, v):
        return struct.pack(self.order + fmt, v)

    def big_endian(self):
        self.order = ">"
        return self

    def with_version(self, v):
        self.version = v
        return self

    def alignment(self, a):
        self.meta.append(("general.alignment", 4, self._u("I", a)))
        self.align = a
        return self

    def split(self, ordinal, count):
        self.meta.append(("split.no", 2, self._u("H", ordinal)))
        self.meta.append(("split.count", 2, self._u("H", count)))
        return self

    def split_count(self, count):
        self.meta.append(("split.tensors.count", 5, self._u("i", count)))
        return self

    def metadata(self, key, ty, raw):
        self.meta.append((key, ty, raw))
        return self

    def tensor(self, name, offset):
        self.tensors.append((name, offset))
        self.payload = max(self.payload, offset + self.align)
        return self

    def payload_bytes(self, n):
        self.payload = n
        return self

    def write(self, path):
        def s(x):
            b = x.encode()
            return self._u("Q", len(b)) + b
        out = (b"GGUF" if self.order == "<" else b"FUGG") + self._u("I", self.version)
        out += self._u("Q", len(self.tensors)) + self._u("Q", len(self.meta))
        for k, ty, raw in self.meta:
            out += s(k) + self._u("I", ty) + raw
        for name, off in self.tensors:
            out += s(name) + self._u("I", 1) + self._u("Q", 1) + self._u("I", 0) + self._u("Q", off)
        data = (len(out) + self.align - 1) // self.align * self.align
        out += b"\0" * (data - len(out) + self.payload)
        with open(path, "wb") as f:
            f.write(out)
        return path


def F():
    return Fixture()


def write(d, name, fx):
    return fx.write(os.path.join(d, name))


def err(entry):
    with pytest.raises(gs.SplitError) as e:
        gs.open_set(entry)
    return e.value


def test_opens_an_ordinary_non_numbered_single_file(tmp_path):
    s = gs.open_set(write(tmp_path, "model.gguf", F().tensor("only", 0)))
    assert len(s.files) == 1 and s.files[0].ordinal == 0 and s.files[0].count == 1
    assert s.tensors.ordered[0].descriptor.name == "only"


def test_accepts_any_numbered_member_and_orders_shards_by_ordinal(tmp_path):
    write(tmp_path, "name-00003-of-00003.gguf", F().split(2, 3).tensor("third", 0))
    entry = write(tmp_path, "name-00001-of-00003.gguf", F().split(0, 3).tensor("first", 0))
    write(tmp_path, "name-00002-of-00003.gguf", F().split(1, 3).tensor("second", 0))
    s = gs.open_set(tmp_path / "name-00003-of-00003.gguf")
    assert [f.ordinal for f in s.files] == [0, 1, 2]
    assert [loc.descriptor.name for loc in s.tensors.ordered] == ["first", "second", "third"]
    assert s.files[0].path == os.path.realpath(entry)
    assert s.tensors.get("second").shard_index == 1 and s.tensors.get("nope") is None


def test_rejects_missing_expected_shard(tmp_path):
    entry = write(tmp_path, "name-00001-of-00003.gguf", F().split(0, 3))
    write(tmp_path, "name-00003-of-00003.gguf", F().split(2, 3))
    assert err(entry).variant == "MissingShard"


@pytest.mark.parametrize("name,fx", [("name-00000-of-00003.gguf", lambda: F().split(0, 3)),
                                     ("name-00004-of-00003.gguf", lambda: F().split(3, 3))])
def test_rejects_zero_or_too_large_filename_index(tmp_path, name, fx):
    assert err(write(tmp_path, name, fx())).variant == "InvalidNumberedFilename"


def test_rejects_inconsistent_total_count_in_sibling_filename(tmp_path):
    entry = write(tmp_path, "name-00001-of-00002.gguf", F().split(0, 2))
    write(tmp_path, "name-00002-of-00003.gguf", F().split(1, 3))
    assert err(entry).variant == "MissingShard"


def test_rejects_duplicate_effective_ordinal_from_metadata(tmp_path):
    entry = write(tmp_path, "name-00001-of-00002.gguf", F().split(0, 2))
    write(tmp_path, "name-00002-of-00002.gguf", F().split(0, 2))
    e = err(entry)
    assert (e.variant, e.fields["key"]) == ("SplitMetadataDisagreement", "split.no")


def test_rejects_filename_and_split_number_disagreement(tmp_path):
    entry = write(tmp_path, "name-00001-of-00002.gguf", F().split(1, 2))
    write(tmp_path, "name-00002-of-00002.gguf", F().split(1, 2))
    e = err(entry)
    assert (e.variant, e.fields["key"]) == ("SplitMetadataDisagreement", "split.no")


def test_rejects_filename_and_split_count_disagreement(tmp_path):
    entry = write(tmp_path, "name-00001-of-00002.gguf", F().split(0, 3))
    write(tmp_path, "name-00002-of-00002.gguf", F().split(1, 2))
    e = err(entry)
    assert (e.variant, e.fields["key"]) == ("SplitMetadataDisagreement", "split.count")


def test_rejects_aggregate_tensor_count_disagreement(tmp_path):
    entry = write(tmp_path, "name-00001-of-00002.gguf", F().split(0, 2).split_count(3).tensor("one", 0))
    write(tmp_path, "name-00002-of-00002.gguf", F().split(1, 2).split_count(3).tensor("two", 0))
    assert err(entry).variant == "AggregateTensorDirectoryDisagreement"


def test_rejects_duplicate_tensor_names_across_shards(tmp_path):
    entry = write(tmp_path, "name-00001-of-00002.gguf", F().split(0, 2).tensor("same", 0))
    write(tmp_path, "name-00002-of-00002.gguf", F().split(1, 2).tensor("same", 0))
    e = err(entry)
    assert e.variant == "DuplicateTensorName" and e.fields["name"] == "same"


@pytest.mark.parametrize("name,offset,payload", [("past-end", 8, 0), ("bad", 4, None)])
def test_rejects_a_nonzero_first_tensor_offset_at_the_parser_boundary(tmp_path, name, offset, payload):
    fx = F().tensor(name, offset)
    if payload is not None:
        fx.payload_bytes(payload)
    e = err(write(tmp_path, "model.gguf", fx))
    inner = e.fields["error"]
    assert e.variant == "Gguf" and inner.variant == "TensorOffsetMismatch"
    assert (inner.fields["name"], inner.fields["actual_offset"], inner.fields["expected_offset"],
            inner.fields["alignment"]) == (name, offset, 0, 32)


def test_rejects_non_file_input(tmp_path):
    assert err(tmp_path).variant == "NotAFile"


def test_ignores_similarly_named_unrelated_siblings(tmp_path):
    entry = write(tmp_path, "name-00001-of-00002.gguf", F().split(0, 2))
    write(tmp_path, "name-00002-of-00002.gguf", F().split(1, 2))
    write(tmp_path, "name-00003-of-00003.gguf", F().split(2, 3))
    assert len(gs.open_set(entry).files) == 2


def test_rejects_missing_required_split_metadata(tmp_path):
    entry = write(tmp_path, "name-00001-of-00002.gguf", F())
    write(tmp_path, "name-00002-of-00002.gguf", F().split(1, 2))
    e = err(entry)
    assert (e.variant, e.fields["key"]) == ("MissingSplitMetadata", "split.no")


def test_rejects_wrongly_typed_required_split_metadata(tmp_path):
    entry = write(tmp_path, "typed-00001-of-00002.gguf",
                  F().metadata("split.no", 4, struct.pack("<I", 0)).metadata("split.count", 2, struct.pack("<H", 2)))
    write(tmp_path, "typed-00002-of-00002.gguf", F().split(1, 2))
    e = err(entry)
    inner = e.fields["error"]
    assert e.variant == "Metadata" and inner.variant == "WrongType"
    assert (inner.fields["key"], inner.fields["expected"], inner.fields["actual"]) == ("split.no", gg.U16, gg.U32)


def test_symlinks_may_not_escape_the_entry_parent(tmp_path):
    inside, outside = tmp_path / "in", tmp_path / "out"
    inside.mkdir()
    outside.mkdir()
    # an ordinary entry symlink
    target = write(outside, "model.gguf", F())
    os.symlink(target, inside / "model.gguf")
    assert err(inside / "model.gguf").variant == "ShardEscapesParent"
    # a numbered entry symlink
    t1 = write(outside, "model-00001-of-00002.gguf", F().split(0, 2))
    write(outside, "model-00002-of-00002.gguf", F().split(1, 2))
    os.symlink(t1, inside / "model-00001-of-00002.gguf")
    assert err(inside / "model-00001-of-00002.gguf").variant == "ShardEscapesParent"
    # an expected sibling symlink
    d = tmp_path / "d"
    d.mkdir()
    entry = write(d, "model-00001-of-00002.gguf", F().split(0, 2))
    o2 = tmp_path / "o2"
    o2.mkdir()
    os.symlink(write(o2, "model-00002-of-00002.gguf", F().split(1, 2)), d / "model-00002-of-00002.gguf")
    assert err(entry).variant == "ShardEscapesParent"


def test_treats_non_five_digit_split_like_names_as_ordinary_files(tmp_path):
    s = gs.open_set(write(tmp_path, "model-1-of-2.gguf", F().tensor("only", 0)))
    assert len(s.files) == 1 and s.files[0].count == 1


def test_rejects_five_digit_totals_that_do_not_fit_split_count_u16(tmp_path):
    e = err(write(tmp_path, "model-00001-of-65536.gguf", F()))
    assert e.variant == "InvalidNumberedFilename" and e.fields["name"] == "model-00001-of-65536.gguf"


def test_rejects_single_file_optional_split_metadata_that_contradicts_ordinal_or_count(tmp_path):
    e = err(write(tmp_path, "ordinal.gguf", F().split(1, 1)))
    assert (e.variant, e.fields["key"]) == ("SplitMetadataDisagreement", "split.no")
    e = err(write(tmp_path, "count.gguf", F().split(0, 2)))
    assert (e.variant, e.fields["key"]) == ("SplitMetadataDisagreement", "split.count")


def test_rejects_negative_or_wrongly_typed_aggregate_tensor_counts(tmp_path):
    assert err(write(tmp_path, "negative.gguf", F().split_count(-1))).variant == "NegativeAggregateTensorCount"
    e = err(write(tmp_path, "wrong-type.gguf", F().metadata("split.tensors.count", 4, struct.pack("<I", 1))))
    inner = e.fields["error"]
    assert e.variant == "Metadata" and (inner.fields["key"], inner.fields["expected"], inner.fields["actual"]) == \
        ("split.tensors.count", gg.I32, gg.U32)


def test_rejects_different_declared_aggregate_counts_between_shards(tmp_path):
    entry = write(tmp_path, "model-00001-of-00002.gguf", F().split(0, 2).split_count(2).tensor("one", 0))
    write(tmp_path, "model-00002-of-00002.gguf", F().split(1, 2).split_count(3).tensor("two", 0))
    assert err(entry).variant == "AggregateTensorCountDisagreement"


@pytest.mark.parametrize("change,message", [
    (lambda f: f.with_version(2), "has version 2, expected common version 3"),
    (lambda f: f.big_endian(), "has endianness Big, expected common endianness Little"),
    (lambda f: f.alignment(64), "has alignment 64, expected common alignment 32"),
])
def test_rejects_shards_with_different_version_endianness_or_alignment(tmp_path, change, message):
    entry = write(tmp_path, "model-00001-of-00002.gguf", F().split(0, 2))
    second = write(tmp_path, "model-00002-of-00002.gguf", change(F()).split(1, 2))
    assert str(err(entry)) == f'GGUF shard "{os.path.realpath(second)}" {message}'


def test_accepts_shards_with_different_metadata_counts(tmp_path):
    entry = write(tmp_path, "model-00001-of-00002.gguf", F().split(0, 2).metadata("extra", 4, struct.pack("<I", 7)))
    write(tmp_path, "model-00002-of-00002.gguf", F().split(1, 2))
    s = gs.open_set(entry)
    assert len(s.files[0].parsed.metadata) == 3 and len(s.files[1].parsed.metadata) == 2


def test_numbered_single_shard_is_rejected(tmp_path):
    """validate_required_split_metadata: a numbered set of one (discovery.rs:80-82)."""
    e = err(write(tmp_path, "one-00001-of-00001.gguf", F().split(0, 1)))
    assert e.variant == "NumberedSingleShard"


def test_tensor_ranges_point_into_their_own_shard(tmp_path):
    """A real two-shard model written by write_gguf: every location's absolute
    range holds that tensor's payload bytes in its shard."""
    import numpy as np
    rng = np.random.default_rng(4)
    a = rng.integers(0, 256, 4 * 144, dtype=np.uint8).tobytes()
    b = rng.integers(0, 256, 2 * 82, dtype=np.uint8).tobytes()
    p1, p2 = tmp_path / "m-00001-of-00002.gguf", tmp_path / "m-00002-of-00002.gguf"
    meta = lambda i: [("split.no", gg.U16, i), ("split.count", gg.U16, 2), ("split.tensors.count", gg.I32, 2)]
    gg.write_gguf(p1, meta(0), [("a", (256, 4), 12, a)])
    gg.write_gguf(p2, meta(1), [("b", (256, 2), 22, b)])
    s = gs.open_set(p2)
    for name, shard, data in (("a", 0, a), ("b", 1, b)):
        loc = s.tensors.get(name)
        assert loc.shard_index == shard
        with open(s.files[shard].path, "rb") as f:
            f.seek(loc.absolute_range.start)
            assert f.read(len(loc.absolute_range)) == data
