"""Pin the CPU oracle against the reference's own golden fixtures.

Mirrors crates/bridge-quant-layout/tests/oracle_vectors.rs:63-182 (decode, Q8_K
bytes and scalar dots, all compared bit for bit) and the table pins of
crates/bridge-quant-layout/src/tables.rs:1564-1594.  The fixtures were produced
by llama.cpp b10153's scalar reference functions (quant-vectors.json).
"""
import hashlib
import json
import struct

import numpy as np
import pytest

from conftest import REF_FIXTURES, read_fixture, PKG

MANIFEST = json.loads((REF_FIXTURES / "quant-vectors.json").read_text())


def test_fixture_files_match_their_manifest_hashes():
    for rec in MANIFEST["files"]:
        data = read_fixture(rec["path"])
        assert len(data) == rec["bytes"], rec["path"]
        assert hashlib.sha256(data).hexdigest() == rec["sha256"], rec["path"]


def test_iq_grid_tables_match_the_pinned_sha256():
    text = (PKG / "csrc" / "lbh_iq_grids.inc").read_text()
    def table(name, width):
        body = text.split(f"#define {name}")[1].split("\n\n")[0]
        vals = [int(t.rstrip("ul"), 16) for t in __import__("re").findall(r"0x[0-9a-f]+", body)]
        return vals
    iq2 = table("LBH_IQ2S_GRID_VALUES", 8)
    iq3 = table("LBH_IQ3S_GRID_VALUES", 4)
    assert len(iq2) == 1024 and len(iq3) == 512
    pins = {t["name"]: t["sha256"] for t in MANIFEST["iq_tables"]}
    assert hashlib.sha256(struct.pack("<1024Q", *iq2)).hexdigest() == pins["iq2s_grid"]
    assert hashlib.sha256(struct.pack("<512I", *iq3)).hexdigest() == pins["iq3s_grid"]
    assert hashlib.sha256(bytes([1 << i for i in range(8)])).hexdigest() == pins["kmask_iq2xs"]
    # Byte alphabets the kernels rely on (grid magnitudes are nonzero and < 64).
    assert {(v >> (8 * i)) & 0xFF for v in iq2 for i in range(8)} == {8, 25, 43}
    assert {(v >> (8 * i)) & 0xFF for v in iq3 for i in range(4)} == set(range(1, 16, 2))


@pytest.mark.parametrize("ty,name,bb", [(12, "q4-k", 144), (13, "q5-k", 176), (22, "iq2-s", 82),
                                        (21, "iq3-s", 110), (0, "f32", 4)])
def test_decode_fixtures_are_bit_exact(oracle, ty, name, bb):
    inp = np.frombuffer(read_fixture(f"decode-{name}.input.bin"), np.uint8)
    exp = np.frombuffer(read_fixture(f"decode-{name}.output-f32le.bin"), np.uint32)
    n = exp.size
    row = oracle.decode_row(ty, inp, n)
    assert np.array_equal(row.view(np.uint32), exp)
    be = 1 if ty == 0 else 256
    for b in range(n // be):
        blk = oracle.decode_row(ty, inp[b * bb:(b + 1) * bb], be)
        assert np.array_equal(blk.view(np.uint32), exp[b * be:(b + 1) * be]), b


def test_q8_k_activation_fixture_is_bit_exact(oracle):
    x = np.frombuffer(read_fixture("q8-k-activations.input-f32le.bin"), np.float32)
    want = np.frombuffer(read_fixture("q8-k-activations.output-q8-k.bin"), np.uint8)
    enc = np.full(want.size, 0xA5, np.uint8)
    oracle.quantize_row_q8_k_into(x, enc)
    assert np.array_equal(enc, want)
    # block_sums recorded in the manifest (the bsums field of every block).
    sums = MANIFEST["q8_k_vectors"][0]["block_sums"]
    got = [int(v) for b in range(3) for v in enc[b * 292 + 260:b * 292 + 292].view(np.int16)]
    assert got == sums


@pytest.mark.parametrize("ty,name", [(12, "q4-k"), (13, "q5-k"), (22, "iq2-s"), (21, "iq3-s")])
@pytest.mark.parametrize("avx2", [False, True])
def test_dot_fixtures_are_bit_exact(oracle, ty, name, avx2):
    w = np.frombuffer(read_fixture(f"decode-{name}.input.bin"), np.uint8)
    q8 = np.frombuffer(read_fixture("q8-k-activations.output-q8-k.bin"), np.uint8)
    want = np.frombuffer(read_fixture(f"dot-{name}-q8-k.output-f32le.bin"), np.uint32)[0]
    got = oracle.vec_dot_q8_k(ty, w, q8, 768, avx2=avx2)
    assert got.view(np.uint32)[0] == want


def test_dot_fixture_values_are_the_documented_ones(oracle):
    vals = {n: np.frombuffer(read_fixture(f"dot-{n}-q8-k.output-f32le.bin"), np.float32)[0]
            for n in ("q4-k", "q5-k", "iq2-s", "iq3-s")}
    assert vals == {"q4-k": np.float32(-13459.150390625), "q5-k": np.float32(-11691.0390625),
                    "iq2-s": np.float32(1177.03955078125), "iq3-s": np.float32(3285.7861328125)}
