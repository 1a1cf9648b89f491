"""GPU tests of GGUF payload ingestion straight to HBM (lbh_matrix_create_streamed
through lbhip.gguf.ingest): tensors located by the GGUF directory reader
(mirror of crates/bridge-gguf/src/reader.rs) are streamed in 32 MiB pinned
chunks and repacked on the device.  The matrix read back from HBM must be the
file's payload byte for byte, its matvec must equal the oracle's gemv_into, a
non-finite scale in a later chunk must be reported like lbh_matrix_create
reports it (block, field, bits, row) with nothing created, and a failing reader
must surface as SourceReadFailed."""
import ctypes as C
import os

import numpy as np
import pytest

from lbhip import gguf as gg
from lbhip import synth

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def be():
    import lbhip
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    b = lbhip.HipBackend(0)
    yield b
    b.close()


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    """A GGUF with a 46 MB Q5_K output head (two chunks), an IQ2_S gate, an
    IQ3_S down, an F32 norm and metadata, 4096-byte aligned like a real model."""
    d = tmp_path_factory.mktemp("gguf")
    mats = {"output.weight": (synth.Q5_K, 16384, 4096), "blk.1.ffn_gate.weight": (synth.IQ2_S, 1536, 4096),
            "blk.1.ffn_down.weight": (synth.IQ3_S, 4096, 1536), "blk.1.attn_v.weight": (synth.Q4_K, 1024, 4096)}
    arrs = {n: synth.random_matrix(t, r, k, seed=len(n)) for n, (t, r, k) in mats.items()}
    norm = np.random.default_rng(0).standard_normal(4096).astype(np.float32)
    tensors = [("output_norm.weight", (4096,), 0, norm.tobytes())]
    tensors += [(n, (k, r), t, arrs[n].tobytes()) for n, (t, r, k) in mats.items()]
    path = d / "model.gguf"
    gg.write_gguf(path, [("general.architecture", gg.STRING, "hy3")], tensors, alignment=4096)
    return path, mats, arrs


def test_ingest_round_trips_and_matvecs_match_the_oracle(be, oracle, model):
    path, mats, arrs = model
    got = gg.ingest(be, path)
    assert set(got) == set(mats)   # the F32 norm is not a dot-typed matrix
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    for name, (ty, rows, k) in mats.items():
        m = got[name]
        assert np.array_equal(m.read_ggml(), arrs[name].reshape(-1)), name
        x = synth.random_activations(k, seed=rows)
        want = oracle.gemv(ex, oracle.make_matrix(ty, rows, k, arrs[name]), x)
        y = torch.full((rows,), float("nan"), device="cuda")
        be.gemv_f32(m, torch.from_numpy(x).cuda(), y)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)), name
        m.close()


def test_non_finite_scale_in_a_later_chunk(be, model, tmp_path):
    import lbhip
    path, mats, arrs = model
    ty, rows, k = mats["output.weight"]
    w = arrs["output.weight"].copy()
    nb = k // 256
    row, blk = 15000, 3                     # unit 60003: in the second 32 MiB chunk
    unit = row * nb + blk
    assert unit * 176 > (32 << 20)
    w.reshape(-1)[unit * 176:unit * 176 + 2] = np.array([0xFC00], np.uint16).view(np.uint8)   # -inf d
    p = tmp_path / "bad.gguf"
    gg.write_gguf(p, [], [("output.weight", (k, rows), ty, w.tobytes())], alignment=4096)
    with pytest.raises(lbhip.QuantError) as e:
        gg.ingest(be, p)
    err = e.value
    assert err.variant == "NonFiniteScale" and err.row == row and err.index == blk and err.field == 0
    assert err.bits == 0xFC00


def test_failing_reader_is_reported(be):
    import lbhip

    @gg._READER
    def broken(user, off, dst, n):
        return 7 if off > 0 else 0

    with pytest.raises(lbhip.KernelError) as e:
        lbhip.DeviceMatrix.streamed(be, synth.Q5_K, 16384, 4096, broken)
    assert e.value.variant == "SourceReadFailed" and e.value.actual == 7 and e.value.index == (32 << 20) // 176 * 176


def test_split_set_ingests_from_both_shards(be, oracle, tmp_path):
    """A two-shard set (crates/bridge-gguf-split: open_set over any member): the
    tensors of each shard stream into HBM from their own file, read back byte for
    byte, and their matvecs equal the oracle's gemv_into."""
    from lbhip import gguf_split as gs
    mats = {"blk.0.ffn_gate.weight": (synth.IQ2_S, 1536, 4096, 0), "blk.0.ffn_down.weight": (synth.IQ3_S, 4096, 1536, 0),
            "blk.0.attn_v.weight": (synth.Q4_K, 1024, 4096, 1), "output.weight": (synth.Q5_K, 8192, 4096, 1)}
    arrs = {n: synth.random_matrix(t, r, k, seed=len(n) + 7) for n, (t, r, k, _) in mats.items()}
    for shard in (0, 1):
        meta = [("split.no", gg.U16, shard), ("split.count", gg.U16, 2), ("split.tensors.count", gg.I32, len(mats))]
        tensors = [(n, (k, r), t, arrs[n].tobytes()) for n, (t, r, k, s) in mats.items() if s == shard]
        gg.write_gguf(tmp_path / f"model-{shard + 1:05d}-of-00002.gguf", meta, tensors, alignment=4096)
    gset = gs.open_set(tmp_path / "model-00002-of-00002.gguf")
    assert [gset.tensors.get(n).shard_index for n in mats] == [s for (_, _, _, s) in mats.values()]
    got = gs.ingest_set(be, gset)
    assert set(got) == set(mats)
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    for name, (ty, rows, k, _) in mats.items():
        m = got[name]
        assert np.array_equal(m.read_ggml(), arrs[name].reshape(-1)), name
        x = synth.random_activations(k, seed=rows + 1)
        want = oracle.gemv(ex, oracle.make_matrix(ty, rows, k, arrs[name]), x)
        y = torch.full((rows,), float("nan"), device="cuda")
        be.gemv_f32(m, torch.from_numpy(x).cuda(), y)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)), name
        m.close()
