"""GPU parity of the matrix-core K-quant GEMM (lbh_gemm_q8_k) against the CPU oracle.

Every output y[t, r] must equal the reference's per-row dot
(dot_q4_or_q5_k, crates/bridge-quant-layout/src/q8_k.rs:247-327) of row r with
token t's Q8_K row, bit for bit: random blocks, negative d/dmin, the integer
extremes (scale 63, mins 63, 5-bit quants 31, activations at +-127), ragged row
and token counts (row and token tiles not multiples of a workgroup's), every
schedule (2 x 2 tiles staged through registers or buffer-to-LDS loads; 3 x 4
tiles in three passes), and the BASELINE configs[4] shape
(Q5_K 12288 x 4096, 512 tokens) in full.
"""
import numpy as np
import pytest

from lbhip import synth
from moe_helpers import dev, host

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
Q4_K, Q5_K = 12, 13


@pytest.fixture(scope="module")
def be():
    import lbhip
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    b = lbhip.HipBackend(0)
    yield b
    b.close()


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def q8_rows(oracle, xs):
    return np.stack([oracle.quantize_q8_k(x) for x in xs])


def run_gemm(be, ty, w, rows, k, q8):
    m = be.upload(ty, rows, k, w)
    m.prepare_gemm()
    n = q8.shape[0]
    ws = torch.zeros(be.gemm_workspace_bytes(n, k), dtype=torch.uint8, device="cuda")
    y = dev(np.full((n, rows), np.nan, np.float32))
    be.gemm_q8_k(m, dev(q8), n, y, ws)
    out = host(y)
    m.close()
    return out


def oracle_gemm(oracle, ty, w, rows, k, q8):
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    om = oracle.make_matrix(ty, rows, k, w)
    return np.stack([oracle.gemv_prequantized(ex, om, q8[t]) for t in range(q8.shape[0])])


@pytest.mark.parametrize("ty", [Q4_K, Q5_K])
@pytest.mark.parametrize("rows,k,n", [(16, 256, 1), (40, 1024, 33), (300, 4096, 70), (64, 512, 32),
                                      (200, 1024, 100), (100, 512, 150), (96, 256, 129), (1000, 2048, 300)])
def test_gemm_random_bit_exact(be, oracle, ty, rows, k, n):
    w = synth.random_matrix(ty, rows, k, seed=rows + k + ty)
    # negative scales on some blocks: flip the f16 sign bits of d and dmin
    blocks = w.reshape(rows, -1, synth.BLOCK_BYTES[ty])
    blocks[::3, ::2, 1] |= 0x80
    blocks[1::4, 1::2, 3] |= 0x80
    xs = np.random.default_rng(n).standard_normal((n, k)).astype(np.float32)
    q8 = q8_rows(oracle, xs)
    assert _same(run_gemm(be, ty, w, rows, k, q8), oracle_gemm(oracle, ty, w, rows, k, q8))


@pytest.mark.parametrize("ty", [Q4_K, Q5_K])
@pytest.mark.parametrize("shape", [0, 3])
def test_gemm_integer_extremes(be, oracle, ty, shape):
    rows, k, n = 48, 512, 40
    bb = synth.BLOCK_BYTES[ty]
    w = np.full((rows, (k // 256) * bb), 0xFF, np.uint8)
    blocks = w.reshape(rows, -1, bb)
    blocks[:, :, 0:2] = np.array([0x3C00], np.uint16).view(np.uint8)   # d = 1.0
    blocks[:, :, 2:4] = np.array([0x3800], np.uint16).view(np.uint8)   # dmin = 0.5
    blocks[:, :, 4:16] = synth.pack_scale_min(np.full((rows * (k // 256), 8), 63),
                                              np.full((rows * (k // 256), 8), 63)).reshape(rows, -1, 12)
    xs = np.where(np.arange(n)[:, None] % 2 == 0, 1.0, -1.0) * np.ones((n, k))
    xs[5] = np.linspace(-1, 1, k)
    xs[6, ::7] = -3.0
    q8 = q8_rows(oracle, xs.astype(np.float32))
    assert np.abs(q8[0, 4:260].view(np.int8)).max() == 127
    be.set_tuning(be.TUNE_GEMM_SHAPE, shape)
    try:
        got = run_gemm(be, ty, w, rows, k, q8)
    finally:
        be.set_tuning(be.TUNE_GEMM_SHAPE, 0)
    assert _same(got, oracle_gemm(oracle, ty, w, rows, k, q8))


@pytest.mark.parametrize("shape", [0, 1, 2, 3])
def test_gemm_staging_modes_give_the_same_bits(be, oracle, shape):
    rows, k, n = 200, 1024, 100
    w = synth.random_matrix(Q5_K, rows, k, seed=9)
    q8 = q8_rows(oracle, np.random.default_rng(10).standard_normal((n, k)).astype(np.float32))
    want = oracle_gemm(oracle, Q5_K, w, rows, k, q8)
    be.set_tuning(be.TUNE_GEMM_SHAPE, shape)
    try:
        got = run_gemm(be, Q5_K, w, rows, k, q8)
    finally:
        be.set_tuning(be.TUNE_GEMM_SHAPE, 0)
    assert _same(got, want)


def test_gemm_requires_preparation_and_workspace(be, oracle):
    import lbhip
    w = synth.random_matrix(Q4_K, 32, 256, seed=1)
    m = be.upload(Q4_K, 32, 256, w)
    q8 = dev(np.zeros((2, 292), np.uint8))
    y = torch.zeros((2, 32), dtype=torch.float32, device="cuda")
    ws = torch.zeros(be.gemm_workspace_bytes(2, 256), dtype=torch.uint8, device="cuda")
    with pytest.raises(lbhip.KernelError):
        be.gemm_q8_k(m, q8, 2, y, ws)           # not prepared
    assert m.device_bytes == m.nbytes == 32 * 144
    m.prepare_gemm()
    # one tile of 32 rows x one block: 17 operands of 1 KiB plus the 32 rows' four scale rows
    assert m.device_bytes == m.nbytes + 17 * 1024 + 32 * 16
    with pytest.raises(lbhip.KernelError):
        be.gemm_q8_k(m, q8, 2, y, ws[:16])      # workspace too small
    iq = be.upload(22, 32, 256, synth.random_matrix(22, 32, 256, seed=2))
    with pytest.raises(lbhip.QuantError) as e:
        iq.prepare_gemm()                       # K-quants only
    assert e.value.variant == "UnsupportedType"


def test_gemm_config5_full_shape_bit_exact(be, oracle):
    """Q8_K activations [512 x 4096] x Q5_K [12288 x 4096]."""
    rows, k, n = 12288, 4096, 512
    w = synth.random_matrix(Q5_K, rows, k, seed=41)
    q8 = q8_rows(oracle, np.random.default_rng(42).standard_normal((n, k)).astype(np.float32))
    got = run_gemm(be, Q5_K, w, rows, k, q8)
    want = oracle_gemm(oracle, Q5_K, w, rows, k, q8)
    bad = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{len(bad)} mismatches, first {bad[:4].tolist()}"
