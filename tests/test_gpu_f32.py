"""F32 matrices through the matvec entry points.  The reference routes an F32
PackedMatrix to dot_f32_row in every execution mode (gemv_into,
crates/bridge-kernels-reference/src/gemv.rs:88-101; the accumulating form,
:128-146): one sequential f32 chain per row, sum += weight * input, each product
and sum rounded, after prepare_dequant's checks (dimensions, finite input, then
finite weights in row-major order, :213-243).  Every output is compared bit for
bit with the oracle's restatement (oracle/lb_oracle.c dot_f32_row), including a
row whose value depends on the summation order, and every error payload with
the oracle's."""
import numpy as np
import pytest

from moe_helpers import dev, host

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
F32, Q4_K = 0, 12


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


def _case(rows, k, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, k)) * 0.05).astype(np.float32)
    x = rng.standard_normal(k).astype(np.float32)
    return w, x


@pytest.mark.parametrize("rows,k", [(1, 256), (7, 512), (300, 1024), (4096, 4096), (1029, 2304)])
def test_f32_matvec_every_entry_bit_exact(be, oracle, rows, k):
    w, x = _case(rows, k, rows + k)
    om = oracle.make_matrix(F32, rows, k, w)
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    want = oracle.gemv(ex, om, x)
    m = be.upload(F32, rows, k, w)
    assert m.read_ggml().view(np.float32).reshape(rows, k).tobytes() == w.tobytes()
    q8 = torch.zeros(k // 256 * 292, dtype=torch.uint8, device="cuda")
    for run in ("gemv_into", "dequant_into", "async"):
        y = dev(np.full(rows, np.nan, np.float32))
        if run == "gemv_into":
            be.gemv_into(m, dev(x), y, q8)
        elif run == "dequant_into":
            be.gemv_dequant_into(m, dev(x), y)
        else:
            be.gemv_dequant_f32(m, dev(x), y)
        assert _same(host(y), want), run
    dest0 = np.random.default_rng(k).standard_normal(rows).astype(np.float32)
    want_acc = dest0.copy()
    oracle.gemv_accumulate(ex, om, x, want_acc, -0.625)
    for run in ("accumulate", "dequant_accumulate", "async"):
        d = dev(dest0)
        if run == "accumulate":
            be.gemv_accumulate_scaled_into(m, dev(x), d, -0.625, q8)
        elif run == "dequant_accumulate":
            be.gemv_dequant_accumulate_scaled_into(m, dev(x), d, -0.625)
        else:
            be.gemv_dequant_f32(m, dev(x), d, coef=-0.625, accumulate=True)
        assert _same(host(d), want_acc), run
    m.close()


def test_f32_row_is_the_sequential_sum(be, oracle):
    """((2^24 + 1) + 1) - 2^24 is 0 in f32 in this order (any pairwise or
    reassociated sum gives 2): the chain follows the reference's element order."""
    k = 256
    w = np.zeros((3, k), np.float32)
    w[0, :4] = 1.0
    w[1] = 1.0
    w[2, 200:204] = [1.0, 1.0, 1.0, 1.0]
    x = np.zeros(k, np.float32)
    x[:4] = [2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)]
    x[200:204] = [2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)]
    want = oracle.gemv(oracle.make_exec(), oracle.make_matrix(F32, 3, k, w), x)
    assert want[0] == 0.0 and want[1] == 0.0 and want[2] == 0.0
    m = be.upload(F32, 3, k, w)
    y = dev(np.full(3, np.nan, np.float32))
    be.gemv_dequant_into(m, dev(x), y)
    assert _same(host(y), want)
    m.close()


def test_f32_errors_match_the_reference(be, oracle):
    import lbhip
    rows, k = 40, 512
    w, x = _case(rows, k, 7)
    ex = oracle.make_exec()
    m = be.upload(F32, rows, k, w)
    q8 = torch.zeros(k // 256 * 292, dtype=torch.uint8, device="cuda")
    # non-finite input: NonFiniteValue, field 0 (GEMV input), the first bad lane
    xb = x.copy()
    xb[300], xb[301] = np.inf, np.nan
    with pytest.raises(oracle.OracleError) as oe:
        oracle.gemv(ex, oracle.make_matrix(F32, rows, k, w), xb)
    sentinel = np.full(rows, 9.5, np.float32)
    y = dev(sentinel)
    with pytest.raises(lbhip.KernelError) as e:
        be.gemv_into(m, dev(xb), y, q8)
    assert e.value.variant == "NonFiniteValue" and e.value.index == oe.value.index == 300
    assert e.value.bits == oe.value.bits and e.value.field == 0
    assert _same(host(y), sentinel)
    # dimension mismatch
    with pytest.raises(lbhip.KernelError) as e:
        be.gemv_into(m, dev(x[:256]), y, q8)
    assert e.value.variant == "DimensionMismatch"
    m.close()
    # non-finite weights: NonFiniteValue "GEMV weights" (field 1), index 0 of the
    # one-element decoded block, the first in row-major order; row and column beside it
    wb = w.copy()
    wb[17, 400] = -np.inf
    wb[23, 3] = np.nan
    with pytest.raises(oracle.OracleError) as oe:
        oracle.gemv(ex, oracle.make_matrix(F32, rows, k, wb), x)
    mb = be.upload(F32, rows, k, wb)
    for run in ("gemv_into", "accumulate"):
        y = dev(sentinel)
        with pytest.raises(lbhip.KernelError) as e:
            if run == "gemv_into":
                be.gemv_into(mb, dev(x), y, q8)
            else:
                be.gemv_accumulate_scaled_into(mb, dev(x), y, 0.5, q8)
        assert e.value.variant == "NonFiniteValue" and e.value.field == 1, run
        assert e.value.index == oe.value.index == 0 and e.value.bits == oe.value.bits, run
        assert (e.value.row, e.value.actual) == (17, 400), run
        assert _same(host(y), sentinel), run
    mb.close()


def test_f32_matrix_outside_the_f32_paths_is_refused(be):
    import lbhip
    w, _ = _case(64, 256, 3)
    m = be.upload(F32, 64, 256, w)
    y = torch.zeros(64, device="cuda")
    x = torch.zeros(256, device="cuda")
    with pytest.raises(lbhip.KernelError) as e:
        be.gemv_f32(m, x, y)
    assert e.value.variant == "UnsupportedType"
    with pytest.raises(lbhip.BackendError) as e:
        m.prepare_gemm()
    assert e.value.variant == "UnsupportedType"
    with pytest.raises(lbhip.BackendError) as e:
        be.upload(F32, 2, 100, np.zeros(800, np.uint8))      # k not a multiple of the chains' 256
    assert e.value.variant == "UnsupportedShape"
    with pytest.raises(lbhip.BackendError) as e:
        be.upload(F32, 2, 256, np.zeros(2047, np.uint8))
    assert e.value.variant == "EncodedLengthMismatch"
    m.close()
