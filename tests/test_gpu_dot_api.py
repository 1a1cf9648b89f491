"""The reference's dot API over caller-supplied bytes, and the DequantF32 mode, on the GPU.

* lbh_vec_dot_q8_k_into / lbh_validate_vec_dot_q8_k take raw GGML rows and a
  Q8_K row in device memory: the cases of
  crates/bridge-quant-layout/tests/q8_k.rs:97-153
  (dot_validation_rejects_bad_types_lengths_and_scales) are replayed through
  the C ABI with the same variants and payloads, every output left unchanged;
  the reference dot fixtures and random rows are bit-exact against the oracle.
* lbh_gemv_q8_k_into is the checked matvec over an uploaded matrix and
  caller-supplied Q8_K (NonFiniteQ8Scale before any write).
* lbh_gemv_dequant_* is ReferenceExecutionMode::DequantF32
  (crates/bridge-kernels-reference/src/gemv.rs:305-328): bit-exact against the
  oracle's dot_dequant_row at the configs[0] shape, ragged shapes and an
  order-sensitive row whose sequential sum is hand-computed.
* The checked matvec's mixed-error precedence (destination before dimensions,
  input before scratch size) matches the reference order.
"""
import numpy as np
import pytest

from conftest import read_fixture
from lbhip import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
F32, Q4_K, Q5_K, Q8_K, IQ3_S, IQ2_S = 0, 12, 13, 15, 21, 22
TYPES = [Q4_K, Q5_K, IQ2_S, IQ3_S]
NAMES = {Q4_K: "q4-k", Q5_K: "q5-k", IQ2_S: "iq2-s", IQ3_S: "iq3-s"}
SENTINEL_BITS = 0x7FC0_00A5


@pytest.fixture(scope="module")
def be():
    import lbhip
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    b = lbhip.HipBackend(0)
    yield b
    b.close()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def sentinel(n):
    return np.full(n, SENTINEL_BITS, np.uint32).view(np.float32)


def expect_error(be, fn, variant, **fields):
    import lbhip
    with pytest.raises(lbhip.BackendError) as e:
        fn()
    assert e.value.variant == variant, e.value
    for k, v in fields.items():
        assert getattr(e.value, k) == v, (k, e.value)
    return e.value


# ------------------------------------------------ tests/q8_k.rs:97-153 through the C ABI

def test_dot_validation_replays_the_reference_cases(be):
    q4 = np.zeros(144, np.uint8)
    q8 = np.zeros(292, np.uint8)
    out = dev(sentinel(1))

    def dot(ty, w, q, n):
        return lambda: be.vec_dot_q8_k_into(ty, dev(w), dev(q), n, out)

    # vec_dot_q8_k(F32, &[], &[], 256) -> UnsupportedType { ty: F32 }
    expect_error(be, dot(F32, np.zeros(0, np.uint8), np.zeros(0, np.uint8), 256), "UnsupportedType", ty=F32)
    # (Q4_K, q4, q8, 0) -> ZeroLogicalElements
    expect_error(be, dot(Q4_K, q4, q8, 0), "ZeroLogicalElements")
    # (Q4_K, q4, q8, 1) -> LogicalElementsNotDivisible { Q4_K, 1, 256 }
    expect_error(be, dot(Q4_K, q4, q8, 1), "LogicalElementsNotDivisible", ty=Q4_K, actual=1, expected=256)
    # (Q4_K, &q4[..143], q8, 256) -> EncodedLengthMismatch { Q4_K, 144, 143 }
    expect_error(be, dot(Q4_K, q4[:143], q8, 256), "EncodedLengthMismatch", ty=Q4_K, expected=144, actual=143)
    # (Q4_K, q4, &q8[..291], 256) -> EncodedLengthMismatch { Q8_K, 292, 291 }
    expect_error(be, dot(Q4_K, q4, q8[:291], 256), "EncodedLengthMismatch", ty=Q8_K, expected=292, actual=291)
    # weight d = 0x7c00 -> NonFiniteScale { Q4_K, block 0, "d", 0x7c00 }
    bad_w = q4.copy()
    bad_w[0:2] = np.array([0x7C00], np.uint16).view(np.uint8)
    expect_error(be, dot(Q4_K, bad_w, q8, 256), "NonFiniteScale", ty=Q4_K, index=0, field=0, bits=0x7C00)
    # Q8 d = NaN -> NonFiniteQ8Scale { block 0, bits }
    bad_q8 = q8.copy()
    nan_bits = np.float32(np.nan).view(np.uint32)
    bad_q8[0:4] = np.array([nan_bits], np.uint32).view(np.uint8)
    expect_error(be, dot(Q4_K, q4, bad_q8, 256), "NonFiniteQ8Scale", index=0, bits=int(nan_bits))
    # every failure left the output alone; the validate-only call agrees
    assert host(out).view(np.uint32)[0] == SENTINEL_BITS
    expect_error(be, lambda: be.validate_vec_dot_q8_k(Q4_K, dev(q4), dev(bad_q8), 256), "NonFiniteQ8Scale")
    be.validate_vec_dot_q8_k(Q4_K, dev(q4), dev(q8), 256)
    # and the valid call computes: an all-zero row dots to +0.0
    be.vec_dot_q8_k_into(Q4_K, dev(q4), dev(q8), 256, out)
    assert host(out).view(np.uint32)[0] == 0


def test_q8_scale_checks_every_block_and_inf(be):
    """validate_q8_scales (q8_k.rs:208-222) walks every block: the first of two bad blocks is reported."""
    for ty in TYPES:
        w = synth.random_matrix(ty, 1, 1024, 3 + ty).reshape(-1)
        q8 = synth_q8(1024, 4)
        q8[2 * 292:2 * 292 + 4] = np.array([0x7F800000], np.uint32).view(np.uint8)
        q8[3 * 292:3 * 292 + 4] = np.array([0xFFC00000], np.uint32).view(np.uint8)
        out = dev(sentinel(1))
        expect_error(be, lambda: be.vec_dot_q8_k_into(ty, dev(w), dev(q8), 1024, out), "NonFiniteQ8Scale",
                     index=2, bits=0x7F800000)
        assert host(out).view(np.uint32)[0] == SENTINEL_BITS


def test_row_order_of_weight_and_q8_errors(be):
    """Rows validate in order, each row's weights before the Q8_K scales
    (prepare_llama_q8k, gemv.rs:268-270, over validate_vec_dot_q8_k_inner)."""
    ty, rows, k = IQ2_S, 4, 512
    w = synth.random_matrix(ty, rows, k, 8).copy()
    q8 = synth_q8(k, 9)
    bad_q8 = q8.copy()
    bad_q8[292:296] = np.array([0x7FC00000], np.uint32).view(np.uint8)
    w_late = w.copy()
    w_late[2, 82:84] = np.array([0xFC00], np.uint16).view(np.uint8)        # row 2, block 1
    out = dev(sentinel(rows))
    # row 0 clean, Q8 bad, row 2 bad: the Q8_K error comes first
    expect_error(be, lambda: be.vec_dot_q8_k_into(ty, dev(w_late.reshape(-1)), dev(bad_q8), k, out, rows=rows),
                 "NonFiniteQ8Scale", index=1)
    # with a clean Q8_K row, row 2's scale is reported with its row and block
    expect_error(be, lambda: be.vec_dot_q8_k_into(ty, dev(w_late.reshape(-1)), dev(q8), k, out, rows=rows),
                 "NonFiniteScale", row=2, index=1, bits=0xFC00)
    # a bad scale in row 0 precedes the bad Q8_K row
    w_first = w.copy()
    w_first[0, 0:2] = np.array([0x7C01], np.uint16).view(np.uint8)
    expect_error(be, lambda: be.vec_dot_q8_k_into(ty, dev(w_first.reshape(-1)), dev(bad_q8), k, out, rows=rows),
                 "NonFiniteScale", row=0, index=0, bits=0x7C01)
    expect_error(be, lambda: be.vec_dot_q8_k_into(ty, dev(w.reshape(-1)), dev(q8), k, dev(np.zeros(3, np.float32)),
                                                  rows=rows), "OutputLengthMismatch", expected=rows, actual=3)
    assert np.all(host(out).view(np.uint32) == SENTINEL_BITS)


def synth_q8(k, seed):
    from oracle import lb_oracle as orc
    return orc.quantize_q8_k(synth.random_activations(k, seed))


@pytest.mark.parametrize("ty", TYPES)
def test_reference_dot_fixtures_through_the_raw_row_dot(be, ty):
    w = np.frombuffer(read_fixture(f"decode-{NAMES[ty]}.input.bin"), np.uint8)
    q8 = np.frombuffer(read_fixture("q8-k-activations.output-q8-k.bin"), np.uint8)
    want = np.frombuffer(read_fixture(f"dot-{NAMES[ty]}-q8-k.output-f32le.bin"), np.uint32)[0]
    got = np.float32(be.vec_dot_q8_k(ty, dev(w), dev(q8), 768))
    assert got.view(np.uint32) == want
    typed = {Q4_K: be.vec_dot_q4_k_q8_k, Q5_K: be.vec_dot_q5_k_q8_k, IQ2_S: be.vec_dot_iq2_s_q8_k,
             IQ3_S: be.vec_dot_iq3_s_q8_k}[ty]
    assert np.float32(typed(dev(w), dev(q8), 768)).view(np.uint32) == want


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("rows,k,offset", [(1, 256, 0), (37, 1536, 1), (200, 4096, 3), (9, 16384, 2)])
def test_raw_row_dots_bit_exact_at_any_alignment(be, oracle, ty, rows, k, offset):
    """Rows of raw GGML bytes at odd device addresses (byte offsets 1-3) dot
    bit-identically to the oracle's vec_dot_q8_k per row."""
    w = synth.random_matrix(ty, rows, k, 17 * rows + ty)
    x = synth.random_activations(k, rows + k)
    q8 = oracle.quantize_q8_k(x)
    want = np.array([oracle.vec_dot_q8_k(ty, w[r], q8, k)[0] for r in range(rows)], np.float32)
    wb = torch.zeros(w.size + 8, dtype=torch.uint8, device="cuda")
    wb[offset:offset + w.size] = dev(w.reshape(-1))
    qb = torch.zeros(q8.size + 8, dtype=torch.uint8, device="cuda")
    qb[offset:offset + q8.size] = dev(q8)
    out = dev(sentinel(rows))
    be.vec_dot_q8_k_into(ty, wb[offset:offset + w.size], qb[offset:offset + q8.size], k, out, rows=rows)
    got = host(out)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}"


# ------------------------------------------------ checked matvec over caller-supplied Q8_K

@pytest.mark.parametrize("ty,rows,k", [(IQ2_S, 1536, 4096), (IQ3_S, 4096, 1536), (Q4_K, 777, 2048),
                                       (Q5_K, 65, 768)])
def test_checked_prequantized_matvec(be, oracle, ty, rows, k):
    w = synth.random_matrix(ty, rows, k, 31 + ty)
    q8 = oracle.quantize_q8_k(synth.random_activations(k, 32 + ty))
    m = be.upload(ty, rows, k, w)
    want = torch.full((rows,), float("nan"), device="cuda")
    be.gemv_q8_k(m, dev(q8), want)
    y = dev(sentinel(rows))
    be.gemv_q8_k_into(m, dev(q8), y)
    assert np.array_equal(host(y).view(np.uint32), host(want).view(np.uint32))
    # accumulate form equals the unchecked accumulate
    d0 = synth.random_activations(rows, 33)
    a, b = dev(d0), dev(d0)
    be.gemv_q8_k(m, dev(q8), a, coef=0.625, accumulate=True)
    be.gemv_q8_k_into(m, dev(q8), b, coef=0.625, accumulate=True)
    assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32))
    # a NaN / Inf Q8_K scale is reported and nothing is written
    for blk, bits in ((0, 0x7FC00001), (k // 256 - 1, 0xFF800000)):
        bad = q8.copy()
        bad[blk * 292:blk * 292 + 4] = np.array([bits], np.uint32).view(np.uint8)
        y = dev(sentinel(rows))
        expect_error(be, lambda: be.gemv_q8_k_into(m, dev(bad), y), "NonFiniteQ8Scale", index=blk, bits=bits)
        assert np.all(host(y).view(np.uint32) == SENTINEL_BITS)
    expect_error(be, lambda: be.gemv_q8_k_into(m, dev(q8[:-1]), dev(sentinel(rows))), "EncodedLengthMismatch",
                 ty=Q8_K, expected=q8.size, actual=q8.size - 1)
    expect_error(be, lambda: be.gemv_q8_k_into(m, dev(q8), dev(sentinel(rows + 1))), "DimensionMismatch",
                 index=1, expected=rows, actual=rows + 1)
    # accumulate: a NaN destination precedes the wrong Q8_K length
    dest = np.zeros(rows, np.float32)
    dest[rows // 2] = np.nan
    expect_error(be, lambda: be.gemv_q8_k_into(m, dev(q8[:-1]), dev(dest), coef=1.0, accumulate=True),
                 "NonFiniteValue", index=rows // 2, field=3)


# ------------------------------------------------ checked matvec error precedence

def test_gemv_checked_error_precedence(be, oracle):
    """gemv_accumulate_scaled_into checks the destination before the dimensions
    (gemv.rs:126-127 then :195-211); validate_dimensions checks the input before
    prepare_llama_q8k checks the scratch (gemv.rs:258-264).  Device and oracle agree."""
    rows, k = 16, 512
    w = synth.random_matrix(Q4_K, rows, k, 41)
    m = be.upload(Q4_K, rows, k, w)
    om = oracle.make_matrix(Q4_K, rows, k, w)
    ex = oracle.make_exec(oracle.MODE_LLAMA_Q8K)
    dest = np.zeros(rows, np.float32)
    dest[5] = np.nan
    q8 = torch.zeros(k // 256 * 292, dtype=torch.uint8, device="cuda")
    # NaN destination + wrong input length -> NonFiniteValue(destination)
    e = expect_error(be, lambda: be.gemv_accumulate_scaled_into(m, dev(np.ones(256, np.float32)), dev(dest), 0.5, q8),
                     "NonFiniteValue", index=5, field=3)
    with pytest.raises(oracle.OracleError) as oe:
        oracle.gemv_accumulate(ex, om, np.ones(256, np.float32), dest.copy(), 0.5)
    assert (oe.value.status, oe.value.index) == ("NonFiniteValue", 5)
    # NaN input + short scratch -> NonFiniteValue(input)
    x = np.ones(k, np.float32)
    x[300] = np.inf
    y = dev(sentinel(rows))
    e = expect_error(be, lambda: be.gemv_into(m, dev(x), y, q8[:100]), "NonFiniteValue", index=300, field=0)
    assert np.all(host(y).view(np.uint32) == SENTINEL_BITS)
    import ctypes as C
    err = oracle.LboError()
    yo = np.zeros(rows, np.float32)
    small = np.zeros(100, np.uint8)
    st = oracle.lib().lbo_gemv(C.byref(ex), C.byref(om), x.ctypes.data, x.size, yo.ctypes.data, rows,
                               small.ctypes.data, small.size, C.byref(err))
    assert (oracle.STATUS[st], err.index) == ("NonFiniteValue", 300)
    del e


# ------------------------------------------------ DequantF32

def _dequant_want(oracle, ty, rows, k, w, x):
    return oracle.gemv(oracle.make_exec(oracle.MODE_DEQUANT_F32), oracle.make_matrix(ty, rows, k, w), x)


@pytest.mark.parametrize("ty,rows,k", [(Q4_K, 4096, 4096), (IQ2_S, 1536, 4096), (IQ3_S, 4096, 1536),
                                       (Q5_K, 301, 2048), (IQ2_S, 25, 256), (Q4_K, 49, 16384)])
def test_dequant_f32_bit_exact(be, oracle, ty, rows, k):
    w = synth.random_matrix(ty, rows, k, 61 + ty + rows)
    x = synth.random_activations(k, 62 + k)
    want = _dequant_want(oracle, ty, rows, k, w, x)
    m = be.upload(ty, rows, k, w)
    y = dev(sentinel(rows))
    be.gemv_dequant_into(m, dev(x), y)
    got = host(y)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {got[bad[:3]]} vs {want[bad[:3]]}"
    # accumulate arm (gemv.rs:146-151)
    d0 = synth.random_activations(rows, 63)
    want_acc = d0.copy()
    oracle.gemv_accumulate(oracle.make_exec(oracle.MODE_DEQUANT_F32), oracle.make_matrix(ty, rows, k, w), x,
                           want_acc, -1.25)
    d = dev(d0)
    be.gemv_dequant_accumulate_scaled_into(m, dev(x), d, -1.25)
    assert np.array_equal(host(d).view(np.uint32), want_acc.view(np.uint32))
    d = dev(d0)
    be.gemv_dequant_f32(m, dev(x), d, coef=-1.25, accumulate=True)
    assert np.array_equal(host(d).view(np.uint32), want_acc.view(np.uint32))


@pytest.mark.parametrize("ty", TYPES)
def test_dequant_f32_on_the_reference_decode_fixtures(be, oracle, ty):
    """The decode fixtures' weights (structural, LCG and zero-scale blocks):
    every row equals the oracle, whose decode the fixtures pin bit for bit."""
    w = np.frombuffer(read_fixture(f"decode-{NAMES[ty]}.input.bin"), np.uint8)
    x = np.frombuffer(read_fixture("q8-k-activations.input-f32le.bin"), np.float32)
    want = _dequant_want(oracle, ty, 3, 768, np.tile(w, 3), x)
    m = be.upload(ty, 3, 768, np.tile(w, 3))
    y = dev(sentinel(3))
    be.gemv_dequant_into(m, dev(x), y)
    assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))


def _unit_q4_k_block():
    """A Q4_K block that decodes to 256 ones: d = 1.0, dmin = 0, every sub-block
    scale 1 and min 0, every nibble 1 (d1 * 1 - 0 = 1.0, k_quants.rs:254-263)."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    blk[4:16] = synth.pack_scale_min(np.ones((1, 8), np.int64), np.zeros((1, 8), np.int64))[0]
    blk[16:144] = 0x11
    return blk


def test_dequant_sum_order_is_sequential(be, oracle):
    """x = [2^24, 1, 1, -2^24, 0, ...] against a row of ones: the reference's
    sequential f32 sum (gemv.rs:322-325) is ((2^24 + 1) + 1) - 2^24 = 0 (each +1
    rounds back to 2^24); a pairwise sum would give 1 and the exact sum 2."""
    w = _unit_q4_k_block()
    assert np.all(oracle.decode_row(Q4_K, w, 256) == 1.0)
    x = np.zeros(256, np.float32)
    x[:4] = [2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)]
    want = _dequant_want(oracle, Q4_K, 1, 256, w, x)
    assert want[0] == 0.0
    m = be.upload(Q4_K, 1, 256, w)
    y = dev(sentinel(1))
    be.gemv_dequant_into(m, dev(x), y)
    assert host(y)[0] == 0.0


def test_dequant_errors(be):
    rows, k = 8, 512
    m = be.upload(IQ3_S, rows, k, synth.random_matrix(IQ3_S, rows, k, 71))
    x = np.ones(k, np.float32)
    x[7] = np.nan
    y = dev(sentinel(rows))
    expect_error(be, lambda: be.gemv_dequant_into(m, dev(x), y), "NonFiniteValue", index=7, field=0)
    expect_error(be, lambda: be.gemv_dequant_into(m, dev(np.ones(256, np.float32)), y), "DimensionMismatch", index=0)
    expect_error(be, lambda: be.gemv_dequant_accumulate_scaled_into(m, dev(np.ones(k, np.float32)), y,
                                                                     float("nan")), "NonFiniteValue", field=2)
    assert np.all(host(y).view(np.uint32) == SENTINEL_BITS)
    # A non-finite destination is rejected before anything is written
    # (gemv.rs:126-127): the other rows keep their values.
    d0 = np.arange(rows, dtype=np.float32)
    d0[5] = np.inf
    d = dev(d0)
    expect_error(be, lambda: be.gemv_dequant_accumulate_scaled_into(m, dev(np.ones(k, np.float32)), d, 0.5),
                 "NonFiniteValue", index=5, field=3)
    assert np.array_equal(host(d).view(np.uint32), d0.view(np.uint32))
