"""GPU parity of the HIP path against the CPU oracle (bit-exact).

Every check calls liblightbridge_hip.so through the C ABI.  Integer stages
(Q8_K bytes, per-block integer sums) and the final f32 outputs are compared bit
for bit; the reference's own fixtures are replayed through the GPU as well.
Sizes: the reference fixtures (K=768), the benchmark shapes of the matvec
configs (4096x4096 Q4_K, 1536x4096 IQ2_S, 4096x1536 IQ3_S) and ragged shapes.
"""
import numpy as np
import pytest

from conftest import read_fixture
from lbhip import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
Q4_K, Q5_K, IQ3_S, IQ2_S = 12, 13, 21, 22
TYPES = [Q4_K, Q5_K, IQ2_S, IQ3_S]


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


def test_f16_conversion_matches_ieee_for_all_inputs(be):
    h = np.arange(65536, dtype=np.uint16)
    src = dev(h.view(np.int16))
    out = torch.empty(65536, dtype=torch.float32, device="cuda")
    be.f16_to_f32(src, out)
    got = host(out)
    want = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))


def test_q8_k_fixture_bytes_on_gpu(be, oracle):
    x = np.frombuffer(read_fixture("q8-k-activations.input-f32le.bin"), np.float32)
    want = np.frombuffer(read_fixture("q8-k-activations.output-q8-k.bin"), np.uint8)
    enc = dev(np.full(want.size, 0xA5, np.uint8))
    be.quantize_row_q8_k_into(dev(x), enc)
    assert np.array_equal(host(enc), want)


@pytest.mark.parametrize("scale", [1.0, 1e-3, 1e-30, 3e37, 1e-42, 0.0])
def test_q8_k_quantize_bit_exact_random(be, oracle, scale):
    rng = np.random.default_rng(int(abs(np.log10(scale + 1e-45)) * 7) + 1)
    x = (rng.standard_normal(64 * 256) * scale).astype(np.float32)
    x[256:512] = 0.0                           # zero block
    x[512:768] = np.float32(-0.0)              # negative-zero block
    x[768 + 5] = x[768 + 9] = np.float32(7.0)  # abs ties inside a block
    x[768 + 200] = np.float32(-7.0)
    want = oracle.quantize_q8_k(x)
    enc = dev(np.zeros(want.size, np.uint8))
    be.quantize_row_q8_k_into(dev(x), enc)
    got = host(enc)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"first mismatch at byte {bad[:8]} (block {bad[0] // 292})"


def test_q8_k_nonfinite_is_reported_and_atomic(be):
    for idx in (0, 255, 256, 4095):
        for bits in (0x7F800000, 0xFFC00001):
            x = np.zeros(4096, np.float32)
            x.view(np.uint32)[idx] = bits
            sentinel = ((np.arange(16 * 292) * 37 + 11) & 0xFF).astype(np.uint8)
            enc = dev(sentinel)
            import lbhip
            with pytest.raises(lbhip.QuantError) as e:
                be.quantize_row_q8_k_into(dev(x), enc)
            assert e.value.variant == "NonFiniteActivation" and e.value.index == idx and e.value.bits == bits
            assert np.array_equal(host(enc), sentinel)


def test_q8_k_shape_errors(be):
    import lbhip
    with pytest.raises(lbhip.QuantError, match="LogicalElementsNotDivisible"):
        be.quantize_row_q8_k_into(dev(np.zeros(255, np.float32)), dev(np.zeros(292, np.uint8)))
    with pytest.raises(lbhip.QuantError, match="EncodedLengthMismatch"):
        be.quantize_row_q8_k_into(dev(np.zeros(256, np.float32)), dev(np.zeros(291, np.uint8)))


@pytest.mark.parametrize("ty", TYPES)
def test_matrix_upload_round_trips_the_ggml_bytes(be, ty):
    w = synth.random_matrix(ty, 33, 1536, seed=ty)
    m = be.upload(ty, 33, 1536, w)
    assert np.array_equal(m.read_ggml(), w.reshape(-1))
    m2 = be.upload(ty, 33, 1536, dev(w.reshape(-1)))
    assert np.array_equal(m2.read_ggml(), w.reshape(-1))
    # GGML bytes at an odd device address (the upload repack's byte-load path)
    buf = dev(np.concatenate([np.zeros(1, np.uint8), w.reshape(-1)]))
    m3 = be.upload(ty, 33, 1536, buf[1:])
    assert np.array_equal(m3.read_ggml(), w.reshape(-1))
    x = np.random.default_rng(ty).standard_normal(1536).astype(np.float32)
    y2, y3 = torch.zeros(33, device="cuda"), torch.zeros(33, device="cuda")
    be.gemv_f32(m2, dev(x), y2)
    be.gemv_f32(m3, dev(x), y3)
    assert np.array_equal(host(y2).view(np.uint32), host(y3).view(np.uint32))


@pytest.mark.parametrize("ty,name", [(Q4_K, "q4-k"), (Q5_K, "q5-k"), (IQ2_S, "iq2-s"), (IQ3_S, "iq3-s")])
def test_reference_dot_fixtures_on_gpu(be, ty, name):
    w = np.frombuffer(read_fixture(f"decode-{name}.input.bin"), np.uint8)
    q8 = np.frombuffer(read_fixture("q8-k-activations.output-q8-k.bin"), np.uint8)
    want = np.frombuffer(read_fixture(f"dot-{name}-q8-k.output-f32le.bin"), np.uint32)[0]
    rows = 5
    m = be.upload(ty, rows, 768, np.tile(w, rows))
    y = torch.full((rows,), float("nan"), device="cuda")
    be.gemv_q8_k(m, dev(q8), y)
    assert np.all(host(y).view(np.uint32) == want)


def _check_gemv(be, oracle, ty, rows, k, seed):
    w = synth.random_matrix(ty, rows, k, seed)
    x = synth.random_activations(k, seed + 1)
    q8 = oracle.quantize_q8_k(x)
    want = oracle.gemv_prequantized(oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True),
                                    oracle.make_matrix(ty, rows, k, w), q8)
    m = be.upload(ty, rows, k, w)
    y = torch.full((rows,), float("nan"), device="cuda")
    be.gemv_q8_k(m, dev(q8), y)
    got = host(y)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {got[bad[:3]]} vs {want[bad[:3]]}"
    # integer stage
    per = 9 if ty in (Q4_K, Q5_K) else 1
    nb = k // 256
    sums = torch.zeros(rows * nb * per, dtype=torch.int32, device="cuda")
    be.block_sums(m, dev(q8), sums)
    gs = host(sums).reshape(rows, -1)
    for r in np.random.default_rng(seed).choice(rows, size=min(rows, 24), replace=False):
        assert np.array_equal(gs[r], oracle.block_sums(ty, w[r], q8).reshape(-1)), r


@pytest.mark.parametrize("ty,rows,k", [(Q4_K, 4096, 4096), (IQ2_S, 1536, 4096), (IQ3_S, 4096, 1536),
                                       (Q5_K, 4096, 4096)])
def test_gemv_bit_exact_at_benchmark_shapes(be, oracle, ty, rows, k):
    _check_gemv(be, oracle, ty, rows, k, seed=1000 + ty)


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("rows,k", [(1, 256), (7, 768), (13, 2304), (65, 1024), (3, 16384)])
def test_gemv_bit_exact_ragged_shapes(be, oracle, ty, rows, k):
    _check_gemv(be, oracle, ty, rows, k, seed=rows * 7 + k)


def test_gemv_into_and_accumulate_match_the_reference_modes(be, oracle):
    for ty in TYPES:
        rows, k = 96, 1536
        w = synth.random_matrix(ty, rows, k, 50 + ty)
        x = synth.random_activations(k, 51)
        om = oracle.make_matrix(ty, rows, k, w)
        want = oracle.gemv(oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 4, True), om, x)
        m = be.upload(ty, rows, k, w)
        y = torch.zeros(rows, device="cuda")
        q8 = torch.zeros(k // 256 * 292, dtype=torch.uint8, device="cuda")
        be.gemv_into(m, dev(x), y, q8)
        assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))
        assert np.array_equal(host(q8), oracle.quantize_q8_k(x))
        dest0 = synth.random_activations(rows, 52)
        want_acc = dest0.copy()
        oracle.gemv_accumulate(oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 4, True), om, x, want_acc, 0.37)
        d = dev(dest0)
        be.gemv_accumulate_scaled_into(m, dev(x), d, 0.37, q8)
        assert np.array_equal(host(d).view(np.uint32), want_acc.view(np.uint32))


def test_gemv_errors_leave_outputs_unchanged(be):
    import lbhip
    rows, k = 8, 512
    w = synth.random_matrix(IQ2_S, rows, k, 3)
    m = be.upload(IQ2_S, rows, k, w)
    sentinel = np.array([np.nan] * rows, np.float32)
    sentinel.view(np.uint32)[:] = 0x7FC000A5
    q8 = torch.zeros(k // 256 * 292, dtype=torch.uint8, device="cuda")
    x = np.ones(k, np.float32)
    x[300] = np.inf
    y = dev(sentinel)
    with pytest.raises(lbhip.KernelError) as e:
        be.gemv_into(m, dev(x), y, q8)
    assert e.value.variant == "NonFiniteValue" and e.value.index == 300
    assert np.array_equal(host(y).view(np.uint32), sentinel.view(np.uint32))
    with pytest.raises(lbhip.KernelError, match="DimensionMismatch"):
        be.gemv_into(m, dev(np.ones(256, np.float32)), y, q8)
    with pytest.raises(lbhip.KernelError, match="ScratchTooSmall"):
        be.gemv_into(m, dev(np.ones(k, np.float32)), y, q8[:291])
    dest = np.zeros(rows, np.float32)
    dest[3] = np.nan
    d = dev(dest)
    with pytest.raises(lbhip.KernelError) as e:
        be.gemv_accumulate_scaled_into(m, dev(np.ones(k, np.float32)), d, 0.5, q8)
    assert e.value.variant == "NonFiniteValue" and e.value.index == 3
    with pytest.raises(lbhip.KernelError, match="NonFiniteValue"):
        be.gemv_accumulate_scaled_into(m, dev(np.ones(k, np.float32)), dev(np.zeros(rows, np.float32)),
                                       float("inf"), q8)


@pytest.mark.parametrize("ty,field", [(Q4_K, 0), (Q4_K, 1), (Q5_K, 1), (IQ2_S, 0), (IQ3_S, 0)])
def test_non_finite_weight_scale_is_rejected_at_upload(be, ty, field):
    import lbhip
    rows, k = 6, 1024
    w = synth.random_matrix(ty, rows, k, 9).copy()
    bb = synth.BLOCK_BYTES[ty]
    # row 4, block 2 gets an infinite d / dmin; row 5 block 0 a NaN (later in order).
    w[4, 2 * bb + 2 * field:2 * bb + 2 * field + 2] = np.array([0x7C00], np.uint16).view(np.uint8)
    w[5, 0:2] = np.array([0x7E01], np.uint16).view(np.uint8)
    with pytest.raises(lbhip.QuantError) as e:
        be.upload(ty, rows, k, w)
    assert (e.value.variant, e.value.row, e.value.index, e.value.field, e.value.bits) == \
        ("NonFiniteScale", 4, 2, field, 0x7C00)


def test_upload_shape_errors(be):
    import lbhip
    with pytest.raises(lbhip.QuantError, match="UnsupportedType"):
        be.upload(1, 1, 256, np.zeros(512, np.uint8))      # F16: not a matrix type of the path
    with pytest.raises(lbhip.QuantError, match="EncodedLengthMismatch"):
        be.upload(Q4_K, 2, 256, np.zeros(143, np.uint8))
    with pytest.raises(lbhip.QuantError, match="LogicalElementsNotDivisible"):
        be.upload(Q4_K, 2, 100, np.zeros(144, np.uint8))


@pytest.mark.parametrize("lpu", [1, 2, 4])
@pytest.mark.parametrize("ty,rows,k", [(Q4_K, 300, 4096), (Q5_K, 97, 2048), (IQ2_S, 515, 4096),
                                       (IQ3_S, 1029, 1536), (IQ2_S, 33, 256), (Q5_K, 17, 16384)])
def test_gemv_every_lanes_per_unit_and_persistent_loop(be, oracle, lpu, ty, rows, k):
    """Every launch shape gives the same bits: lanes per unit 1/2/4, one or two
    row steps in flight per wave: the shape's default and every forced depth 1-4
    (one lane per unit at depth 1: 1024-thread workgroups reading the
    activations from LDS), and a workgroup cap of 3 so each wave walks many
    rows of the persistent loop."""
    try:
        for depth, cap in ((0, 0), (0, 3), (1, 0), (1, 3), (2, 3), (3, 3), (4, 0)):
            be.set_tuning(be.TUNE_GEMV_LPU, lpu)
            be.set_tuning(be.TUNE_GEMV_DEPTH, depth)
            be.set_tuning(be.TUNE_GEMV_MAX_BLOCKS, cap)
            _check_gemv(be, oracle, ty, rows, k, seed=rows + lpu + cap + depth)
    finally:
        be.set_tuning(be.TUNE_GEMV_LPU, 0)
        be.set_tuning(be.TUNE_GEMV_DEPTH, 0)
        be.set_tuning(be.TUNE_GEMV_MAX_BLOCKS, 0)


@pytest.mark.parametrize("ty,rows,k", [(Q4_K, 4096, 4096), (IQ2_S, 1536, 4096), (IQ3_S, 4096, 1536),
                                       (Q5_K, 333, 768)])
def test_fused_quantize_gemv_matches_quantize_then_dot(be, oracle, ty, rows, k):
    """lbh_gemv_f32 quantizes inside the matvec kernel: its published Q8_K bytes
    and its outputs equal quantize_row_q8_k_into followed by the row dots."""
    w = synth.random_matrix(ty, rows, k, 77 + ty)
    x = synth.random_activations(k, 78 + ty)
    x[:256] *= 1e-3                       # a block with a different scale
    q8_ref = oracle.quantize_q8_k(x)
    om = oracle.make_matrix(ty, rows, k, w)
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    want = oracle.gemv_prequantized(ex, om, q8_ref)
    m = be.upload(ty, rows, k, w)
    y = torch.full((rows,), float("nan"), device="cuda")
    q8 = torch.zeros(q8_ref.size, dtype=torch.uint8, device="cuda")
    be.gemv_f32(m, dev(x), y, q8)
    assert np.array_equal(host(q8), q8_ref)
    assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))
    # accumulate form: dest += coef * dot, the order of gemv_accumulate_scaled_into
    dest0 = synth.random_activations(rows, 79)
    want_acc = dest0.copy()
    oracle.gemv_accumulate(ex, om, x, want_acc, -0.75)
    d = dev(dest0)
    be.gemv_f32(m, dev(x), d, None, coef=-0.75, accumulate=True)
    assert np.array_equal(host(d).view(np.uint32), want_acc.view(np.uint32))


@pytest.mark.parametrize("ty,rows,k", [(Q4_K, 37, 256), (Q5_K, 129, 768), (Q4_K, 9, 16384), (Q5_K, 700, 4096),
                                       (IQ2_S, 70, 16384), (IQ3_S, 513, 2304), (Q4_K, 8192, 4096),
                                       (Q5_K, 8192, 4096), (IQ2_S, 9000, 4096), (IQ3_S, 4096, 8192),
                                       (IQ2_S, 13312, 4096), (IQ3_S, 4096, 13312)])
def test_fused_quantize_gemv_every_launch_shape(be, oracle, ty, rows, k):
    """The fused kernel quantizes x in every workgroup (K-quant types also into a
    residue-major copy) and picks its workgroup size and lanes per unit from the
    shape (512 threads at >= 2 * 64 * 4 units per CU): every choice, and a
    workgroup cap that makes each wave walk many rows, gives the bits of
    quantize_row_q8_k_into followed by the reference row dots."""
    w = synth.random_matrix(ty, rows, k, 3 * rows + k + ty)
    x = synth.random_activations(k, rows + k)
    x[:256] *= 1e-3                       # a block with a different scale
    q8_ref = oracle.quantize_q8_k(x)
    want = oracle.gemv_prequantized(oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True),
                                    oracle.make_matrix(ty, rows, k, w), q8_ref)
    m = be.upload(ty, rows, k, w)
    xd = dev(x)
    try:
        for lpu, depth in ((0, 0), (1, 0), (2, 0), (4, 0), (1, 1), (1, 2), (2, 3), (4, 4)):
            for cap in (0, 3):
                be.set_tuning(be.TUNE_GEMV_LPU, lpu)
                be.set_tuning(be.TUNE_GEMV_DEPTH, depth)
                be.set_tuning(be.TUNE_GEMV_MAX_BLOCKS, cap)
                y = torch.full((rows,), float("nan"), device="cuda")
                q8 = torch.zeros(q8_ref.size, dtype=torch.uint8, device="cuda")
                be.gemv_f32(m, xd, y, q8)
                assert np.array_equal(host(q8), q8_ref), (lpu, depth, cap)
                got = host(y)
                bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
                assert bad.size == 0, (lpu, depth, cap, bad.size, bad[:5])
    finally:
        be.set_tuning(be.TUNE_GEMV_LPU, 0)
        be.set_tuning(be.TUNE_GEMV_DEPTH, 0)
        be.set_tuning(be.TUNE_GEMV_MAX_BLOCKS, 0)


def test_floor_reference_kernels(be):
    """The roofline floor kernels (no reference counterpart): an empty launch and
    plain reads of a matrix in every launch shape the bench sweeps; bad shapes
    are refused with InvalidParameter."""
    import lbhip
    m = be.upload(IQ2_S, 1536, 4096, synth.random_matrix(IQ2_S, 1536, 4096, 5))
    sink = torch.zeros(4 * 4096, dtype=torch.int32, device="cuda")
    be.empty_kernel()
    for unroll in (1, 2, 4, 8):
        for grid in (1, 7, 492, 4096):
            for slab in (False, True):
                be.read_matrix(m, sink, grid, unroll, slab)
    torch.cuda.synchronize()
    for grid, unroll in ((0, 1), (be.READ_MAX_GRID + 1, 1), (4, 3), (4, 16)):
        with pytest.raises(lbhip.KernelError, match="InvalidParameter"):
            be.read_matrix(m, sink, grid, unroll)
