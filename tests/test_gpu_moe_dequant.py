"""moe_routed_by_id_into in the DequantF32 execution mode
(crates/bridge-kernels-reference/src/moe.rs:64-147 with
ReferenceExecutionMode::DequantF32: every matvec is dot_dequant_row,
gemv.rs:33-41) through lbh_moe_routed_by_id_dequant_f32_into.  Outputs and
error payloads are compared bit for bit with the oracle run in the same mode
(oracle/lb_oracle.c lbo_moe_routed_by_id with LBO_MODE_DEQUANT_F32): random
routes at small and at the configs[2] shapes, the routing errors, a non-finite
input, a SwiGLU overflow and an accumulation overflow (output left as the
reference leaves it)."""
import numpy as np
import pytest

from moe_helpers import Layer, dev, host

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
Q4_K, Q5_K, IQ3_S, IQ2_S = 12, 13, 21, 22


@pytest.fixture(scope="module")
def be():
    import lbhip
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    b = lbhip.HipBackend(0)
    yield b
    b.close()


@pytest.fixture(scope="module")
def small(be, oracle):
    return Layer(be, oracle, 6, 512, 256, 512, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=61)


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def _want(oracle, layer, ids, coefs, x, sentinel):
    out = sentinel.copy()
    ex = oracle.make_exec(oracle.MODE_DEQUANT_F32)
    err = oracle.moe_routed_by_id_status(ex, ids, coefs, layer.orc_experts, layer.orc_shared, x, out)
    return out, err


def _run(be, layer, ids, coefs, x, sentinel):
    import lbhip
    y = dev(sentinel)
    try:
        be.moe_routed_by_id_dequant_f32_into(layer.moe, np.asarray(ids, np.uint32), np.asarray(coefs, np.float32),
                                             dev(x), y)
        e = None
    except lbhip.BackendError as ex:
        e = ex
    return host(y), e


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_dequant_moe_bit_exact(be, oracle, small, seed):
    rng = np.random.default_rng(seed)
    k = [1, 3, 6][seed - 1]
    ids = np.sort(rng.choice(6, k, replace=False)).astype(np.uint32)
    coefs = rng.dirichlet(np.ones(k)).astype(np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    sentinel = np.full(512, np.nan, np.float32)
    want, err = _want(oracle, small, ids, coefs, x, sentinel)
    assert err.status == 0
    got, e = _run(be, small, ids, coefs, x, sentinel)
    assert e is None and _same(got, want)
    # not the Q8_K mode's result (the two modes round differently)
    y8 = dev(sentinel)
    be.moe_routed_by_id_into(small.moe, ids, coefs, dev(x), y8)
    assert not _same(host(y8), want)


def test_dequant_moe_configs2_shapes_bit_exact(be, oracle):
    """configs[2] widths (hidden 4096, routed ffn 1536, Q4_K/Q5_K shared ffn 4096), top-8 of 12 experts."""
    layer = Layer(be, oracle, 12, 4096, 1536, 4096, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=71)
    rng = np.random.default_rng(72)
    ids = np.sort(rng.choice(12, 8, replace=False)).astype(np.uint32)
    coefs = rng.dirichlet(np.ones(8)).astype(np.float32)
    x = rng.standard_normal(4096).astype(np.float32)
    sentinel = np.full(4096, np.nan, np.float32)
    want, err = _want(oracle, layer, ids, coefs, x, sentinel)
    assert err.status == 0
    got, e = _run(be, layer, ids, coefs, x, sentinel)
    assert e is None and _same(got, want)


ERROR_CASES = {
    "empty": ([], []),
    "duplicate": ([1, 1], [0.5, 0.5]),
    "order": ([3, 1], [0.5, 0.5]),
    "bad_id": ([2, 9], [0.5, 0.5]),
    "nan_coef_first": ([0, 1], [np.nan, 0.5]),
    "inf_coef_later": ([0, 1, 4], [0.5, 0.25, np.inf]),
}


@pytest.mark.parametrize("case", sorted(ERROR_CASES))
def test_dequant_moe_routing_errors(be, oracle, small, case):
    ids, coefs = ERROR_CASES[case]
    ids, coefs = np.array(ids, np.uint32), np.array(coefs, np.float32)
    x = np.random.default_rng(5).standard_normal(512).astype(np.float32)
    sentinel = np.arange(512, dtype=np.float32) * np.float32(0.25) - 7
    want, err = _want(oracle, small, ids, coefs, x, sentinel)
    got, e = _run(be, small, ids, coefs, x, sentinel)
    assert err.status != 0 and e is not None
    assert (e.code, e.index, e.bits) == (err.status, err.index, err.bits)
    assert _same(got, want) and _same(got, sentinel)


def test_dequant_moe_nonfinite_input(be, oracle, small):
    x = np.random.default_rng(6).standard_normal(512).astype(np.float32)
    x[301] = -np.inf
    sentinel = np.full(512, 3.5, np.float32)
    ids, coefs = np.array([1, 2], np.uint32), np.array([0.5, 0.5], np.float32)
    want, err = _want(oracle, small, ids, coefs, x, sentinel)
    got, e = _run(be, small, ids, coefs, x, sentinel)
    assert e is not None and e.variant == "NonFiniteValue"
    assert (e.code, e.index, e.bits) == (err.status, err.index, err.bits) and e.index == 301
    assert _same(got, sentinel)


def test_dequant_moe_swiglu_and_accumulation_overflows(be, oracle):
    # Expert 2's gate/up rows from 40 on get the largest f16 scale: with |x|
    # ~ 1e15 their SwiGLU product overflows; huge coefficients overflow the
    # accumulation of the others.
    def scale(e, g, u, d):
        if e == 2:
            for m in (g, u):
                blocks = m.reshape(m.shape[0], -1, 82)
                blocks[40:, :, 0:2] = np.array([0x7BFF], np.uint16).view(np.uint8)
    layer = Layer(be, oracle, 4, 512, 256, 256, (IQ2_S, IQ3_S, IQ2_S, IQ3_S), seed=81, scale=scale)
    x = (np.random.default_rng(7).standard_normal(512) * 1e15).astype(np.float32)
    sentinel = np.full(512, -1.25, np.float32)
    outcomes = []
    for ids, coefs in (([0, 2, 3], [0.5, 0.5, 0.5]), ([2], [0.5]), ([0, 1], [0.5, 0.5]),
                       ([0, 1, 3], [3e38, 3e38, 0.5])):
        ids, coefs = np.array(ids, np.uint32), np.array(coefs, np.float32)
        want, err = _want(oracle, layer, ids, coefs, x, sentinel)
        outcomes.append((err.status, err.field))
        got, e = _run(be, layer, ids, coefs, x, sentinel)
        if err.status == 0:
            assert e is None
        else:
            assert e is not None and (e.code, e.index, e.bits) == (err.status, err.index, err.bits)
        assert _same(got, want)
    # SwiGLU (field 5) twice, a clean call, then a destination overflow (field 3)
    assert [o[0] != 0 for o in outcomes] == [True, True, False, True], outcomes
    assert outcomes[0][1] == outcomes[1][1] == 5 and outcomes[3][1] == 3, outcomes
