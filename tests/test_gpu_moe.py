"""GPU parity of the MoE expert FFN block (lbh_moe_*) against the CPU oracle.

The oracle restates moe_routed_by_id_into (crates/bridge-kernels-reference/
src/moe.rs:64-147) with the reference's per-expert SwiGLU (activation.rs) and
the host C library's expf.  Outputs are compared bit for bit; error cases
compare the variant, index and bits and the output buffer afterwards
(unchanged, or the reference's partial accumulation).
"""
import numpy as np
import pytest

from lbhip import synth

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


from moe_helpers import Layer, dev, host  # noqa: E402


def _run(be, layer, ids, coefs, x, sentinel=None):
    y = dev(np.full(layer.hidden, np.nan, np.float32) if sentinel is None else sentinel)
    import lbhip
    try:
        be.moe_routed_by_id_into(layer.moe, ids, coefs, dev(x), y)
        e = None
    except lbhip.BackendError as ex:
        e = ex
    return host(y), e


def _same(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module")
def small(be, oracle):
    return Layer(be, oracle, 6, 512, 256, 512, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=11)


@pytest.fixture(scope="module")
def config3(be, oracle):
    # BASELINE configs[2] shapes with 16 experts (the per-token work of top-8 is the same).
    return Layer(be, oracle, 16, 4096, 1536, 4096, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=23)


def test_device_expf_matches_libm(be, oracle):
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 32, size=1 << 24, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32).copy()
    x[:4] = [float.fromhex("0x1.04845ep+5"), float.fromhex("-0x1.f8cbb2p+5"), 88.72283, -103.97208]
    x[4:4 + 200000] = np.linspace(-110, 95, 200000, dtype=np.float32)
    want = oracle.expf_array(x)
    out = torch.empty(x.size, dtype=torch.float32, device="cuda")
    be.expf(dev(x), out)
    got = host(out)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert _same(got[~nan], want[~nan])


@pytest.mark.parametrize("ids", [[0, 2, 5], [4], [0, 1, 2, 3, 4, 5]])
def test_moe_small_bit_exact(be, oracle, small, ids):
    rng = np.random.default_rng(len(ids))
    coefs = rng.random(len(ids)).astype(np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    want, err = small.oracle_out(oracle, ids, coefs, x)
    assert err.status == 0
    got, e = _run(be, small, ids, coefs, x)
    assert e is None and _same(got, want)


def test_moe_config3_shapes_bit_exact_and_repeatable(be, oracle, config3):
    rng = np.random.default_rng(9)
    for call in range(3):   # arrival counters must reset between calls
        logits = rng.standard_normal(16).astype(np.float32)
        ids, coefs = oracle.route_softmax_topk(logits, 8)
        x = rng.standard_normal(4096).astype(np.float32)
        want, err = config3.oracle_out(oracle, ids, coefs, x)
        assert err.status == 0
        got, e = _run(be, config3, ids, coefs, x)
        assert e is None and _same(got, want), f"call {call}"
        # the unchecked asynchronous form computes the same bits
        y = dev(np.zeros(4096, np.float32))
        config3.moe.be.moe_forward(config3.moe, ids, coefs, dev(x), y)
        assert _same(host(y), want)


@pytest.mark.parametrize("top_k", [1, 2, 3])
def test_down_launches_of_fewer_than_four_routed_experts(be, oracle, small, top_k):
    """A down launch whose workgroup would hold fewer than four waves (top-1..3 without
    the shared expert's down in it: the routed launch of the two-stream schedule, or a
    layer without a shared expert) still fills its whole codebook: the device codebook
    loader spreads it over 256 threads.  The layer without a shared expert shares the
    small layer's routed matrices and is checked against the oracle with an all-zero
    shared expert (its down rows are +0.0, which leaves every accumulation unchanged),
    through the host-routed forward and through the device-router block decode."""
    rng = np.random.default_rng(40 + top_k)
    ids = np.sort(rng.choice(6, size=top_k, replace=False)).astype(np.uint32)
    coefs = rng.random(top_k).astype(np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    want, err = small.oracle_out(oracle, ids, coefs, x)
    assert err.status == 0
    small.moe.set_streams(True)
    try:
        y = dev(np.zeros(512, np.float32))
        be.moe_forward(small.moe, ids, coefs, dev(x), y)
        assert _same(host(y), want), "two-stream schedule"
    finally:
        small.moe.set_streams(False)

    zero = [np.zeros_like(m) for m in small.shared_np]
    orc_zero = oracle.make_expert(oracle.make_matrix(Q4_K, 512, 512, zero[0]),
                                  oracle.make_matrix(Q4_K, 512, 512, zero[1]),
                                  oracle.make_matrix(Q5_K, 512, 512, zero[2]))
    want0 = np.full(512, np.nan, np.float32)
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    err = oracle.moe_routed_by_id_status(ex, ids, coefs, small.orc_experts, orc_zero, x, want0)
    assert err.status == 0
    plain = be.moe_create(small._keep[0], None)
    import lbhip
    w = synth.router_weights(6, 512, 50 + top_k)
    r = lbhip.Router(be, w)
    try:
        y = dev(np.zeros(512, np.float32))
        be.moe_forward(plain, ids, coefs, dev(x), y)
        assert _same(host(y), want0), "no shared expert"
        # the block decode (router chains, selection, routed launches) on the same layer
        rids, rcoefs = oracle.route_softmax_topk(oracle.router_logits_f32(w, x), top_k)
        want_b = np.full(512, np.nan, np.float32)
        err = oracle.moe_routed_by_id_status(ex, rids, rcoefs, small.orc_experts, orc_zero, x, want_b)
        assert err.status == 0
        y = dev(np.zeros(512, np.float32))
        lbhip.moe_block_forward(be, plain, r, dev(x), y, top_k)
        assert _same(host(y), want_b), "block decode, no shared expert"
    finally:
        r.close()
        plain.close()


@pytest.mark.parametrize("tiles", [(1, 1, 1), (7, 3, 7), (512, 512, 256), (300, 200, 20)])
def test_moe_launch_shapes_give_the_same_bits(be, oracle, config3, tiles):
    rng = np.random.default_rng(sum(tiles))
    ids = np.sort(rng.choice(16, size=8, replace=False)).astype(np.uint32)
    coefs = rng.random(8).astype(np.float32)
    x = rng.standard_normal(4096).astype(np.float32)
    want, _ = config3.oracle_out(oracle, ids, coefs, x)
    config3.moe.set_tiles(*tiles)
    try:
        got, e = _run(be, config3, ids, coefs, x)
    finally:
        config3.moe.set_tiles(320, 192, 16)
    assert e is None and _same(got, want)


def test_moe_real_hy3_types(be, oracle):
    """Hy3's own shared expert is IQ2_S/IQ3_S with ffn 1536 (profile.rs, schema.rs)."""
    layer = Layer(be, oracle, 4, 1024, 512, 512, (IQ2_S, IQ3_S, IQ2_S, IQ3_S), seed=31)
    ids, coefs = np.array([1, 3], np.uint32), np.array([0.7, 0.3], np.float32)
    x = np.random.default_rng(1).standard_normal(1024).astype(np.float32)
    want, _ = layer.oracle_out(oracle, ids, coefs, x)
    got, e = _run(be, layer, ids, coefs, x)
    assert e is None and _same(got, want)
    layer2 = Layer(be, oracle, 3, 512, 256, 256, (IQ2_S, IQ2_S, IQ2_S, IQ2_S), seed=32)
    want, _ = layer2.oracle_out(oracle, [0, 2], [0.5, 0.25], x[:512])
    got, e = _run(be, layer2, [0, 2], np.array([0.5, 0.25], np.float32), x[:512])
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
def test_moe_routing_errors_match_and_leave_output_unchanged(be, oracle, small, case):
    ids, coefs = ERROR_CASES[case]
    ids, coefs = np.array(ids, np.uint32), np.array(coefs, np.float32)
    x = np.random.default_rng(2).standard_normal(512).astype(np.float32)
    sentinel = np.arange(512, dtype=np.float32) * np.float32(0.25) - 7
    want, err = small.oracle_out(oracle, ids, coefs, x, sentinel)
    got, e = _run(be, small, ids, coefs, x, sentinel)
    assert err.status != 0 and e is not None
    assert e.code == err.status and e.index == err.index and e.bits == err.bits, (e, err.status, err.index)
    assert _same(got, want) and _same(got, sentinel)


def test_moe_nonfinite_input_is_rejected(be, oracle, small):
    x = np.random.default_rng(4).standard_normal(512).astype(np.float32)
    x[77] = np.inf
    sentinel = np.full(512, 3.5, np.float32)
    want, err = small.oracle_out(oracle, [1, 2], np.array([0.5, 0.5], np.float32), x, sentinel)
    got, e = _run(be, small, [1, 2], np.array([0.5, 0.5], np.float32), x, sentinel)
    assert e.variant == "NonFiniteValue" and e.index == err.index == 77 and e.bits == err.bits
    assert _same(got, sentinel)


def test_moe_swiglu_overflow_is_reported_at_the_reference_lane(be, oracle):
    # Expert 2's gate/up rows from 40 on get the largest f16 scale on every
    # block: with |x| ~ 1e15 their SwiGLU product overflows, the other experts'
    # stays finite (~1e29).
    def scale(e, g, u, d):
        if e == 2:
            for m in (g, u):
                blocks = m.reshape(m.shape[0], -1, 82)
                blocks[40:, :, 0:2] = np.array([0x7BFF], np.uint16).view(np.uint8)
    layer = Layer(be, oracle, 4, 512, 256, 256, (IQ2_S, IQ3_S, IQ2_S, IQ3_S), seed=41, scale=scale)
    x = (np.random.default_rng(6).standard_normal(512) * 1e15).astype(np.float32)
    sentinel = np.full(512, -1.25, np.float32)
    outcomes = []
    for ids in ([0, 2, 3], [2], [0, 1]):
        coefs = np.full(len(ids), 0.5, np.float32)
        want, err = layer.oracle_out(oracle, ids, coefs, x, sentinel)
        outcomes.append(err.status)
        got, e = _run(be, layer, ids, coefs, x, sentinel)
        if err.status == 0:
            assert e is None and _same(got, want)
        else:
            assert e is not None and (e.code, e.index, e.bits) == (err.status, err.index, err.bits)
            assert _same(got, want)
    assert outcomes[0] != 0 and outcomes[1] != 0 and outcomes[2] == 0, outcomes


def test_moe_accumulation_overflow_keeps_the_reference_partial_output(be, oracle, small):
    x = np.random.default_rng(8).standard_normal(512).astype(np.float32)
    ids = np.array([0, 3, 5], np.uint32)
    coefs = np.array([3e38, 3e38, 0.5], np.float32)
    sentinel = np.zeros(512, np.float32)
    want, err = small.oracle_out(oracle, ids, coefs, x, sentinel)
    got, e = _run(be, small, ids, coefs, x, sentinel)
    assert err.status != 0, "the case must overflow"
    assert e is not None and (e.code, e.index, e.bits) == (err.status, err.index, err.bits)
    assert _same(got, want)


# ------------------------------------------------------------------ router

def _router(be, n_experts, hidden, seed, bias=False):
    import lbhip
    w = synth.router_weights(n_experts, hidden, seed)
    b = (np.random.default_rng(seed + 1).standard_normal(n_experts) * 0.05).astype(np.float32) if bias else None
    return lbhip.Router(be, w, b), w, b


@pytest.mark.parametrize("n_experts,hidden,top_k", [(192, 4096, 8), (16, 4096, 8), (7, 256, 3), (256, 1536, 16)])
def test_router_logits_and_softmax_route_bit_exact(be, oracle, n_experts, hidden, top_k):
    r, w, _ = _router(be, n_experts, hidden, seed=n_experts)
    rng = np.random.default_rng(hidden)
    for _ in range(3):
        x = rng.standard_normal(hidden).astype(np.float32)
        ids, coefs, logits = r.route_into(dev(x), top_k, want_logits=True)
        want_logits = oracle.router_logits_f32(w, x)
        assert _same(logits, want_logits)
        wid, wco = oracle.route_softmax_topk(want_logits, top_k)
        assert np.array_equal(ids, wid) and _same(coefs, wco)


def test_router_sigmoid_bias_matches_route_experts_into(be, oracle):
    r, w, b = _router(be, 192, 4096, seed=5, bias=True)
    x = np.random.default_rng(4).standard_normal(4096).astype(np.float32)
    ids, coefs = r.route_into(dev(x), 8, mode=1, weight_scale=2.826)
    wid, wco = oracle.route_sigmoid_bias(oracle.router_logits_f32(w, x), b, 8, 2.826)
    assert np.array_equal(ids, wid) and _same(coefs, wco)


def test_router_ties_prefer_the_lower_id(be, oracle):
    import lbhip
    w = synth.router_weights(64, 256, 3)
    w[[9, 20, 41]] = w[5]      # four identical rows: equal logits
    w[[3, 30]] = -w[5]
    b = np.zeros(64, np.float32)
    r = lbhip.Router(be, w, b)
    x = np.abs(np.random.default_rng(2).standard_normal(256)).astype(np.float32)
    x *= np.sign(w[5]) * 0 + 1
    logits = oracle.router_logits_f32(w, x)
    for mode in (0, 1):
        ids, coefs = r.route_into(dev(x), 3, mode=mode, weight_scale=1.0)
        want = oracle.route_softmax_topk(logits, 3) if mode == 0 else oracle.route_sigmoid_bias(logits, b, 3, 1.0)
        assert np.array_equal(ids, want[0]) and _same(coefs, want[1])


def test_router_rejects_non_finite_input_and_bias(be, oracle):
    import lbhip
    r, w, b = _router(be, 32, 512, seed=9, bias=True)
    x = np.ones(512, np.float32)
    x[100] = np.nan
    with pytest.raises(lbhip.KernelError) as e:
        r.route_into(dev(x), 4)
    assert e.value.variant == "NonFiniteValue" and e.value.index == 100
    b2 = b.copy()
    b2[17] = np.inf
    r2 = lbhip.Router(be, w, b2)
    with pytest.raises(lbhip.KernelError) as e:
        r2.route_into(dev(np.ones(512, np.float32)), 4, mode=1)
    with pytest.raises(oracle.OracleError) as oe:
        oracle.route_sigmoid_bias(oracle.router_logits_f32(w, np.ones(512, np.float32)), b2, 4, 1.0)
    assert e.value.index == oe.value.index == 17 and e.value.bits == oe.value.bits


def test_moe_block_forward_router_plus_experts_bit_exact(be, oracle, config3):
    import lbhip
    r, w, _ = _router(be, 16, 4096, seed=77)
    rng = np.random.default_rng(12)
    for _ in range(3):
        x = rng.standard_normal(4096).astype(np.float32)
        ids, coefs = oracle.route_softmax_topk(oracle.router_logits_f32(w, x), 8)
        want, err = config3.oracle_out(oracle, ids, coefs, x)
        y = dev(np.zeros(4096, np.float32))
        lbhip.moe_block_forward(be, config3.moe, r, dev(x), y, 8)
        assert err.status == 0 and _same(host(y), want)
