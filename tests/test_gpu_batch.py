"""GPU parity of the batched MoE decode (lbh_moe_*_batch, lbh_route_experts_batch).

The reference decodes token by token (moe_routed_by_id_into,
crates/bridge-kernels-reference/src/moe.rs:64-147, called per token by
crates/bridge-runtime/src/hy3_scalar.rs:504-650).  Every token of a batch must
come out bit-identical to the CPU oracle's moe_routed_by_id on that token
alone, whatever the grouping: hot experts split over several chunks, ragged
row tiles, one token, the BASELINE configs[3] shape with Zipf-skewed routing.
"""
import numpy as np
import pytest

from lbhip import synth
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


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def zipf_routing(oracle, n_tokens, n_experts, top_k, seed, s=1.1):
    """Per-token softmax top-k of seeded Zipf-skewed logits (the configs[3] routing)."""
    logits = synth.zipf_routes(n_tokens, n_experts, top_k, s, seed)
    ids = np.zeros((n_tokens, top_k), np.uint32)
    coefs = np.zeros((n_tokens, top_k), np.float32)
    for t in range(n_tokens):
        ids[t], coefs[t] = oracle.route_softmax_topk(logits[t], top_k)
    return logits, ids, coefs


def oracle_batch(oracle, layer, ids, coefs, xs):
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    return np.stack([oracle.moe_routed_by_id(ex, ids[t], coefs[t], layer.orc_experts, layer.orc_shared, xs[t],
                                             preflight=False) for t in range(xs.shape[0])])


def run_checked(be, layer, ids, coefs, xs, sentinel=None):
    y = dev(np.full(xs.shape, np.nan, np.float32) if sentinel is None else sentinel)
    be.moe_routed_by_id_batch_into(layer.moe, ids, coefs, dev(xs), y)
    return host(y)


@pytest.fixture(scope="module")
def small(be, oracle):
    layer = Layer(be, oracle, 12, 512, 256, 512, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=51)
    layer.moe.reserve_batch(64, 8)
    return layer


def test_batch_small_every_token_bit_exact(be, oracle, small):
    _, ids, coefs = zipf_routing(oracle, 37, 12, 4, seed=3)
    xs = np.random.default_rng(4).standard_normal((37, 512)).astype(np.float32)
    want = oracle_batch(oracle, small, ids, coefs, xs)
    got = run_checked(be, small, ids, coefs, xs)
    for t in range(37):
        assert _same(got[t], want[t]), f"token {t}"


def test_batch_equals_single_token_path(be, oracle, small):
    _, ids, coefs = zipf_routing(oracle, 9, 12, 3, seed=5)
    xs = np.random.default_rng(6).standard_normal((9, 512)).astype(np.float32)
    got = run_checked(be, small, ids, coefs, xs)
    for t in range(9):
        y = dev(np.zeros(512, np.float32))
        be.moe_forward(small.moe, ids[t], coefs[t], dev(xs[t]), y)
        assert _same(host(y), got[t])


def test_batch_hot_expert_spans_several_chunks(be, oracle, small):
    # Every token routes to experts 0..3: 40 tokens per expert, five chunks of eight.
    n = 40
    ids = np.tile(np.arange(4, dtype=np.uint32), (n, 1))
    coefs = np.random.default_rng(7).random((n, 4)).astype(np.float32)
    xs = np.random.default_rng(8).standard_normal((n, 512)).astype(np.float32)
    want = oracle_batch(oracle, small, ids, coefs, xs)
    got = run_checked(be, small, ids, coefs, xs)
    assert all(_same(got[t], want[t]) for t in range(n))


def test_batch_single_token_single_expert(be, oracle, small):
    ids, coefs = np.array([[7]], np.uint32), np.array([[0.375]], np.float32)
    xs = np.random.default_rng(9).standard_normal((1, 512)).astype(np.float32)
    want = oracle_batch(oracle, small, ids, coefs, xs)
    assert _same(run_checked(be, small, ids, coefs, xs)[0], want[0])


@pytest.mark.parametrize("tiles", [(1, 7, 5, 9, 3), (3, 64, 256, 20, 512), (16, 128, 128, 320, 128), (5, 2, 1, 1, 2)])
def test_batch_launch_shapes_give_the_same_bits(be, oracle, small, tiles):
    _, ids, coefs = zipf_routing(oracle, 21, 12, 4, seed=sum(tiles))
    xs = np.random.default_rng(10).standard_normal((21, 512)).astype(np.float32)
    want = oracle_batch(oracle, small, ids, coefs, xs)
    small.moe.set_batch_tiles(*tiles)
    try:
        got = run_checked(be, small, ids, coefs, xs)
    finally:
        small.moe.set_batch_tiles()
    assert all(_same(got[t], want[t]) for t in range(21))


@pytest.mark.parametrize("engine", [(0, 0, 0), (1, 0, 0), (6, 0, 0), (3, 32, 64), (1, 64, 16), (16, 16, 32)])
def test_batch_engines_bit_exact(be, oracle, small, engine):
    """The IQ streams on the VALU integer dots (0), all chunks on the f16 matrix
    cores (1), the per-chunk split at several thresholds and row tiles, with hot
    experts past one 16-token chunk and single-token experts."""
    _, ids, coefs = zipf_routing(oracle, 40, 12, 4, seed=15)
    xs = np.random.default_rng(16).standard_normal((40, 512)).astype(np.float32)
    want = oracle_batch(oracle, small, ids, coefs, xs)
    small.moe.set_batch_engine(*engine)
    try:
        got = run_checked(be, small, ids, coefs, xs)
    finally:
        small.moe.set_batch_engine()
    assert all(_same(got[t], want[t]) for t in range(40))


@pytest.mark.parametrize("bad", [(-1, 0, 0), (17, 0, 0), (4, 48, 0), (4, 0, 8), (4, 128, 0)])
def test_batch_engine_rejects_bad_settings(small, bad):
    import lbhip
    with pytest.raises(lbhip.KernelError) as e:
        small.moe.set_batch_engine(*bad)
    assert e.value.variant == "InvalidParameter"
    small.moe.set_batch_engine()


@pytest.mark.parametrize("types", [(IQ2_S, IQ3_S, IQ2_S, IQ3_S), (IQ2_S, IQ2_S, IQ2_S, IQ2_S),
                                   (IQ2_S, IQ2_S, IQ2_S, IQ3_S)])
def test_batch_type_sets(be, oracle, types):
    """Hy3's own shared expert is IQ2_S/IQ3_S (profile.rs, schema.rs)."""
    layer = Layer(be, oracle, 6, 1024, 512, 256, types, seed=61)
    layer.moe.reserve_batch(16, 3)
    _, ids, coefs = zipf_routing(oracle, 11, 6, 3, seed=12)
    xs = np.random.default_rng(13).standard_normal((11, 1024)).astype(np.float32)
    want = oracle_batch(oracle, layer, ids, coefs, xs)
    got = run_checked(be, layer, ids, coefs, xs)
    assert all(_same(got[t], want[t]) for t in range(11))


def test_batch_device_routing_softmax_and_sigmoid(be, oracle, small):
    logits, ids_w, coefs_w = zipf_routing(oracle, 30, 12, 4, seed=14)
    ids = torch.zeros((30, 4), dtype=torch.int32, device="cuda")
    coefs = torch.zeros((30, 4), dtype=torch.float32, device="cuda")
    be.route_experts_batch(dev(logits), 4, ids, coefs)
    assert np.array_equal(host(ids).view(np.uint32), ids_w) and _same(host(coefs), coefs_w)
    bias = (np.random.default_rng(15).standard_normal(12) * 0.05).astype(np.float32)
    be.route_experts_batch(dev(logits), 4, ids, coefs, mode=1, weight_scale=2.826, bias=dev(bias))
    for t in range(30):
        wid, wco = oracle.route_sigmoid_bias(logits[t], bias, 4, 2.826)
        assert np.array_equal(host(ids)[t].view(np.uint32), wid) and _same(host(coefs)[t], wco)
    # the device routing feeds the asynchronous batched forward directly
    be.route_experts_batch(dev(logits), 4, ids, coefs)
    xs = np.random.default_rng(16).standard_normal((30, 512)).astype(np.float32)
    y = dev(np.zeros((30, 512), np.float32))
    be.moe_forward_batch(small.moe, ids, coefs, dev(xs), y)
    want = oracle_batch(oracle, small, ids_w, coefs_w, xs)
    got = host(y)
    assert all(_same(got[t], want[t]) for t in range(30))


ERRORS = {
    "order": (lambda i, c: i.__setitem__((5, slice(None)), [3, 1, 4, 6]), "RoutedExpertOrder", 5),
    "duplicate": (lambda i, c: i.__setitem__((2, slice(None)), [1, 1, 4, 6]), "DuplicateRoutedExpert", 2),
    "bad_id": (lambda i, c: i.__setitem__((7, slice(None)), [1, 2, 4, 12]), "InvalidParameter", 7),
    "nan_coef": (lambda i, c: c.__setitem__((3, 2), np.nan), "NonFiniteValue", 3),
}


@pytest.mark.parametrize("case", sorted(ERRORS))
def test_batch_routing_errors_leave_the_output_unchanged(be, oracle, small, case):
    import lbhip
    ids = np.tile(np.array([0, 2, 5, 9], np.uint32), (10, 1))
    coefs = np.full((10, 4), 0.25, np.float32)
    mutate, variant, token = ERRORS[case]
    mutate(ids, coefs)
    xs = np.random.default_rng(17).standard_normal((10, 512)).astype(np.float32)
    sentinel = np.arange(10 * 512, dtype=np.float32).reshape(10, 512) * np.float32(0.5)
    y = dev(sentinel)
    with pytest.raises(lbhip.KernelError) as e:
        be.moe_routed_by_id_batch_into(small.moe, ids, coefs, dev(xs), y)
    assert e.value.variant == variant and e.value.row == token
    assert _same(host(y), sentinel)


def test_batch_nonfinite_input_is_rejected(be, oracle, small):
    import lbhip
    ids = np.tile(np.array([1, 3], np.uint32), (4, 1))
    coefs = np.full((4, 2), 0.5, np.float32)
    xs = np.random.default_rng(18).standard_normal((4, 512)).astype(np.float32)
    xs[2, 301] = -np.inf
    sentinel = np.full((4, 512), 2.5, np.float32)
    y = dev(sentinel)
    with pytest.raises(lbhip.KernelError) as e:
        be.moe_routed_by_id_batch_into(small.moe, ids, coefs, dev(xs), y)
    assert e.value.variant == "NonFiniteValue" and e.value.index == 301 and e.value.row == 2
    assert e.value.bits == 0xFF800000
    assert _same(host(y), sentinel)


def test_batch_capacity_is_enforced(be, oracle, small):
    import lbhip
    xs = np.zeros((65, 512), np.float32)
    ids = np.tile(np.array([1, 3], np.uint32), (65, 1))
    with pytest.raises(lbhip.KernelError) as e:
        be.moe_routed_by_id_batch_into(small.moe, ids, np.ones((65, 2), np.float32), dev(xs), dev(xs))
    assert e.value.variant == "ScratchTooSmall"


def test_batch_async_invalid_device_ids_leave_the_output_unchanged(be, oracle, small):
    ids = torch.tensor([[0, 3], [2, 12]], dtype=torch.int32, device="cuda")     # 12 >= n_experts
    coefs = torch.full((2, 2), 0.5, dtype=torch.float32, device="cuda")
    sentinel = np.full((2, 512), -3.0, np.float32)
    y = dev(sentinel)
    be.moe_forward_batch(small.moe, ids, coefs, dev(np.ones((2, 512), np.float32)), y)
    assert _same(host(y), sentinel)
    ids = torch.tensor([[0, 3], [5, 5]], dtype=torch.int32, device="cuda")      # a repeated id
    be.moe_forward_batch(small.moe, ids, coefs, dev(np.ones((2, 512), np.float32)), y)
    assert _same(host(y), sentinel)


def test_batch_config4_shapes_zipf_bit_exact(be, oracle):
    """64 tokens, hidden 4096, routed IQ2_S/IQ3_S ffn 1536,
    Q4_K/Q5_K shared ffn 4096, top-8 of Zipf(1.1) logits (over 32 experts here so
    the oracle finishes in seconds; hot experts span several chunks)."""
    layer = Layer(be, oracle, 32, 4096, 1536, 4096, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=71)
    layer.moe.reserve_batch(64, 8)
    _, ids, coefs = zipf_routing(oracle, 64, 32, 8, seed=72)
    xs = np.random.default_rng(73).standard_normal((64, 4096)).astype(np.float32)
    want = oracle_batch(oracle, layer, ids, coefs, xs)
    for rep in range(2):   # the plan and scratch are reused across calls
        got = run_checked(be, layer, ids, coefs, xs)
        bad = [t for t in range(64) if not _same(got[t], want[t])]
        assert not bad, f"call {rep}: tokens {bad[:8]}"
