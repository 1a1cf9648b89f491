"""GPU parity of the batched decode with 16-row tile copies of the routed IQ
matrices (lbh_moe_make_batch_tile_copies): the matrix-core streams read the
copies, every other kernel the caller's matrices, and every token must still be
bit-identical to the CPU oracle's moe_routed_by_id on that token alone
(crates/bridge-kernels-reference/src/moe.rs:64-147), with copies of every
expert, of some experts, after a replacement and after they are dropped.
"""
import ctypes as C

import numpy as np
import pytest

from moe_helpers import Layer, dev, host
from test_gpu_batch import _same, oracle_batch, run_checked, zipf_routing

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
    layer = Layer(be, oracle, 12, 512, 256, 512, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=151)
    layer.moe.reserve_batch(64, 8)
    yield layer
    layer.moe.make_batch_tile_copies([])


def copy_bytes(layer, experts):
    """Bytes of the copies: each expert's gate, up and down, 256-byte aligned."""
    return sum((m.nbytes + 255) // 256 * 256 for e in experts for m in layer._keep[0][e])


def batch_case(oracle, layer, n_tokens, n_experts, top_k, seed):
    _, ids, coefs = zipf_routing(oracle, n_tokens, n_experts, top_k, seed=seed)
    xs = np.random.default_rng(seed + 1).standard_normal((n_tokens, layer.hidden)).astype(np.float32)
    return ids, coefs, xs, oracle_batch(oracle, layer, ids, coefs, xs)


@pytest.mark.parametrize("engine", [(1, 0, 0), (4, 0, 0), (3, 64, 64), (3, 32, 64), (1, 64, 16), (16, 16, 32)])
def test_tile_copies_of_every_expert_bit_exact(be, oracle, small, engine):
    """Every chunk size on the matrix cores (1), the split defaults (4), the
    defaults with copies (3, one wave per tile) and other row tiles (waves per
    16-row tile 1, 2, 4)."""
    ids, coefs, xs, want = batch_case(oracle, small, 40, 12, 4, seed=21)
    small.moe.make_batch_tile_copies()
    assert small.moe.batch_tile_copy_bytes == copy_bytes(small, range(12))
    small.moe.set_batch_engine(*engine)
    try:
        got = run_checked(be, small, ids, coefs, xs)
    finally:
        small.moe.set_batch_engine()
    assert all(_same(got[t], want[t]) for t in range(40))


def test_tile_copies_of_some_experts_replaced_and_dropped(be, oracle, small):
    """Chunks of copied and uncopied experts in one call; a second call replaces
    the copies; an empty list drops them; a hot expert spans several chunks."""
    n = 40
    ids = np.tile(np.array([0, 3, 5, 9], np.uint32), (n, 1))
    ids[::3] = [1, 3, 7, 11]
    coefs = np.random.default_rng(31).random((n, 4)).astype(np.float32)
    xs = np.random.default_rng(32).standard_normal((n, 512)).astype(np.float32)
    want = oracle_batch(oracle, small, ids, coefs, xs)
    small.moe.set_batch_engine(1)
    try:
        for experts in ([3, 9, 3], [0, 1, 5, 7, 11], []):
            small.moe.make_batch_tile_copies(experts)
            assert small.moe.batch_tile_copy_bytes == copy_bytes(small, sorted(set(experts)))
            got = run_checked(be, small, ids, coefs, xs)
            assert all(_same(got[t], want[t]) for t in range(n)), f"copies of {experts}"
    finally:
        small.moe.set_batch_engine()
    assert small.moe.batch_tile_copy_bytes == 0


def test_tile_copies_leave_the_single_token_path_alone(be, oracle, small):
    small.moe.make_batch_tile_copies()
    try:
        rng = np.random.default_rng(41)
        for t in range(3):
            ids = np.sort(rng.choice(12, 4, replace=False)).astype(np.uint32)
            coefs = rng.random(4).astype(np.float32)
            x = rng.standard_normal(512).astype(np.float32)
            want, err = small.oracle_out(oracle, ids, coefs, x)
            assert err.status == 0
            y = dev(np.zeros(512, np.float32))
            be.moe_forward(small.moe, ids, coefs, dev(x), y)
            assert _same(host(y), want), f"token {t}"
    finally:
        small.moe.make_batch_tile_copies([])


def test_tile_copies_reject_bad_expert_ids(small):
    import lbhip
    with pytest.raises(lbhip.KernelError) as e:
        small.moe.make_batch_tile_copies([2, 12])
    assert e.value.variant == "InvalidParameter" and e.value.index == 1


@pytest.mark.parametrize("types", [(IQ2_S, IQ3_S, IQ2_S, IQ3_S), (IQ2_S, IQ2_S, IQ2_S, IQ2_S)])
def test_tile_copies_with_an_iq_shared_expert(be, oracle, types):
    """The shared expert's matrix-core streams keep reading its own matrices;
    routed downs of either IQ type read their copies."""
    layer = Layer(be, oracle, 6, 1024, 512, 256, types, seed=161)
    layer.moe.reserve_batch(32, 3)
    ids, coefs, xs, want = batch_case(oracle, layer, 24, 6, 3, seed=51)
    layer.moe.make_batch_tile_copies()
    layer.moe.set_batch_engine(1)
    got = run_checked(be, layer, ids, coefs, xs)
    assert all(_same(got[t], want[t]) for t in range(24))


def test_tile_copies_config3_shapes_zipf_bit_exact(be, oracle):
    """BASELINE configs[3] shapes (hidden 4096, routed IQ2_S/IQ3_S ffn 1536,
    Q4_K/Q5_K shared ffn 4096, 64 tokens of Zipf(1.1) top-8) over 32 experts,
    every expert copied, the default engine, two calls."""
    layer = Layer(be, oracle, 32, 4096, 1536, 4096, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=171)
    layer.moe.reserve_batch(64, 8)
    layer.moe.make_batch_tile_copies()
    ids, coefs, xs, want = batch_case(oracle, layer, 64, 32, 8, seed=61)
    for rep in range(2):
        got = run_checked(be, layer, ids, coefs, xs)
        bad = [t for t in range(64) if not _same(got[t], want[t])]
        assert not bad, f"call {rep}: tokens {bad[:8]}"


def test_tile_copies_refused_on_a_cached_layer(be):
    """A layer over an expert cache has no static expert table to copy."""
    import lbhip
    from lbhip.cache import CachedMoeLayer, ExpertCache
    hidden, ffn = 512, 256
    entry = 2 * ffn * (hidden // 256) * 82 + hidden * (ffn // 256) * 110
    cache = ExpertCache(be, 2 * entry, 1, hidden, ffn, IQ2_S, IQ3_S)
    layer = CachedMoeLayer(be, cache)
    try:
        err = lbhip.LbhError()
        st = lbhip.lib().lbh_moe_make_batch_tile_copies(be.ctx, layer.handle, None, 0, C.byref(err))
        assert st == 25 and err.status == 25   # LBH_INVALID_PARAMETER
    finally:
        layer.close()
        cache.close()


def test_tile_copies_async_device_routed_and_residual(be, oracle, small):
    """The asynchronous batched forward over the copies with device-selected
    routes (lbh_route_experts_batch), and its residual form (hidden += the
    block's output, residual_add_in_place, crates/bridge-kernels-reference/
    src/norm.rs:83-98) against the oracle."""
    logits, ids_w, coefs_w = zipf_routing(oracle, 30, 12, 4, seed=71)
    xs = np.random.default_rng(72).standard_normal((30, 512)).astype(np.float32)
    want = oracle_batch(oracle, small, ids_w, coefs_w, xs)
    hidden0 = (np.random.default_rng(73).standard_normal((30, 512)) * 2).astype(np.float32)
    small.moe.make_batch_tile_copies()
    try:
        ids = torch.zeros((30, 4), dtype=torch.int32, device="cuda")
        coefs = torch.zeros((30, 4), dtype=torch.float32, device="cuda")
        be.route_experts_batch(dev(logits), 4, ids, coefs)
        y = dev(np.zeros((30, 512), np.float32))
        be.moe_forward_batch(small.moe, ids, coefs, dev(xs), y)
        got = host(y)
        assert all(_same(got[t], want[t]) for t in range(30))
        h = dev(hidden0)
        be.moe_forward_batch_residual(small.moe, ids, coefs, dev(xs), h)
        got_h = host(h)
        for t in range(30):
            w = hidden0[t].copy()
            oracle.residual_add_in_place(w, want[t])
            assert _same(got_h[t], w), f"token {t}"
    finally:
        small.moe.make_batch_tile_copies([])
