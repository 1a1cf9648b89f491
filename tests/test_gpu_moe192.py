"""GPU parity of the MoE paths on 192-expert layers, the router's summation
order and bounded waits, and the largest single-token down launch.

* 192 routed experts (the BASELINE configs[2]/[3] expert count) at hidden 4096
  with the configs' shared expert (Q4_K/Q5_K, ffn 4096) and a reduced routed
  ffn of 512 so the layer uploads in seconds: the device-router block decode
  (lbh_moe_block_forward) and the 64-token batched decode over Zipf(1.1)
  routes, where most of the ~120 experts hit get chunks of 1-3 tokens (the
  engine mix the configs[3] bench times), every token bit-exact against the
  oracle's moe_routed_by_id (crates/bridge-kernels-reference/src/moe.rs:64-147).
* The router logit is one sequential f32 chain (dot_f32_row,
  crates/bridge-kernels-reference/src/gemv.rs:286-303): for inputs
  [2^24, 1, 1, -2^24] against unit weights it is 0 exactly (a pairwise sum
  gives 1, the exact sum 2); device and oracle must both give 0.
* A router whose bounded ring waits are forced to give up reports
  DeviceTimeout and the block decode leaves its output unchanged.
* 16 routed experts of ffn 4096 need more than 64 KiB of LDS in the down
  launch; a layer whose largest launch would exceed 160 KiB is refused at
  creation.
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


@pytest.fixture(scope="module")
def layer192(be, oracle):
    layer = Layer(be, oracle, 192, 4096, 512, 4096, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=301)
    layer.moe.reserve_batch(64, 8)
    return layer


def test_block_decode_192_experts_device_router(be, oracle, layer192):
    import lbhip
    w = synth.router_weights(192, 4096, 302)
    r = lbhip.Router(be, w)
    rng = np.random.default_rng(303)
    for t in range(4):
        x = rng.standard_normal(4096).astype(np.float32)
        ids, coefs = oracle.route_softmax_topk(oracle.router_logits_f32(w, x), 8)
        want, err = layer192.oracle_out(oracle, ids, coefs, x)
        assert err.status == 0
        y = dev(np.zeros(4096, np.float32))
        lbhip.moe_block_forward(be, layer192.moe, r, dev(x), y, 8)
        assert _same(host(y), want), f"token {t}"
    r.close()


def test_batched_decode_192_experts_zipf(be, oracle, layer192):
    logits = synth.zipf_routes(64, 192, 8, 1.1, 304)
    ids = np.zeros((64, 8), np.uint32)
    coefs = np.zeros((64, 8), np.float32)
    for t in range(64):
        ids[t], coefs[t] = oracle.route_softmax_topk(logits[t], 8)
    hits = np.bincount(ids.reshape(-1), minlength=192)
    assert (hits > 0).sum() > 90 and ((hits > 0) & (hits < 4)).sum() > 50   # mostly 1-3-token chunks
    xs = np.random.default_rng(305).standard_normal((64, 4096)).astype(np.float32)
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    want = np.stack([oracle.moe_routed_by_id(ex, ids[t], coefs[t], layer192.orc_experts, layer192.orc_shared, xs[t],
                                             preflight=False) for t in range(64)])
    y = dev(np.full((64, 4096), np.nan, np.float32))
    be.moe_routed_by_id_batch_into(layer192.moe, ids, coefs, dev(xs), y)
    got = host(y)
    bad = [t for t in range(64) if not _same(got[t], want[t])]
    assert not bad, f"tokens {bad[:8]}"
    # the device selection feeding the asynchronous batch gives the same bits
    ids_d = torch.zeros((64, 8), dtype=torch.int32, device="cuda")
    coefs_d = torch.zeros((64, 8), dtype=torch.float32, device="cuda")
    be.route_experts_batch(dev(logits), 8, ids_d, coefs_d)
    y2 = dev(np.full((64, 4096), np.nan, np.float32))
    be.moe_forward_batch(layer192.moe, ids_d, coefs_d, dev(xs), y2)
    assert _same(host(y2), want)


def test_router_logit_is_a_sequential_sum(be, oracle):
    import lbhip
    w = np.zeros((4, 256), np.float32)
    w[0] = 1.0
    w[1, :4] = [1.0, 1.0, 1.0, 1.0]
    w[2, 2:6] = 0.5
    x = np.zeros(256, np.float32)
    x[:4] = [2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)]
    logits = oracle.router_logits_f32(w, x)
    assert logits[0] == 0.0 and logits[1] == 0.0          # ((2^24 + 1) + 1) - 2^24 in f32
    assert logits[2] == np.float32(0.5 * 1.0 + 0.5 * -(2.0 ** 24))
    r = lbhip.Router(be, w)
    _, _, got = r.route_into(dev(x), 2, want_logits=True)
    assert _same(got, logits)
    r.close()


def test_router_give_up_is_reported_and_leaves_the_output(be, oracle):
    import lbhip
    layer = Layer(be, oracle, 8, 1024, 256, 512, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=311)
    w = synth.router_weights(8, 1024, 312)
    r = lbhip.Router(be, w)
    x = dev(np.random.default_rng(313).standard_normal(1024).astype(np.float32))
    r.set_spin_limit(-1)                      # every unmet ring wait gives up at once
    with pytest.raises(lbhip.BackendError) as e:
        r.route_into(x, 2)
    assert e.value.variant == "DeviceTimeout"
    assert r.take_status() == 0               # the synchronous route reported its own give-up
    sentinel = np.full(1024, 7.5, np.float32)
    y = dev(sentinel)
    lbhip.moe_block_forward(be, layer.moe, r, x, y, 2)
    assert _same(host(y), sentinel)
    lbhip.moe_block_forward(be, layer.moe, r, x, y, 2)
    with pytest.raises(lbhip.BackendError) as e:   # the async steps' give-up, reported once
        r.take_status()
    assert e.value.variant == "DeviceTimeout"
    assert r.take_status() == 0               # cleared by the read
    r.set_spin_limit(0)                       # default bound: routes again, bit-exact
    ids, coefs = r.route_into(x, 2)
    want_ids, want_coefs = oracle.route_softmax_topk(oracle.router_logits_f32(w, x.cpu().numpy()), 2)
    assert np.array_equal(ids, want_ids) and _same(coefs, want_coefs)
    lbhip.moe_block_forward(be, layer.moe, r, x, y, 2)
    want, _ = layer.oracle_out(oracle, want_ids, want_coefs, x.cpu().numpy())
    assert _same(host(y), want)
    assert r.take_status() == 0               # a clean step records nothing
    r.close()


def test_block_decode_rejection_is_reported_with_the_reference_error(be, oracle):
    """A block step whose selection sees a non-finite bias leaves the output and
    records the rejection: take_status raises route_experts_into's error
    (routing.rs:72-77: NonFiniteValue, expert index and value bits) once, counting
    every rejected step."""
    import lbhip
    layer = Layer(be, oracle, 8, 1024, 256, 512, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=331)
    w = synth.router_weights(8, 1024, 332)
    bias = (np.random.default_rng(333).standard_normal(8) * 0.1).astype(np.float32)
    bias[5] = np.inf
    r = lbhip.Router(be, w, bias)
    xh = np.random.default_rng(334).standard_normal(1024).astype(np.float32)
    sentinel = np.full(1024, -2.25, np.float32)
    y = dev(sentinel)
    for _ in range(3):
        lbhip.moe_block_forward(be, layer.moe, r, dev(xh), y, 2, mode=1)
    assert _same(host(y), sentinel)
    with pytest.raises(lbhip.BackendError) as e:
        r.take_status()
    with pytest.raises(oracle.OracleError) as oe:
        oracle.route_sigmoid_bias(oracle.router_logits_f32(w, xh), bias, 2, 1.0)
    assert e.value.variant == "NonFiniteValue"
    assert e.value.index == oe.value.index == 5 and e.value.bits == oe.value.bits
    assert r.take_status() == 0
    r.close()


def test_down_launch_beyond_64k_lds_and_the_limit(be, oracle):
    import lbhip
    layer = Layer(be, oracle, 16, 512, 4096, 4096, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=321)
    rng = np.random.default_rng(322)
    x = rng.standard_normal(512).astype(np.float32)
    ids = np.arange(16, dtype=np.uint32)
    coefs = (rng.random(16) / 16).astype(np.float32)
    want, err = layer.oracle_out(oracle, ids, coefs, x)
    assert err.status == 0
    y = dev(np.zeros(512, np.float32))
    be.moe_routed_by_id_into(layer.moe, ids, coefs, dev(x), y)
    assert _same(host(y), want)
    # ffn 8192 x 16 routed experts would stage 150 KB of Q8_K: refused at creation
    g = be.upload(IQ2_S, 8192, 512, synth.random_matrix(IQ2_S, 8192, 512, 323))
    d = be.upload(IQ3_S, 512, 8192, synth.random_matrix(IQ3_S, 512, 8192, 324))
    sh = layer._keep[1]
    with pytest.raises(lbhip.BackendError) as e:
        be.moe_create([(g, g, d)] * 2, sh)
    assert e.value.variant == "UnsupportedShape"


def test_block_decode_with_the_residual_add(be, oracle, layer192):
    """hy3_block_forward_token ends with residual_add_in_place(hidden, ffn_delta)
    (crates/bridge-kernels-reference/src/layer.rs:464): the fused form equals the
    oracle's block output added to the hidden state by its residual add."""
    import lbhip
    w = synth.router_weights(192, 4096, 331)
    r = lbhip.Router(be, w)
    rng = np.random.default_rng(332)
    x = rng.standard_normal(4096).astype(np.float32)
    hidden0 = rng.standard_normal(4096).astype(np.float32) * 3
    ids, coefs = oracle.route_softmax_topk(oracle.router_logits_f32(w, x), 8)
    delta, err = layer192.oracle_out(oracle, ids, coefs, x)
    assert err.status == 0
    want = hidden0.copy()
    oracle.residual_add_in_place(want, delta)
    h = dev(hidden0)
    lbhip.moe_block_forward_residual(be, layer192.moe, r, dev(x), h, 8)
    assert _same(host(h), want)
    r.close()


def test_batched_decode_with_the_residual_add(be, oracle, layer192):
    logits = synth.zipf_routes(16, 192, 8, 1.1, 341)
    ids = np.zeros((16, 8), np.uint32)
    coefs = np.zeros((16, 8), np.float32)
    for t in range(16):
        ids[t], coefs[t] = oracle.route_softmax_topk(logits[t], 8)
    rng = np.random.default_rng(342)
    xs = rng.standard_normal((16, 4096)).astype(np.float32)
    hidden0 = rng.standard_normal((16, 4096)).astype(np.float32)
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    want = hidden0.copy()
    for t in range(16):
        delta = oracle.moe_routed_by_id(ex, ids[t], coefs[t], layer192.orc_experts, layer192.orc_shared, xs[t],
                                        preflight=False)
        row = want[t].copy()
        oracle.residual_add_in_place(row, delta)
        want[t] = row
    h = dev(hidden0)
    be.moe_forward_batch_residual(layer192.moe, dev(ids.astype(np.int32)), dev(coefs), dev(xs), h)
    assert _same(host(h), want)


def test_two_stream_schedule_gives_the_same_bits(be, oracle, layer192):
    """The shared expert on the layer's second stream (lbh_moe_set_streams(1)):
    host-routed and device-routed forwards equal the oracle, also under graph capture."""
    import lbhip
    w = synth.router_weights(192, 4096, 351)
    r = lbhip.Router(be, w)
    rng = np.random.default_rng(352)
    xs = rng.standard_normal((3, 4096)).astype(np.float32)
    wants = []
    for t in range(3):
        ids, coefs = oracle.route_softmax_topk(oracle.router_logits_f32(w, xs[t]), 8)
        want, _ = layer192.oracle_out(oracle, ids, coefs, xs[t])
        wants.append((ids, coefs, want))
    layer192.moe.set_streams(True)
    try:
        xd = dev(xs)
        y = torch.zeros((3, 4096), device="cuda")
        for t, (ids, coefs, want) in enumerate(wants):
            be.moe_forward(layer192.moe, ids, coefs, xd[t], y[t])
            assert _same(host(y[t]), want)
        s = torch.cuda.Stream()
        be.set_stream(s)
        y2 = torch.zeros((3, 4096), device="cuda")
        with torch.cuda.stream(s):
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for t in range(3):
                    lbhip.moe_block_forward(be, layer192.moe, r, xd[t], y2[t], 8)
            for rep in range(3):
                y2.zero_()
                g.replay()
                s.synchronize()
                got = y2.cpu().numpy()
                assert all(_same(got[t], wants[t][2]) for t in range(3)), f"replay {rep}"
    finally:
        be.set_stream(torch.cuda.current_stream())
        layer192.moe.set_streams(False)
        r.close()
