"""The MoE layer at its production size (BASELINE configs[2]/[3]): 192 routed
experts, IQ2_S gate/up 1536x4096 and IQ3_S down 4096x1536, a Q4_K/Q5_K shared
expert with ffn 4096, an F32 router 4096x192 with softmax top-8.  Every output
is compared bit for bit with the oracle's moe_routed_by_id
(crates/bridge-kernels-reference/src/moe.rs:64-147), which only touches the
experts each token routes to, so the full layer costs seconds: a few
single-token block decodes with the device router and with host routing, and a
64-token batch under Zipf(1.1) expert popularity, checked and asynchronous."""
import numpy as np
import pytest

from lbhip import synth
from moe_helpers import Layer, dev, host

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
Q4_K, Q5_K, IQ3_S, IQ2_S = 12, 13, 21, 22
H, FFN, NE, TOPK = 4096, 1536, 192, 8


@pytest.fixture(scope="module")
def be():
    import lbhip
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    b = lbhip.HipBackend(0)
    yield b
    b.close()


@pytest.fixture(scope="module")
def layer(be, oracle):
    lay = Layer(be, oracle, NE, H, FFN, 4096, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=801)
    lay.moe.reserve_batch(64, TOPK)
    return lay


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def test_full_layer_single_token_block_decode(be, oracle, layer):
    import lbhip
    w = synth.router_weights(NE, H, 802)
    r = lbhip.Router(be, w)
    rng = np.random.default_rng(803)
    for t in range(3):
        x = rng.standard_normal(H).astype(np.float32)
        ids, coefs = oracle.route_softmax_topk(oracle.router_logits_f32(w, x), TOPK)
        want, err = layer.oracle_out(oracle, ids, coefs, x)
        assert err.status == 0
        y = dev(np.full(H, np.nan, np.float32))
        lbhip.moe_block_forward(be, layer.moe, r, dev(x), y, TOPK)
        assert _same(host(y), want), f"token {t}: device router"
        y2 = dev(np.full(H, np.nan, np.float32))
        be.moe_routed_by_id_into(layer.moe, ids, coefs, dev(x), y2)
        assert _same(host(y2), want), f"token {t}: host routing"
    assert r.take_status() == 0
    r.close()


def test_full_layer_batched_decode_zipf(be, oracle, layer):
    logits = synth.zipf_routes(64, NE, TOPK, 1.1, 804)
    ids = np.zeros((64, TOPK), np.uint32)
    coefs = np.zeros((64, TOPK), np.float32)
    for t in range(64):
        ids[t], coefs[t] = oracle.route_softmax_topk(logits[t], TOPK)
    hits = np.bincount(ids.reshape(-1), minlength=NE)
    assert hits.max() >= 16 and (hits > 0).sum() > 90      # hot experts over several chunks, a long tail
    xs = np.random.default_rng(805).standard_normal((64, H)).astype(np.float32)
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    want = np.stack([oracle.moe_routed_by_id(ex, ids[t], coefs[t], layer.orc_experts, layer.orc_shared, xs[t],
                                             preflight=False) for t in range(64)])
    y = dev(np.full((64, H), np.nan, np.float32))
    be.moe_routed_by_id_batch_into(layer.moe, ids, coefs, dev(xs), y)
    got = host(y)
    bad = [t for t in range(64) if not _same(got[t], want[t])]
    assert not bad, f"checked batch: tokens {bad[:8]}"
    ids_d = torch.zeros((64, TOPK), dtype=torch.int32, device="cuda")
    coefs_d = torch.zeros((64, TOPK), dtype=torch.float32, device="cuda")
    be.route_experts_batch(dev(logits), TOPK, ids_d, coefs_d)
    y2 = dev(np.full((64, H), np.nan, np.float32))
    be.moe_forward_batch(layer.moe, ids_d, coefs_d, dev(xs), y2)
    got2 = host(y2)
    bad = [t for t in range(64) if not _same(got2[t], want[t])]
    assert not bad, f"device-routed batch: tokens {bad[:8]}"
