"""Allocation discipline of the boundary.  The reference counts heap allocations
around moe_selected_into after its scratch is built and requires none
(crates/bridge-kernels-reference/tests/allocation.rs:1-67); the device
counterpart: once matrices, layers, routers, batch scratch and workspaces exist,
repeated calls of every hot entry point leave the device's free memory
unchanged, and the [async] entry points record into a HIP graph (stream capture
refuses device allocation) whose replays give the eager results bit for bit."""
import numpy as np
import pytest

from lbhip import synth
from moe_helpers import Layer, dev

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
Q4_K, Q5_K, IQ3_S, IQ2_S = 12, 13, 21, 22
H, FR, FS, NE, TOPK, NT = 1024, 512, 1024, 16, 4, 16


@pytest.fixture(scope="module")
def be():
    import lbhip
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    b = lbhip.HipBackend(0)
    s = torch.cuda.Stream()
    b.set_stream(s)
    b.stream = s
    yield b
    b.close()


@pytest.fixture(scope="module")
def setup(be, oracle):
    """Everything the calls need, created before any counting."""
    import lbhip
    st = {}
    with torch.cuda.stream(be.stream):
        st["layer"] = Layer(be, oracle, NE, H, FR, FS, (IQ2_S, IQ3_S, Q4_K, Q5_K), seed=701)
        st["layer"].moe.reserve_batch(NT, TOPK)
        st["router"] = lbhip.Router(be, synth.router_weights(NE, H, 702))
        st["m_iq2"] = be.upload(IQ2_S, 512, H, synth.random_matrix(IQ2_S, 512, H, 703))
        st["m_iq3"] = be.upload(IQ3_S, H, 512, synth.random_matrix(IQ3_S, H, 512, 704))
        st["m_q5"] = be.upload(Q5_K, 256, H, synth.random_matrix(Q5_K, 256, H, 705))
        st["m_q5"].prepare_gemm()
        rng = np.random.default_rng(706)
        st["x"] = dev(rng.standard_normal(H).astype(np.float32))
        st["x512"] = dev(rng.standard_normal(512).astype(np.float32))
        st["xb"] = dev(rng.standard_normal((NT, H)).astype(np.float32))
        st["q8"] = torch.zeros(H // 256 * 292, dtype=torch.uint8, device="cuda")
        st["q8b"] = torch.zeros((NT, H // 256 * 292), dtype=torch.uint8, device="cuda")
        st["y512"] = torch.zeros(512, device="cuda")
        st["yH"] = torch.zeros(H, device="cuda")
        st["yH2"] = torch.zeros(H, device="cuda")
        st["yH3"] = torch.zeros(H, device="cuda")
        st["sums"] = torch.zeros(512 * (H // 256), dtype=torch.int32, device="cuda")
        st["logits"] = dev(synth.zipf_routes(NT, NE, TOPK, 1.1, seed=707))
        st["ids"] = torch.zeros((NT, TOPK), dtype=torch.int32, device="cuda")
        st["coefs"] = torch.zeros((NT, TOPK), device="cuda")
        st["yb"] = torch.zeros((NT, H), device="cuda")
        st["yg"] = torch.zeros((NT, 256), device="cuda")
        st["yg2"] = torch.zeros((NT, 256), device="cuda")
        st["ws"] = torch.zeros(be.gemm_workspace_bytes(NT, H), dtype=torch.uint8, device="cuda")
        st["ids1"] = np.array([1, 4, 9, 13], np.uint32)
        st["coefs1"] = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    be.stream.synchronize()
    return st


def _async_calls(be, s):
    """The [async] hot entry points, each writing (not accumulating) its outputs."""
    import lbhip
    L = s["layer"]
    return [
        lambda: be.quantize_q8_k_rows(s["xb"], s["q8b"], NT, H),
        lambda: be.gemv_f32(s["m_iq2"], s["x"], s["y512"], s["q8"]),
        lambda: be.gemv_q8_k(s["m_iq3"], s["q8b"][0, :2 * 292], s["yH"]),
        lambda: be.block_sums(s["m_iq2"], s["q8"], s["sums"]),
        lambda: be.gemv_dequant_f32(s["m_iq3"], s["x512"], s["yH2"]),
        lambda: be.moe_forward(L.moe, s["ids1"], s["coefs1"], s["x"], s["yH3"]),
        lambda: lbhip.moe_block_forward(be, L.moe, s["router"], s["x"], s["yH3"], TOPK),
        lambda: be.route_experts_batch(s["logits"], TOPK, s["ids"], s["coefs"]),
        lambda: be.moe_forward_batch(L.moe, s["ids"], s["coefs"], s["xb"], s["yb"]),
        lambda: be.gemm_q8_k(s["m_q5"], s["q8b"], NT, s["yg"], s["ws"]),
        lambda: be.gemm_q8_k_noalloc(s["m_q5"], s["q8b"], NT, s["yg2"]),
    ]


def _sync_calls(be, s):
    """The [sync] checked entry points (they validate and wait for their result)."""
    L = s["layer"]
    return [
        lambda: be.gemv_into(s["m_iq2"], s["x"], s["y512"], s["q8"]),
        lambda: be.gemv_accumulate_scaled_into(s["m_iq2"], s["x"], s["y512"], 0.5, s["q8"]),
        lambda: be.gemv_q8_k_into(s["m_iq2"], s["q8"], s["y512"]),
        lambda: be.gemv_dequant_into(s["m_iq3"], s["x512"], s["yH2"]),
        lambda: be.moe_routed_by_id_into(L.moe, s["ids1"], s["coefs1"], s["x"], s["yH3"]),
        lambda: s["router"].route_into(s["x"], TOPK),
        lambda: s["router"].take_status(),
    ]


def test_hot_entry_points_allocate_nothing_after_setup(be, setup):
    calls = _async_calls(be, setup) + _sync_calls(be, setup)
    with torch.cuda.stream(be.stream):
        for f in calls:              # first calls: per-kernel launch state
            f()
        be.stream.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        for _ in range(100):
            for f in calls:
                f()
        be.stream.synchronize()
        free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"device free memory moved by {free0 - free1} bytes over 100 rounds"


def test_async_entry_points_capture_into_a_graph_and_replay_bit_exact(be, setup):
    s = setup
    outs = ["q8b", "y512", "q8", "yH", "sums", "yH2", "yH3", "ids", "coefs", "yb", "yg", "yg2"]
    calls = _async_calls(be, s)
    with torch.cuda.stream(be.stream):
        for f in calls:
            f()
        be.stream.synchronize()
        want = {k: s[k].clone() for k in outs}
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=be.stream):
            for f in calls:
                f()
        for rep in range(3):
            for k in outs:                       # eager work between the replays
                s[k].zero_()
            be.stream.synchronize()
            g.replay()
            be.stream.synchronize()
            for k in outs:
                a, b = s[k].cpu().numpy(), want[k].cpu().numpy()
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"replay {rep}: {k}"
        del g
