"""GPU parity of the decode matvecs at the Hy3 model's own tensor shapes.

The reference's schema (crates/bridge-model-hy3/src/schema.rs:96-201, sizes
from crates/bridge-model-hy3/src/profile.rs:17-44) places the same four
quantized types on the attention projections, the dense layer-0 FFN and the
output head.  Each shape runs through lbh_gemv_f32 (Q8_K quantization fused
into the matvec, built-in launch shape) and must equal the oracle's
gemv_into (quantize, then one vec_dot_q8_k per row) bit for bit, together with
the Q8_K bytes the kernel publishes.
"""
import numpy as np
import pytest

from lbhip import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
Q4_K, Q5_K, IQ3_S, IQ2_S = 12, 13, 21, 22

HIDDEN, HEADS, KV_HEADS, HEAD_DIM, DENSE_FFN, VOCAB = 4096, 64, 8, 128, 13312, 120832

# (name, type, rows = output width, K = input width): schema.rs lines cited per entry.
SHAPES = [
    ("attn_q", IQ2_S, HEADS * HEAD_DIM, HIDDEN),          # schema.rs:148-154
    ("attn_k", IQ2_S, KV_HEADS * HEAD_DIM, HIDDEN),       # schema.rs:120-126
    ("attn_v", Q4_K, KV_HEADS * HEAD_DIM, HIDDEN),        # schema.rs:162-168
    ("attn_output", IQ3_S, HIDDEN, HEADS * HEAD_DIM),     # schema.rs:141-147
    ("dense_gate", IQ2_S, DENSE_FFN, HIDDEN),             # schema.rs:187-193
    ("dense_down", IQ3_S, HIDDEN, DENSE_FFN),             # schema.rs:180-186
    ("output", Q5_K, VOCAB, HIDDEN),                      # schema.rs:111-117
]


@pytest.fixture(scope="module")
def be():
    import lbhip
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    b = lbhip.HipBackend(0)
    yield b
    b.close()


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("name,ty,rows,k", SHAPES, ids=[s[0] for s in SHAPES])
def test_model_shape_matvec_bit_exact(be, oracle, name, ty, rows, k):
    w = synth.random_matrix(ty, rows, k, seed=rows + k + ty)
    x = synth.random_activations(k, seed=rows + 3)
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    want = oracle.gemv(ex, oracle.make_matrix(ty, rows, k, w), x)
    q8_want = oracle.quantize_q8_k(x)
    m = be.upload(ty, rows, k, w)
    try:
        y = torch.full((rows,), float("nan"), device="cuda")
        q8 = torch.zeros(q8_want.size, dtype=torch.uint8, device="cuda")
        be.gemv_f32(m, torch.from_numpy(x).cuda(), y, q8)
        got = _host(y)
        assert np.array_equal(_host(q8), q8_want)
        bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
        assert bad.size == 0, f"{name}: {bad.size} of {rows} rows differ, first {bad[:5]}"
    finally:
        m.close()


@pytest.mark.parametrize("lpu,cap", [(1, 0), (2, 0), (1, 7)])
def test_output_head_every_launch_shape(be, oracle, lpu, cap):
    """The output head at one and two lanes per unit, with the resident grid and
    with 7 workgroups (every wave walks hundreds of row steps)."""
    rows, k = VOCAB, HIDDEN
    w = synth.random_matrix(Q5_K, rows, k, seed=9)
    x = synth.random_activations(k, seed=10)
    want = oracle.gemv(oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True), oracle.make_matrix(Q5_K, rows, k, w), x)
    m = be.upload(Q5_K, rows, k, w)
    try:
        be.set_tuning(be.TUNE_GEMV_LPU, lpu)
        be.set_tuning(be.TUNE_GEMV_MAX_BLOCKS, cap)
        y = torch.full((rows,), float("nan"), device="cuda")
        be.gemv_f32(m, torch.from_numpy(x).cuda(), y)
        got = _host(y)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        be.set_tuning(be.TUNE_GEMV_LPU, 0)
        be.set_tuning(be.TUNE_GEMV_MAX_BLOCKS, 0)
        m.close()
