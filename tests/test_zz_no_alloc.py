"""lbh_gemm_q8_k_noalloc: the prefill GEMM with its activation tiles in the
library's static per-GPU scratch instead of a caller workspace.  Two calls in
a row (the second with fewer tokens, so it runs over the first call's leftover
tiles) must equal lbh_gemm_q8_k bit for bit, and that must equal the oracle's
per-row dots (vec_dot_q8_k, crates/bridge-quant-layout/src/q8_k.rs:80-89) on
sampled tokens; a batch whose tiles exceed the scratch is refused."""
import numpy as np
import pytest

from lbhip import synth

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
Q4_K, Q5_K = 12, 13


@pytest.fixture(scope="module")
def be():
    import lbhip
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    b = lbhip.HipBackend(0)
    yield b
    b.close()


def _q8(oracle, n_tokens, k, seed):
    xs = np.random.default_rng(seed).standard_normal((n_tokens, k)).astype(np.float32)
    return np.stack([oracle.quantize_q8_k(xs[t]) for t in range(n_tokens)])


@pytest.mark.parametrize("ty,rows,k", [(Q5_K, 1536, 4096), (Q4_K, 700, 2048)])
def test_noalloc_gemm_matches_the_workspace_gemm(be, oracle, ty, rows, k):
    w = synth.random_matrix(ty, rows, k, seed=900 + ty)
    m = be.upload(ty, rows, k, w)
    m.prepare_gemm()
    ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
    om = oracle.make_matrix(ty, rows, k, w)
    for call, n_tokens in enumerate((512, 37)):
        q8 = _q8(oracle, n_tokens, k, seed=910 + call)
        q8d = torch.from_numpy(q8.reshape(-1)).cuda()
        y_ws = torch.full((n_tokens, rows), float("nan"), device="cuda")
        ws = torch.zeros(be.gemm_workspace_bytes(n_tokens, k), dtype=torch.uint8, device="cuda")
        be.gemm_q8_k(m, q8d, n_tokens, y_ws, ws)
        y_na = torch.full((n_tokens, rows), float("nan"), device="cuda")
        be.gemm_q8_k_noalloc(m, q8d, n_tokens, y_na)
        torch.cuda.synchronize()
        a, b = y_ws.cpu().numpy(), y_na.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"call {call}: {n_tokens} tokens"
        for t in (0, n_tokens // 2, n_tokens - 1):
            want = oracle.gemv_prequantized(ex, om, q8[t])
            assert np.array_equal(b[t].view(np.uint32), want.view(np.uint32)), f"call {call} token {t}"
    m.close()


def test_noalloc_gemm_refuses_batches_beyond_the_scratch(be):
    import lbhip
    m = be.upload(Q5_K, 64, 4096, synth.random_matrix(Q5_K, 64, 4096, seed=920))
    m.prepare_gemm()
    for n in (929, 1024):                          # 30 or 32 tiles x 16 blocks x 17,536 B > 8 MiB
        need = be.gemm_workspace_bytes(n, 4096)
        assert need > be.NOALLOC_SCRATCH_BYTES
        q8 = torch.zeros(n * 16 * 292, dtype=torch.uint8, device="cuda")
        y = torch.full((n, 64), 3.0, device="cuda")
        with pytest.raises(lbhip.BackendError) as e:
            be.gemm_q8_k_noalloc(m, q8, n, y)
        assert e.value.variant == "ScratchTooSmall" and e.value.expected == need
        assert e.value.actual == be.NOALLOC_SCRATCH_BYTES
        torch.cuda.synchronize()
        assert bool((y == 3.0).all())
    # the documented limit itself runs: 928 tokens (29 tiles) at k = 4096
    n = 928
    q8 = torch.zeros(n * 16 * 292, dtype=torch.uint8, device="cuda")
    y = torch.full((n, 64), 3.0, device="cuda")
    be.gemm_q8_k_noalloc(m, q8, n, y)
    torch.cuda.synchronize()
    assert bool((y == 0.0).all())                  # zero activations: every dot is 0
    m.close()


def test_noalloc_gemm_refuses_an_overlapping_call_on_another_stream(be):
    """A call queued on stream 1 behind a long (bounded) spin still holds the
    scratch: a call on stream 2 is refused with ScratchInUse and launches
    nothing; once stream 1 has finished, stream 2's call runs and gives the
    same result."""
    import lbhip
    n, rows, k = 64, 256, 4096
    m = be.upload(Q5_K, rows, k, synth.random_matrix(Q5_K, rows, k, seed=930))
    m.prepare_gemm()
    q8h = np.random.default_rng(931).integers(0, 256, (n * 16, 292), dtype=np.uint8)
    q8h[:, :4] = np.array([0.01], np.float32).view(np.uint8)                  # finite d
    q8 = torch.from_numpy(q8h.reshape(-1)).cuda()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    y1 = torch.full((n, rows), float("nan"), device="cuda")
    y2 = torch.full((n, rows), 5.0, device="cuda")
    torch.cuda.synchronize()
    try:
        be.set_stream(s1)
        with torch.cuda.stream(s1):
            torch.cuda._sleep(200_000_000)          # a bounded spin: ~0.1 s at the shader clock
        be.gemm_q8_k_noalloc(m, q8, n, y1)
        be.set_stream(s2)
        with pytest.raises(lbhip.BackendError) as e:
            be.gemm_q8_k_noalloc(m, q8, n, y2)
        assert e.value.variant == "ScratchInUse" and e.value.actual == n
        s1.synchronize()
        assert bool((y2 == 5.0).all())
        be.gemm_q8_k_noalloc(m, q8, n, y2)
        s2.synchronize()
        assert np.array_equal(y1.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))
        assert bool(torch.isfinite(y1).all())
    finally:
        torch.cuda.synchronize()
        be.set_stream(torch.cuda.current_stream())
        m.close()
