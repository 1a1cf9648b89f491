"""Closed-form, invariant and error-path checks of the CPU oracle.

What the golden fixtures leave open is pinned here by mathematics rather than by
retyping the oracle's formulas:
* the integer stage of every dot equals sum(decode(w) * q8) computed from the
  fixture-pinned decoders on blocks whose f16 scales are set to 1.0 / 0.0 (the
  decoded weights are then exact integers, so the identity is exact);
* f16 -> f32 conversion equals numpy's IEEE conversion on all 65536 inputs;
* Q8_K invariants (bsums, |q| <= 127, round-half-even KAT of q8_k.rs:737-751);
* error atomicity (crates/bridge-quant-layout/tests/q8_k.rs:12-153);
* MoE / SwiGLU / routing closed forms (crates/bridge-kernels-reference/tests/moe.rs,
  crates/bridge-model-hy3/tests/routing.rs).
"""
import numpy as np
import pytest

from lbhip import synth

Q4_K, Q5_K, IQ3_S, IQ2_S, F32 = 12, 13, 21, 22, 0
TYPES = [Q4_K, Q5_K, IQ2_S, IQ3_S]


def sentinel_bytes(n):
    return ((np.arange(n) * 37 + 11) & 0xFF).astype(np.uint8)


def test_f16_conversion_is_exact_for_every_bit_pattern(oracle):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    lib = oracle.lib()
    got = np.array([lib.lbo_f16_to_f32(int(v)) for v in h], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isinf(got[np.isinf(want)]))


def test_nearest_int_rounds_half_to_even(oracle):
    # max |x| = 127 at lane 0 (negative) gives iscale = -127 / -127 = 1.0 exactly,
    # so q = nearest_int(x) for the other lanes (q8_k.rs:737-751 cases).
    x = np.zeros(256, np.float32)
    x[0] = -127.0
    cases = [(-2.5, -2), (-1.5, -2), (-0.5, 0), (0.5, 0), (1.5, 2), (2.5, 2), (3.5, 4)]
    for i, (v, _) in enumerate(cases, start=1):
        x[i] = v
    enc = oracle.quantize_q8_k(x)
    q = enc[4:260].view(np.int8)
    assert q[0] == -127
    assert [int(q[i]) for i in range(1, 8)] == [e for _, e in cases]
    assert enc[0:4].view(np.float32)[0] == np.float32(1.0)


def test_first_index_wins_an_abs_tie_and_sets_the_sign(oracle):
    x = np.zeros(256, np.float32)
    x[3], x[9] = 2.0, -2.0
    enc = oracle.quantize_q8_k(x)
    assert enc[4 + 3].view(np.int8) == -127 and enc[4 + 9].view(np.int8) == 127
    x[3], x[9] = -2.0, 2.0
    enc = oracle.quantize_q8_k(x)
    assert enc[4 + 3].view(np.int8) == -127 and enc[4 + 9].view(np.int8) == 127
    assert enc[0:4].view(np.float32)[0] > 0


def test_q8_k_invariants_on_random_rows(oracle):
    rng = np.random.default_rng(7)
    for scale in (1.0, 1e-30, 1e30, 1e-42):
        x = (rng.standard_normal(4096) * scale).astype(np.float32)
        enc = oracle.quantize_q8_k(x)
        for b in range(16):
            blk = enc[b * 292:(b + 1) * 292]
            q = blk[4:260].view(np.int8).astype(np.int32)
            bs = blk[260:292].view(np.int16).astype(np.int32)
            assert np.all(np.abs(q) <= 127)
            assert np.array_equal(bs, q.reshape(16, 16).sum(1))
            xb = x[b * 256:(b + 1) * 256]
            amax_i = int(np.argmax(np.abs(xb)))
            with np.errstate(over="ignore"):
                iscale = np.float32(-127.0) / xb[amax_i]
            d = blk[0:4].view(np.float32)[0]
            assert d.view(np.uint32) == (np.float32(1.0) / iscale).view(np.uint32)
            if np.isfinite(iscale):
                assert q[amax_i] == -127
            else:
                # Subnormal block maximum: -127/max overflows, every quant
                # becomes nearest_int(+-inf) = -0x400000 -> i8 0, d = -0.0 or +0.0.
                assert np.all(q == 0) and d == 0.0


def test_zero_blocks_are_fully_deterministic(oracle):
    out = np.full(584, 0xA5, np.uint8)
    oracle.quantize_row_q8_k_into(np.zeros(512, np.float32), out)
    assert np.all(out == 0)
    out = np.full(292, 0xA5, np.uint8)
    oracle.quantize_row_q8_k_into(-np.zeros(256, np.float32), out)
    assert np.all(out == 0)


def test_quantize_errors_leave_output_unchanged(oracle):
    out = sentinel_bytes(292)
    before = out.copy()
    with pytest.raises(oracle.OracleError) as e:
        oracle.quantize_row_q8_k_into(np.zeros(0, np.float32), out)
    assert e.value.status == "ZeroLogicalElements"
    with pytest.raises(oracle.OracleError) as e:
        oracle.quantize_row_q8_k_into(np.zeros(255, np.float32), out)
    assert e.value.status == "LogicalElementsNotDivisible" and e.value.actual == 255
    for n in (0, 1, 291, 293):
        buf = sentinel_bytes(n)
        b0 = buf.copy()
        with pytest.raises(oracle.OracleError) as e:
            oracle.quantize_row_q8_k_into(np.zeros(256, np.float32), buf)
        assert e.value.status == "EncodedLengthMismatch" and e.value.actual == n
        assert np.array_equal(buf, b0)
    for idx in (0, 127, 255, 256, 511):
        for bits in (0x7F800000, 0xFF800000, 0x7FC00001, 0xFFA12345):
            x = np.zeros(512, np.float32)
            x.view(np.uint32)[idx] = bits
            buf = sentinel_bytes(584)
            b0 = buf.copy()
            with pytest.raises(oracle.OracleError) as e:
                oracle.quantize_row_q8_k_into(x, buf)
            assert e.value.status == "NonFiniteActivation"
            assert (e.value.index, e.value.bits) == (idx, bits)
            assert np.array_equal(buf, b0)
    assert np.array_equal(out, before)


def test_dot_validation_errors(oracle):
    q4 = np.zeros(144, np.uint8)
    q8 = np.zeros(292, np.uint8)
    with pytest.raises(oracle.OracleError, match="UnsupportedType"):
        oracle.vec_dot_q8_k(F32, q4, q8, 256)
    with pytest.raises(oracle.OracleError, match="ZeroLogicalElements"):
        oracle.vec_dot_q8_k(Q4_K, q4, q8, 0)
    with pytest.raises(oracle.OracleError, match="LogicalElementsNotDivisible"):
        oracle.vec_dot_q8_k(Q4_K, q4, q8, 1)
    with pytest.raises(oracle.OracleError) as e:
        oracle.vec_dot_q8_k(Q4_K, q4[:143], q8, 256)
    assert (e.value.status, e.value.expected, e.value.actual) == ("EncodedLengthMismatch", 144, 143)
    with pytest.raises(oracle.OracleError) as e:
        oracle.vec_dot_q8_k(Q4_K, q4, q8[:291], 256)
    assert (e.value.status, e.value.ty, e.value.actual) == ("EncodedLengthMismatch", 15, 291)
    bad = q4.copy()
    bad[0:2] = np.array([0x7C00], np.uint16).view(np.uint8)
    with pytest.raises(oracle.OracleError) as e:
        oracle.vec_dot_q8_k(Q4_K, bad, q8, 256)
    assert (e.value.status, e.value.index, e.value.field, e.value.bits) == ("NonFiniteScale", 0, 0, 0x7C00)
    bad = q4.copy()
    bad[2:4] = np.array([0xFC00], np.uint16).view(np.uint8)
    with pytest.raises(oracle.OracleError) as e:
        oracle.vec_dot_q8_k(Q4_K, bad, q8, 256)
    assert (e.value.status, e.value.field) == ("NonFiniteScale", 1)
    nq = q8.copy()
    nq[0:4] = np.array([0x7FC00000], np.uint32).view(np.uint8)
    with pytest.raises(oracle.OracleError) as e:
        oracle.vec_dot_q8_k(Q4_K, q4, nq, 256)
    assert (e.value.status, e.value.bits) == ("NonFiniteQ8Scale", 0x7FC00000)


def _unit_scales(ty, blk, d=0x3C00, dmin=0x0000):
    blk = blk.copy()
    blk[:, 0:2] = np.array([d], np.uint16).view(np.uint8)
    if ty in (Q4_K, Q5_K):
        blk[:, 2:4] = np.array([dmin], np.uint16).view(np.uint8)
    return blk


@pytest.mark.parametrize("ty", TYPES)
def test_integer_block_sums_equal_decoded_weights_times_q8(oracle, ty):
    """With d = 1 (and dmin = 0) the decoded weights are exact small integers
    (IQ2_S: scaled by 1/8), so sum(decode * q) pins the integer stage exactly."""
    rng = np.random.default_rng(100 + ty)
    nb = 6
    blk = synth.random_blocks(ty, nb, rng)
    x = rng.standard_normal(nb * 256).astype(np.float32)
    q8 = oracle.quantize_q8_k(x)
    q = np.concatenate([q8[b * 292 + 4:b * 292 + 260].view(np.int8) for b in range(nb)]).astype(np.int64)
    w1 = _unit_scales(ty, blk)
    dec = oracle.decode_row(ty, w1.reshape(-1), nb * 256).astype(np.float64)
    sums = oracle.block_sums(ty, w1.reshape(-1), q8)
    if ty in (IQ2_S, IQ3_S):
        mult = 8.0 if ty == IQ2_S else 1.0
        ints = np.rint(dec * mult).astype(np.int64)
        assert np.array_equal(ints, dec * mult)
        want = (ints * q).reshape(nb, 256).sum(1)
        assert np.array_equal(sums, want)
    else:
        ints = np.rint(dec).astype(np.int64)
        assert np.array_equal(ints, dec)
        prod = (ints * q).reshape(nb, 32, 8)
        assert np.array_equal(sums[:, :8], prod.sum(1))
        # d = 0, dmin = 1: decode = -min, so sum(decode * q) = -minimum_sum.
        w0 = _unit_scales(ty, blk, d=0x0000, dmin=0x3C00)
        dec0 = oracle.decode_row(ty, w0.reshape(-1), nb * 256).astype(np.float64)
        ms = oracle.block_sums(ty, w0.reshape(-1), q8)[:, 8]
        assert np.array_equal(ms, -(np.rint(dec0).astype(np.int64) * q).reshape(nb, 256).sum(1))


@pytest.mark.parametrize("ty", TYPES)
def test_dot_matches_dequantized_closed_form(oracle, ty):
    rng = np.random.default_rng(200 + ty)
    for trial in range(4):
        nb = 16
        w = synth.random_blocks(ty, nb, rng).reshape(-1)
        x = rng.standard_normal(nb * 256).astype(np.float32)
        q8 = oracle.quantize_q8_k(x)
        dot = float(oracle.vec_dot_q8_k(ty, w, q8, nb * 256)[0])
        dec = oracle.decode_row(ty, w, nb * 256).astype(np.float64)
        d8 = np.repeat([q8[b * 292:b * 292 + 4].view(np.float32)[0] for b in range(nb)], 256)
        q = np.concatenate([q8[b * 292 + 4:b * 292 + 260].view(np.int8) for b in range(nb)])
        terms = dec * d8.astype(np.float64) * q
        assert abs(dot - terms.sum()) <= 1e-5 * np.abs(terms).sum() + 1e-30


@pytest.mark.parametrize("ty", TYPES)
def test_scalar_and_avx2_dots_are_bit_identical(oracle, ty):
    rng = np.random.default_rng(300 + ty)
    for trial in range(16):
        nb = int(rng.integers(1, 20))
        w = synth.random_blocks(ty, nb, rng).reshape(-1)
        q8 = oracle.quantize_q8_k((rng.standard_normal(nb * 256) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32))
        a = oracle.vec_dot_q8_k(ty, w, q8, nb * 256, avx2=False)
        b = oracle.vec_dot_q8_k(ty, w, q8, nb * 256, avx2=True)
        assert a.view(np.uint32)[0] == b.view(np.uint32)[0]


@pytest.mark.parametrize("ty", TYPES)
def test_parallel_gemv_equals_scalar_gemv(oracle, ty):
    """bridge-kernels-reference/tests/gemv.rs:131-168: CpuParallelQ8K == LlamaQ8K bit for bit."""
    rows, k = 37, 1024
    w = synth.random_matrix(ty, rows, k, seed=ty)
    x = synth.random_activations(k, seed=1)
    m = oracle.make_matrix(ty, rows, k, w)
    a = oracle.gemv(oracle.make_exec(oracle.MODE_LLAMA_Q8K), m, x)
    b = oracle.gemv(oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, threads=4, avx2=True), m, x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    q8 = oracle.quantize_q8_k(x)
    for r in range(rows):
        assert oracle.vec_dot_q8_k(ty, w[r], q8, k).view(np.uint32)[0] == a.view(np.uint32)[r]


def test_f32_router_gemv_known_answer(oracle):
    """bridge-kernels-reference/tests/gemv.rs:44-73."""
    w = np.array([1.0, 2.0, 3.0, -1.0, 0.5, 4.0, 0.25, -0.75, 2.5, 3.0, -2.0, 1.0], np.float32)
    m = oracle.make_matrix(F32, 4, 3, w.view(np.uint8))
    for mode in (oracle.MODE_LLAMA_Q8K, oracle.MODE_CPU_PARALLEL_Q8K):
        y = oracle.gemv(oracle.make_exec(mode, threads=2), m, np.array([2.0, -1.0, 0.5], np.float32))
        assert y.tolist() == [1.5, -0.5, 2.5, 8.5]
    assert oracle.router_logits_f32(w, np.array([2.0, -1.0, 0.5], np.float32)).tolist() == [1.5, -0.5, 2.5, 8.5]


def test_scaled_accumulation_preserves_initialized_destination(oracle):
    w = np.array([1.0, 2.0, 3.0, -1.0, 0.5, 4.0], np.float32)
    m = oracle.make_matrix(F32, 2, 3, w.view(np.uint8))
    dest = np.array([10.0, -4.0], np.float32)
    oracle.gemv_accumulate(oracle.make_exec(oracle.MODE_DEQUANT_F32), m, np.array([2.0, -1.0, 0.5], np.float32),
                           dest, 0.5)
    assert dest.tolist() == [10.75, -4.25]


def _f32_expert(oracle, g, u, d):
    mats = [oracle.make_matrix(F32, 1, 1, np.array([v], np.float32).view(np.uint8)) for v in (g, u, d)]
    return oracle.make_expert(*mats)


def test_routed_and_shared_accumulate_in_declared_order(oracle):
    """bridge-kernels-reference/tests/moe.rs:106-154 (bit-exact closed form)."""
    f = np.float32
    ex = np.frompyfunc(lambda v: oracle.lib().lbo_expf(float(v)), 1, 1)

    def se(x, g, u, d):
        gate, up = f(g) * f(x), f(u) * f(x)
        e = f(ex(-gate))
        return f(d) * (gate / (f(1.0) + e) * up)

    a, b, s = _f32_expert(oracle, 1.0, 2.0, 3.0), _f32_expert(oracle, -1.0, 0.5, 4.0), _f32_expert(oracle, 0.25, 3.0, -2.0)
    experts = [a] * 2 + [a] + [a] * 4 + [b]
    want = f(f(f(0.25) * se(2.0, 1.0, 2.0, 3.0)) + f(f(0.75) * se(2.0, -1.0, 0.5, 4.0))) + se(2.0, 0.25, 3.0, -2.0)
    for pre in (True, False):
        out = oracle.moe_routed_by_id(oracle.make_exec(oracle.MODE_DEQUANT_F32), [2, 7], [0.25, 0.75], experts, s,
                                      np.array([2.0], np.float32), preflight=pre)
        assert out.view(np.uint32)[0] == np.array([want], np.float32).view(np.uint32)[0]


def test_zero_weight_iq_expert_outputs_zero(oracle):
    """bridge-kernels-reference/tests/moe.rs:79-104."""
    gate = oracle.make_matrix(IQ2_S, 256, 256, np.zeros(82 * 256, np.uint8))
    up = oracle.make_matrix(IQ2_S, 256, 256, np.zeros(82 * 256, np.uint8))
    down = oracle.make_matrix(IQ3_S, 1, 256, np.zeros(110, np.uint8))
    e = oracle.make_expert(gate, up, down)
    x = np.full(256, 0.25, np.float32)
    for mode in (oracle.MODE_DEQUANT_F32, oracle.MODE_LLAMA_Q8K):
        out = oracle.moe_routed_by_id(oracle.make_exec(mode), [0], [1.0], [e], e, x)
        assert out.tolist() == [0.0]


def test_moe_rejects_order_and_duplicates(oracle):
    e = _f32_expert(oracle, 1.0, 1.0, 1.0)
    x = np.array([1.0], np.float32)
    ex = oracle.make_exec(oracle.MODE_DEQUANT_F32)
    with pytest.raises(oracle.OracleError, match="RoutedExpertOrder"):
        oracle.moe_routed_by_id(ex, [3, 2], [0.5, 0.5], [e] * 4, e, x)
    with pytest.raises(oracle.OracleError, match="DuplicateRoutedExpert"):
        oracle.moe_routed_by_id(ex, [2, 2], [0.5, 0.5], [e] * 4, e, x)
    with pytest.raises(oracle.OracleError, match="InvalidParameter"):
        oracle.moe_routed_by_id(ex, [5], [0.5], [e] * 4, e, x)
    with pytest.raises(oracle.OracleError, match="NonFiniteValue"):
        oracle.moe_routed_by_id(ex, [1], [np.inf], [e] * 4, e, x)


def test_moe_preflight_and_single_pass_agree_on_quantized_experts(oracle):
    rng_seed = 11
    hidden, ffn = 512, 256
    experts = []
    for i in range(4):
        g = oracle.make_matrix(IQ2_S, ffn, hidden, synth.random_matrix(IQ2_S, ffn, hidden, rng_seed + 3 * i))
        u = oracle.make_matrix(IQ2_S, ffn, hidden, synth.random_matrix(IQ2_S, ffn, hidden, rng_seed + 3 * i + 1))
        d = oracle.make_matrix(IQ3_S, hidden, ffn, synth.random_matrix(IQ3_S, hidden, ffn, rng_seed + 3 * i + 2))
        experts.append(oracle.make_expert(g, u, d))
    sh = oracle.make_expert(
        oracle.make_matrix(Q4_K, 512, hidden, synth.random_matrix(Q4_K, 512, hidden, 90)),
        oracle.make_matrix(Q4_K, 512, hidden, synth.random_matrix(Q4_K, 512, hidden, 91)),
        oracle.make_matrix(Q5_K, hidden, 512, synth.random_matrix(Q5_K, hidden, 512, 92)))
    x = synth.random_activations(hidden, 5)
    a = oracle.moe_routed_by_id(oracle.make_exec(oracle.MODE_LLAMA_Q8K), [0, 2, 3], [0.2, 0.3, 0.5], experts, sh, x, True)
    b = oracle.moe_routed_by_id(oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 4, True), [0, 2, 3], [0.2, 0.3, 0.5],
                                experts, sh, x, False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.all(np.isfinite(a)) and np.any(a != 0)


def test_sigmoid_routing_ties_bias_sorting_and_floor(oracle):
    """crates/bridge-model-hy3/tests/routing.rs:45-126."""
    ids, coefs = oracle.route_sigmoid_bias(np.zeros(4), np.zeros(4), 3, 2.826)
    assert ids.tolist() == [0, 1, 2]
    assert np.allclose(coefs, 2.826 / 3.0, atol=1e-6)
    ids, coefs = oracle.route_sigmoid_bias([3.0, 1.0, -1.0, -3.0], [0.0, 0.0, 2.0, 4.0], 2, 2.0)
    assert ids.tolist() == [2, 3]
    w2, w3 = 1 / (1 + np.exp(1.0)), 1 / (1 + np.exp(3.0))
    assert np.allclose(coefs, [w2 / (w2 + w3) * 2.0, w3 / (w2 + w3) * 2.0], atol=1e-6)
    ids, _ = oracle.route_sigmoid_bias([0.0, 4.0, -4.0, 2.0], np.zeros(4), 3, 1.0)
    assert ids.tolist() == [0, 1, 3]
    fmin = np.finfo(np.float32).min
    ids, coefs = oracle.route_sigmoid_bias([fmin, fmin], [0.0, 0.0], 2, 2.826)
    assert coefs.tolist() == [0.0, 0.0]
    with pytest.raises(oracle.OracleError, match="InvalidParameter"):
        oracle.route_sigmoid_bias([0.0, 1.0, 2.0], np.zeros(3), 0, 1.0)
    with pytest.raises(oracle.OracleError, match="InvalidParameter"):
        oracle.route_sigmoid_bias([0.0, 1.0, 2.0], np.zeros(3), 4, 1.0)
    with pytest.raises(oracle.OracleError) as e:
        oracle.route_sigmoid_bias([0.0, np.inf, 2.0], np.zeros(3), 2, 1.0)
    assert e.value.index == 1


def test_softmax_topk_router_matches_float64_softmax(oracle):
    rng = np.random.default_rng(3)
    for trial in range(20):
        logits = rng.standard_normal(192).astype(np.float32)
        ids, coefs = oracle.route_softmax_topk(logits, 8)
        top = np.argsort(-logits.astype(np.float64), kind="stable")[:8]
        assert ids.tolist() == sorted(top.tolist())
        l64 = logits[ids].astype(np.float64)
        p = np.exp(l64 - l64.max())
        p /= p.sum()
        assert np.allclose(coefs, p, rtol=1e-6, atol=0)
        assert abs(float(coefs.astype(np.float64).sum()) - 1.0) < 1e-6


def test_residual_add_restates_the_reference_tests(oracle):
    """crates/bridge-kernels-reference/tests/norm.rs:41-46 and :76-79."""
    v = np.array([1.0, -2.0, 3.5], np.float32)
    oracle.residual_add_in_place(v, [2.0, 1.0, -0.5])
    assert v.tolist() == [3.0, -1.0, 3.0]
    r = np.array([np.finfo(np.float32).max, 1.0], np.float32)
    before = r.copy()
    with pytest.raises(oracle.OracleError) as e:
        oracle.residual_add_in_place(r, [np.finfo(np.float32).max, 2.0])
    assert e.value.status == "NonFiniteValue" and e.value.index == 0 and e.value.field == 2
    assert np.array_equal(r.view(np.uint32), before.view(np.uint32))
    with pytest.raises(oracle.OracleError, match="DimensionMismatch"):
        oracle.residual_add_in_place(np.zeros(3, np.float32), [1.0, 2.0])
    d = np.array([1.0, np.nan], np.float32)
    with pytest.raises(oracle.OracleError) as e:
        oracle.residual_add_in_place(d, [1.0, 1.0])
    assert (e.value.index, e.value.field) == (1, 0)
    with pytest.raises(oracle.OracleError) as e:
        oracle.residual_add_in_place(np.ones(2, np.float32), [1.0, np.inf])
    assert (e.value.index, e.value.field) == (1, 1)


def test_dequant_sum_is_sequential_in_the_oracle(oracle):
    """dot_dequant_row (gemv.rs:322-325) is one f32 chain in element order: a row
    decoding to ones against [2^24, 1, 1, -2^24] sums to 0 (each +1 rounds back to
    2^24); pairwise summation would give 1 and exact summation 2."""
    from lbhip import synth
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    blk[4:16] = synth.pack_scale_min(np.ones((1, 8), np.int64), np.zeros((1, 8), np.int64))[0]
    blk[16:144] = 0x11
    assert np.all(oracle.decode_row(12, blk, 256) == 1.0)
    x = np.zeros(256, np.float32)
    x[:4] = [2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)]
    y = oracle.gemv(oracle.make_exec(oracle.MODE_DEQUANT_F32), oracle.make_matrix(12, 1, 256, blk), x)
    assert y[0] == 0.0


def test_router_logits_are_a_sequential_sum_in_the_oracle(oracle):
    """dot_f32_row (gemv.rs:286-303): ((2^24 + 1) + 1) - 2^24 = 0 in f32."""
    w = np.ones((2, 256), np.float32)
    x = np.zeros(256, np.float32)
    x[:4] = [2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)]
    assert oracle.router_logits_f32(w, x).tolist() == [0.0, 0.0]
