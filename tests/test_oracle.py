"""Pins the CPU oracle (oracle/) against things other than itself: exact rational arithmetic, the committed
known-answer fixtures of tests/golden/, the reference's own bounds, closed forms and invariants. CPU only."""

from __future__ import annotations

import json
import math
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import linear_set as OL
from oracle import mlstm as OM
from oracle import numerics as ON
from oracle import skinny as OS
from tests.exact import BF16, FP16, bf16_bits_exact, exact_round

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---- bf16 / fp16 rounding ---------------------------------------------------------------------------------------


def _f32(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", bits))[0]


@pytest.mark.parametrize("bits,expect", [
    (0x3F800000, 0x3F80),  # 1.0
    (0x3F808000, 0x3F80),  # 1 + 2^-8: exact tie, even mantissa stays
    (0x3F818000, 0x3F82),  # 1 + 3 * 2^-8: tie, odd mantissa rounds up
    (0x3F808001, 0x3F81),  # just above the tie
    (0x3FFF8000, 0x4000),  # carry into the exponent: 1.99609375 -> 2.0
    (0x7F7FFFFF, 0x7F80),  # float max rounds to inf
    (0xFF7FFFFF, 0xFF80),  # -float max -> -inf
    (0x80000000, 0x8000),  # -0.0
    (0x00000001, 0x0000),  # smallest subnormal rounds to +0
    (0x00018000, 0x0002),  # subnormal tie with odd mantissa -> rounds up
    (0x7F800000, 0x7F80),  # inf
])
def test_bf16_rounding_known_answers(bits, expect):
    assert int(ON.bf16_bits(np.array([_f32(bits)], np.float32))[0]) == expect
    assert bf16_bits_exact(_f32(bits)) == expect


def test_bf16_rounding_nan_stays_nan():
    out = ON.bf16_round(np.array([np.nan, -np.nan], np.float32))
    assert np.isnan(out).all()


def test_bf16_rounding_matches_exact_rounding_on_sampled_patterns():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=4000, dtype=np.uint64).astype(np.uint32)
    # add patterns near ties: low 16 bits = 0x8000 +- 1
    hi = rng.integers(0, 2**16, size=600, dtype=np.uint64).astype(np.uint32) << 16
    bits = np.concatenate([bits, hi | 0x8000, hi | 0x7FFF, hi | 0x8001])
    vals = bits.view(np.float32)
    got = ON.bf16_bits(vals)
    for v, g in zip(vals, got):
        if math.isnan(v):
            continue
        assert bf16_bits_exact(float(v)) == int(g), hex(struct.unpack('<I', struct.pack('<f', float(v)))[0])


def test_f16_rounding_matches_exact_rounding():
    rng = np.random.default_rng(1)
    vals = (rng.standard_normal(2000) * rng.choice([1e-6, 1e-3, 1.0, 100.0, 6e4], 2000)).astype(np.float32)
    got = ON.f16_round(vals)
    for v, g in zip(vals, got):
        r = exact_round(Fraction(float(v)), FP16)
        assert (float(r) if not isinstance(r, float) else r) == float(g)


# ---- matmul oracle ----------------------------------------------------------------------------------------------


def test_matmul_oracle_against_exact_rational_sum():
    rng = np.random.default_rng(2)
    x = ON.bf16_round(rng.standard_normal((3, 40)).astype(np.float32))
    w = ON.bf16_round((rng.standard_normal((5, 40)) * 0.02).astype(np.float32))
    y = OS.matmul(x, w)
    for a in range(3):
        for b in range(5):
            exact = sum(Fraction(float(p)) * Fraction(float(q)) for p, q in zip(x[a], w[b]))
            assert abs(Fraction(float(y[a, b])) - exact) <= abs(exact) * Fraction(1, 2**48) + Fraction(1, 2**100)


def test_skinny_oracle_against_committed_exact_fixture():
    cases = json.loads((GOLDEN / "skinny_kat.json").read_text())["cases"]
    for c in cases:
        x = np.array(c["x"], np.float32)
        w = np.array(c["w"], np.float32)
        got = ON.bf16_bits(OS.skinny_bf16(x, w))
        want = np.array(c["y_bf16_bits"], np.uint16)
        # the oracle rounds float64 -> float32 -> bf16; the fixture rounds the exact sum once. They may differ only
        # where the exact value sits within float64 error of a bf16 tie; none of these cases does.
        assert np.array_equal(got, want), (c["m"], c["n"], c["k"])


def test_skinny_oracle_known_answer_by_hand():
    x = np.array([[1.0, 2.0, -1.0, 0.5]], np.float32)
    w = np.array([[1.0, 1.0, 1.0, 1.0], [0.5, -0.25, 2.0, 4.0], [0.0, 0.0, 0.0, 0.0]], np.float32)
    assert OS.skinny_bf16(x, w).tolist() == [[2.5, 0.0, 0.0]]
    q = np.array([[1, -2, 3, 127]], np.int8)
    assert OS.skinny_int8(x, q, np.array([0.5], np.float32)).tolist() == [[0.5 * (1 - 4 - 3 + 63.5)]]


def test_dequantize_known_answer():
    q = np.array([[1, -127], [64, 0]], np.int8)
    s = np.array([0.25, 2.0 ** -7], np.float32)
    assert OS.dequantize("int8", q, s).tolist() == [[0.25, -31.75], [0.5, 0.0]]


# ---- int8 quantizer ---------------------------------------------------------------------------------------------


def test_quantizer_against_committed_exact_fixture():
    cases = json.loads((GOLDEN / "quantizer_kat.json").read_text())["cases"]
    assert len(cases) >= 16
    for c in cases:
        q, s = OS.quantize_rowwise_int8(np.array([c["w"]], np.float32), c["scale_dtype"])
        assert q[0].tolist() == c["q"], c
        assert float(s[0]) == c["scale"], c


def test_quantizer_error_bound_of_the_reference_test():
    """byteprof tests/test_quant_int8.py:10-16: per-row error <= 0.51 step + 1e-3, |q| <= 127."""
    rng = np.random.default_rng(3)
    w = ON.bf16_round(rng.standard_normal((16, 256)).astype(np.float32))
    q, s = OS.quantize_rowwise_int8(w)
    assert np.abs(q.astype(np.int32)).max() <= 127
    deq = q.astype(np.float32) * s[:, None]
    assert (np.abs(deq - w).max(axis=1) <= s * 0.51 + 1e-3).all()
    # the row maximum maps to +-127 (within one step of the bf16-rounded scale)
    am = np.abs(w).argmax(axis=1)
    assert (np.abs(q[np.arange(16), am].astype(np.int32)) >= 126).all()


# ---- mLSTM oracle -----------------------------------------------------------------------------------------------


def _mlstm_inputs(t, nh, dq, dv, seed, m_scale=1.0):
    rng = np.random.default_rng(seed)
    c = rng.standard_normal((nh, dq, dv)) * 0.1
    n = rng.standard_normal((nh, dq)) * 0.1
    m = rng.standard_normal(nh) * m_scale
    q = rng.standard_normal((t, nh, dq))
    k = rng.standard_normal((t, nh, dq))
    v = rng.standard_normal((t, nh, dv))
    i = rng.standard_normal((t, nh))
    f = rng.standard_normal((t, nh)) + 3.0
    return c, n, m, q, k, v, i, f


@pytest.mark.parametrize("t", [1, 2, 5, 9])
def test_mlstm_stabilised_equals_unstabilised_closed_form(t):
    """The stabiliser only rescales C, n by exp(-m_t): with no roundings and eps = 0 both formulas agree."""
    c, n, m, q, k, v, i, f = _mlstm_inputs(t, 3, 8, 5, seed=t)
    h, _ = OM.multistep(c, n, m, q, k, v, i, f, eps=0.0, io="f64")
    ref = OM.unstabilised(c, n, m, q, k, v, i, f)
    assert np.allclose(h, ref, rtol=1e-11, atol=1e-13)


def test_mlstm_composition_of_steps():
    c, n, m, q, k, v, i, f = _mlstm_inputs(7, 2, 8, 4, seed=11)
    h_all, st_all = OM.multistep(c, n, m, q, k, v, i, f, eps=1e-6, io="bf16")
    h1, st1 = OM.multistep(c, n, m, q[:3], k[:3], v[:3], i[:3], f[:3], eps=1e-6, io="bf16")
    h2, st2 = OM.multistep(*st1, q[3:], k[3:], v[3:], i[3:], f[3:], eps=1e-6, io="bf16")
    assert np.array_equal(h_all, np.concatenate([h1, h2]))
    for a, b in zip(st_all, st2):
        assert np.array_equal(a, b)


def test_mlstm_pure_decay_when_the_input_gate_is_closed():
    """i -> -inf: C_T = C_0 exp(sum logsigmoid(f) + m_0 - m_T), no k v^T contribution."""
    c, n, m, q, k, v, i, f = _mlstm_inputs(4, 2, 8, 4, seed=5)
    i = np.full_like(i, -1e4)
    _, (C, N, M) = OM.multistep(c, n, m, q, k, v, i, f, eps=0.0, io="f64")
    decay = np.exp(OM.logsigmoid(f).sum(axis=0) + m - M)
    assert np.allclose(C, c * decay[:, None, None], rtol=1e-12)
    assert np.allclose(N, n * decay[:, None], rtol=1e-12)
    assert np.allclose(M, m + OM.logsigmoid(f).sum(axis=0), rtol=1e-12)


def test_mlstm_single_step_from_an_empty_state():
    """T = 1 from C = n = 0 and m_0 = -inf-like: m_1 = i, C_1 = k v^T, n_1 = k, h = qs.(k v^T) / max(|qs.k|, e^-i)."""
    rng = np.random.default_rng(7)
    dq, dv = 8, 3
    q = rng.standard_normal((1, 1, dq))
    k = rng.standard_normal((1, 1, dq))
    v = rng.standard_normal((1, 1, dv))
    i = np.array([[0.3]])
    f = np.array([[2.0]])
    h, (C, N, M) = OM.multistep(np.zeros((1, dq, dv)), np.zeros((1, dq)), np.array([-1e9]), q, k, v, i, f,
                                eps=0.0, io="f64")
    qs = q[0, 0] / math.sqrt(dq)
    want = (qs @ k[0, 0]) * v[0, 0] / max(abs(qs @ k[0, 0]), math.exp(-0.3))
    assert np.allclose(h[0, 0], want, rtol=1e-12)
    assert np.allclose(C[0], np.outer(k[0, 0], v[0, 0]), rtol=1e-12) and M[0] == pytest.approx(0.3)


def test_mlstm_io_rounding_is_applied_to_h():
    c, n, m, q, k, v, i, f = _mlstm_inputs(3, 2, 8, 4, seed=9)
    h, _ = OM.multistep(c, n, m, q, k, v, i, f, eps=1e-6, io="bf16")
    assert np.array_equal(h, ON.bf16_round(h.astype(np.float32)).astype(np.float64))
    h32, _ = OM.multistep(c, n, m, q, k, v, i, f, eps=1e-6, io="f32")
    assert ON.normwise_error(h, h32) < 1e-2  # bf16 roundings stay inside the reference's bf16 tolerance


def test_literal_gate_reading_differs_from_the_reference_reading():
    """Read literally, the stabiliser is m_t = max(f + m, i) with f ~ N(3, 1); the reference applies logsigmoid(f) first
    (mlstm_multistep.py:25-26). With f taken literally as a log forget gate the state grows ~e^3 per step
    (in the stabilised form: m grows by ~3 per step while C keeps its scale), so the two readings give different h."""
    c, n, m, q, k, v, i, f = _mlstm_inputs(6, 2, 8, 4, seed=13)
    h_ref, st_ref = OM.multistep(c, n, m, q, k, v, i, f, eps=1e-6, io="f64")
    h_lit, st_lit = OM.multistep(c, n, m, q, k, v, i, f, eps=1e-6, io="f64", literal_gate=True)
    assert ON.normwise_error(h_lit, h_ref) > 1e-2
    assert (st_lit[2] - m).min() > 6 * 2.0  # m grew by about f per step (f ~ 3)
    assert (st_ref[2] - m).max() < 6 * 0.5  # logsigmoid(f) ~ -0.05: m barely moves


def test_error_metrics():
    y = np.array([[1.0, 2.0]])
    assert ON.normwise_error(y, np.array([[1.0, 2.5]])) == pytest.approx(0.2)
    x = np.array([[1.0, -1.0]])
    w = np.array([[1.0, 1.0]])  # exact output 0 (cancelling): componentwise error normalises by |x||w| = 2
    assert ON.componentwise_error(np.array([[0.01]]), x, w) == pytest.approx(0.005)


# ---- decode-step set oracle -------------------------------------------------------------------------------------


def test_unit_rms_of_a_constant_vector_is_all_ones():
    # mean(c^2) = c^2 exactly, sqrt = |c|: a dropped mean or square root would give sqrt(K) or c instead of 1
    for c in (0.375, -3.0, 17.0):
        out = OL.unit_rms(np.full(2048, c, np.float32))
        assert np.all(out == np.sign(c))


def test_unit_rms_is_invariant_to_power_of_two_scaling():
    rng = np.random.default_rng(7)
    x = ON.bf16_round(rng.standard_normal(4096).astype(np.float32))
    base = OL.unit_rms(x)
    for e in (-20, -3, 5, 30):
        assert np.array_equal(OL.unit_rms(x * np.float32(2.0 ** e)), base)


def test_unit_rms_output_has_unit_mean_square_and_zero_stays_zero():
    rng = np.random.default_rng(8)
    x = ON.bf16_round((rng.standard_normal(8192) * 40).astype(np.float32))
    out = OL.unit_rms(x)
    assert abs(float(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 2.0 ** -7
    assert np.array_equal(ON.bf16_round(out), out)  # bf16 values
    assert np.all(OL.unit_rms(np.zeros(512, np.float32)) == 0)


def test_chain_second_stage_reads_the_first_stage_output():
    """Two stages by hand: stage 1 reads stage 0's outputs 2..5 renormalised; K = 4, exact small integers."""
    w0 = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [1, 1, 0, 0], [0, 0, 1, 1], [2, 0, 0, 2], [0, 0, 0, 1]], np.float32)
    w1 = np.array([[1, 1, 1, 1]], np.float32)
    x0 = np.array([1, 2, 3, 4], np.float32)
    st0 = OL.OracleStage([w0], ("ext", x0), renorm=False)
    st1 = OL.OracleStage([w1], ("stage", 0, 2), renorm=True)
    xs, ys = OL.chain([st0, st1])
    assert np.array_equal(ys[0], [1, 2, 3, 7, 10, 4])
    # stage 1 input: unit_rms([3, 7, 10, 4]) = [3, 7, 10, 4] / sqrt(174 / 4)
    expect = ON.bf16_round(np.array([3, 7, 10, 4], np.float32) * np.float32(1.0 / np.sqrt(43.5)))
    assert np.array_equal(xs[1], expect)
    assert np.array_equal(ys[1], ON.bf16_round(np.array([expect.astype(np.float64).sum()], np.float32)))


# ---- int4 group-128 format ---------------------------------------------------------------------------------------


@pytest.mark.parametrize("n,rows", [(32, 32), (37, 32), (5, 16), (64, 16)])
def test_int4_pack_round_trip_and_documented_layout(n, rows):
    """byteprof tests/test_skinny.py:47-53: byte j of a row's group holds code j (low nibble), code j + 64 (high)."""
    rng = np.random.default_rng(n + rows)
    q = rng.integers(0, 16, (n, 384), dtype=np.uint8)
    packed = OS.pack_int4(q, rows)
    assert packed.shape == (-(-n // rows), 3, rows, 64) and packed.dtype == np.uint8
    assert np.array_equal(OS.unpack_int4(packed, n), q)
    assert int(packed[0, 1, 0, 5]) == int(q[0, 128 + 5]) | (int(q[0, 128 + 64 + 5]) << 4)
    if n % rows:
        assert not packed[-1, :, n % rows:].any()  # padding rows are zero


def test_int4_quantizer_known_answer_by_hand():
    """A group from -1.5 to 6: scale = 7.5 / 15 = 0.5 and zero = 3 are exact; code = rint(w / 0.5 + 3) with ties to
    even: 0.25 -> 3.5 -> 4, 0.75 -> 4.5 -> 4, 1.25 -> 5.5 -> 6; the extremes map to 0 and 15."""
    w = np.zeros((1, 128), np.float32)
    w[0, :6] = [-1.5, 6.0, 0.25, 0.75, 1.25, -0.5]
    packed, scale, zero = OS.quantize_int4(w, 16)
    assert scale.shape == zero.shape == (1, 1) and scale[0, 0] == 0.5 and zero[0, 0] == 3.0
    codes = OS.unpack_int4(packed, 1)[0]
    assert list(codes[:6]) == [0, 15, 4, 4, 6, 2]
    assert (codes[6:] == 3).all()  # w = 0 -> zero


def test_int4_quantizer_rounds_scale_and_zero_to_their_stored_types():
    """scale is stored in bf16 and zero in fp16 before the codes are computed (the codes use the stored values)."""
    rng = np.random.default_rng(3)
    w = ON.bf16_round((rng.standard_normal((8, 256)) * 0.05).astype(np.float32))
    packed, scale, zero = OS.quantize_int4(w)
    assert np.array_equal(scale, ON.bf16_round(scale)) and np.array_equal(zero, ON.f16_round(zero))
    codes = OS.unpack_int4(packed, 8).astype(np.float32).reshape(8, 2, 128)
    want = np.clip(np.rint((w.reshape(8, 2, 128) / scale.T[..., None]).astype(np.float32) + zero.T[..., None]), 0, 15)
    assert np.array_equal(codes, want)


def test_int4_quantization_error_is_at_most_half_a_step():
    """byteprof tests/test_skinny.py:56-62."""
    rng = np.random.default_rng(4)
    w = ON.bf16_round((rng.standard_normal((24, 256)) * 0.05).astype(np.float32))
    packed, scale, zero = OS.quantize_int4(w)
    deq = OS.dequantize_int4(packed, scale, zero)
    step = np.repeat(scale.T, 128, axis=1)
    assert (np.abs(deq - w) <= 0.55 * step + 1e-3).all()
    assert OS.unpack_int4(packed, 24).max() <= 15
    with pytest.raises(ValueError):
        OS.quantize_int4(np.zeros((4, 100), np.float32))


def test_int4_skinny_oracle_against_exact_rational_sum():
    rng = np.random.default_rng(5)
    n, k, m = 5, 256, 3
    codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
    packed = OS.pack_int4(codes, 16)
    scale = ON.bf16_round(rng.uniform(0.01, 0.1, (2, n)).astype(np.float32))
    zero = ON.f16_round(rng.uniform(0, 15, (2, n)).astype(np.float32))
    x = ON.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    y = OS.skinny_int4(x, packed, scale, zero)
    for i in range(m):
        for j in range(n):
            exact = sum(Fraction(float(x[i, kk])) * (int(codes[j, kk]) - Fraction(float(zero[kk // 128, j])))
                        * Fraction(float(scale[kk // 128, j])) for kk in range(k))
            assert y[i, j] == np.float32(exact_round(exact, BF16)), (i, j)


# ---- drafting bookkeeping ----------------------------------------------------------------------------------------


def test_accepted_length_known_answers_of_the_reference():
    """byteprof tests/test_fused_kernels_gpu.py:116-126 (drafts ids[1:] against the verifier's tokens)."""
    from oracle import draft as OD

    ids = [10, 5, 6, 7, 8, 9]
    for tok, want in (([5, 6, 99, 8, 9, 3], 2), ([5, 6, 7, 8, 9 + 260, 3], 4), ([1, 6, 7, 8, 9, 3], 0),
                      ([5, 6, 7, 8, 9, 3], 5)):
        assert OD.accepted_length(ids, tok, 6) == want
    assert OD.accepted_length(ids, [5], 1) == 0  # a single position has no draft to accept


def test_committed_state_is_the_multistep_state_of_the_prefix():
    from oracle import draft as OD

    rng = np.random.default_rng(6)
    t, nh, dq, dv = 5, 2, 4, 3
    c, n, m = rng.standard_normal((nh, dq, dv)), rng.standard_normal((nh, dq)), rng.standard_normal(nh)
    k, v = rng.standard_normal((t, nh, dq)), rng.standard_normal((t, nh, dv))
    i, f = rng.standard_normal((t, nh)), rng.standard_normal((t, nh)) + 2
    for length in (0, 2, 4, 9):
        st = OD.committed_state(c, n, m, k, v, i, f, length, "f64")
        steps = min(length + 1, t)
        _, want = OM.multistep(c, n, m, k[:steps], k[:steps], v[:steps], i[:steps], f[:steps], eps=1e-6, io="f64")
        for a, b in zip(st, want):
            assert np.array_equal(a, b)
    c0, n0, m0 = OD.committed_state(c, n, m, k, v, i, f, -1, "f64")
    assert np.array_equal(c0, c) and np.array_equal(n0, n) and np.array_equal(m0, m)
