"""Pin the NumPy oracle of the W8A8 path against KATs, brute force and closed forms."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
import q8_0_kats
from conftest import load_golden


def test_w8a8_kat_matches_native_smoke() -> None:
    # integrations/llama_cpp/tests/qpu_llama_w8a8_smoke.c:58-66
    g = load_golden("kat_w8a8")
    acc = oracle.int8_gemm_i32(g["activation"], np.ascontiguousarray(g["weight_kn"].T))
    np.testing.assert_array_equal(acc, g["expected"])


@pytest.mark.parametrize("shape", [(16, 16, 16), (32, 64, 32)])
def test_int8_gemm_matches_python_brute_force(shape) -> None:
    p, q, r = shape
    rng = np.random.default_rng(91 + q)  # seeds of tests/test_qpu_xla_gemm_int8.py:28-54
    left = rng.integers(-127, 128, size=(p, q), dtype=np.int8)
    right = rng.integers(-127, 128, size=(q, r), dtype=np.int8)
    acc = oracle.int8_gemm_i32(left, np.ascontiguousarray(right.T))
    for i in range(0, p, 7):
        for j in range(0, r, 5):
            assert acc[i, j] == sum(int(left[i, k]) * int(right[k, j]) for k in range(q))


def test_int8_gemm_float64_path_is_exact_at_the_int32_limit() -> None:
    rng = np.random.default_rng(17)
    k = 4096
    a = rng.choice(np.array([-127, 127], np.int8), size=(8, k))
    w = rng.choice(np.array([-127, 127], np.int8), size=(1024, k))
    w[0] = a[0]  # acc[0, 0] = 4096 * 127**2, the largest magnitude this K allows
    exact = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.int32)
    got = oracle.int8_gemm_i32(a, w)  # M*N*K > 2**24: float64 BLAS branch
    np.testing.assert_array_equal(got, exact)
    assert got[0, 0] == k * 127 * 127


def test_overflow_guard_matches_reference_bound() -> None:
    limit = (2**31 - 1) // (127 * 127)
    oracle.w8a8.check_accumulation_range(limit)
    with pytest.raises(ValueError):
        oracle.w8a8.check_accumulation_range(limit + 1)


def test_pack_int8_quads_layout() -> None:
    # tests/test_qpu_xla_gemm_int8.py:17-25 in the reference.
    left = np.array([[-128, -1, 0, 127, 3, -4, 5, -6]], dtype=np.int8)
    right = np.arange(-16, 16, dtype=np.int8).reshape(8, 4)
    packed_left, packed_right = oracle.pack_int8_gemm_operands(left, right)
    assert packed_left.shape == (1, 2) and packed_right.shape == (2, 4)
    np.testing.assert_array_equal(packed_left.view(np.uint8).reshape(1, 8).view(np.int8), left)
    np.testing.assert_array_equal(oracle.pack_int8_quads(np.ascontiguousarray(right.T)).view(np.uint8).reshape(4, 8).view(np.int8), right.T)
    assert packed_left[0, 0] == (0x80 | 0xFF << 8 | 0x00 << 16 | 0x7F << 24)


def test_row_quantiser_reference_reconstruction() -> None:
    # tests/test_qpu_xla_quantization.py:28-34 in the reference.
    weight = np.array([[0.0, -1.0, 0.25], [2.0, -0.5, 1.0]], dtype=np.float32)
    values, scales = oracle.quantize_per_output_channel_int8(weight)
    assert values.dtype == np.int8
    np.testing.assert_allclose(values.astype(np.float32) * scales[:, None], weight, atol=0.01, rtol=0.01)


def test_row_quantiser_invariants_and_floor() -> None:
    rng = np.random.default_rng(23)
    x = rng.standard_normal((5, 300), dtype=np.float32)
    x[1] *= np.float32(1e-3)  # absmax/127 < 1/127: floor active
    x[2] = 0.0
    q, s = oracle.quantize_rows_int8(x)
    assert np.all(s >= np.float32(1.0 / 127.0))
    assert s[1] == np.float32(1.0 / 127.0) and s[2] == np.float32(1.0 / 127.0)
    np.testing.assert_array_equal(q[2], 0)
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    for r in (0, 3, 4):
        assert s[r] == np.abs(x[r]).max() / np.float32(127.0)
        assert abs(int(q[r, np.abs(x[r]).argmax()])) == 127
    err = np.abs(x - q.astype(np.float32) * s[:, None])
    assert np.all(err <= s[:, None] * 0.5000001)


def test_row_quantiser_half_even_at_unit_scale() -> None:
    # At scale 1 division and reciprocal agree; this pins only the rounding.
    x = np.array([[127.0, 2.5, 3.5, -2.5, -126.5, 0.5]], dtype=np.float32)
    q, s = oracle.quantize_rows_int8(x)
    assert s[0] == np.float32(1.0)
    np.testing.assert_array_equal(q[0], [127, 2, 4, -2, -126, 0])


@pytest.mark.parametrize("kat", q8_0_kats.row_kats(), ids=lambda k: k[0])
def test_row_quantiser_known_answer_rows(kat) -> None:
    # Literal codes and scale bits at non-unit scales (tests/q8_0_kats.py
    # gives the fp32 quotient each literal rounds).
    name, row, floor, scale_bits, codes = kat
    q, s = oracle.quantize_rows_int8(row[None, :], floor=floor)
    assert int(s.view(np.uint32)[0]) == scale_bits, name
    np.testing.assert_array_equal(q[0].astype(np.int64), q8_0_kats.expected_codes(codes, row.size), err_msg=name)
    exact_s, exact = q8_0_kats.exact_row(row, floor=floor)
    assert exact == q8_0_kats.expected_codes(codes, row.size), name
    assert float(exact_s) == float(s[0]), name


def test_row_known_answers_reject_the_plausible_mistakes() -> None:
    # A reciprocal product instead of the true quotient, or half-away-from-zero
    # rounding, changes at least one literal code of the separator row; the
    # floor row's codes change without the floor.
    name, row, floor, _, codes = q8_0_kats.row_kats()[0]
    want = q8_0_kats.expected_codes(codes, row.size)
    for mistake in ("reciprocal", "half_away"):
        _, wrong = q8_0_kats.exact_row(row, floor=floor, **{mistake: True})
        assert wrong != want, mistake
    _, row, _, _, codes = q8_0_kats.row_kats()[1]
    assert q8_0_kats.exact_row(row, floor=False)[1] != q8_0_kats.expected_codes(codes, row.size)


def test_weight_scale_floor_is_active_at_baseline_shapes() -> None:
    # BASELINE cfg1 weights ~N(0, 0.05) at K=512: absmax < 1, so scale = 1/127.
    rng = np.random.default_rng(1)
    w = rng.standard_normal((512, 512), dtype=np.float32) * np.float32(0.05)
    _, s = oracle.quantize_per_output_channel_int8(w)
    assert np.all(s == np.float32(1.0 / 127.0))


def test_epilogue_multiplies_in_order_then_adds_bias_separately() -> None:
    # (1 * (1 + 2**-12)) * (1 + 2**-12) = 1 + 2**-11 + 2**-24 rounds (tie to even)
    # to 1 + 2**-11; the separate bias add of -1 then gives exactly 2**-11.  A fused
    # multiply-add would keep the 2**-24 term.
    acc = np.array([[1]], np.int32)
    s = np.array([1 + 2.0**-12], np.float32)
    y = oracle.dequantize_epilogue(acc, s, s, np.array([-1.0], np.float32))
    assert y[0, 0] == np.float32(2.0**-11)


def test_fused_fixture_matches_reference_expression() -> None:
    # tests/test_qpu_xla_gemm_int8.py:57-92: expected = acc.astype(f32) * sa[:, None] * sw[None, :]
    g = load_golden("oracle_w8a8_fused_seed1765")
    acc = (g["left"].astype(np.int64) @ g["right"].astype(np.int64)).astype(np.int32)
    np.testing.assert_array_equal(acc, g["acc"])
    expected = acc.astype(np.float32) * g["row_scales"][:, None] * g["column_scales"][None, :]
    np.testing.assert_array_equal(g["expected"], expected)


def test_linear_reference_composes_quantiser_gemm_and_bias() -> None:
    rng = np.random.default_rng(73)
    x = rng.standard_normal((3, 32), dtype=np.float32)
    w = rng.standard_normal((5, 32), dtype=np.float32)
    bias = rng.standard_normal(5, dtype=np.float32)
    qw, sw = oracle.quantize_per_output_channel_int8(w)
    y = oracle.w8a8_linear_reference(x, qw, sw, bias)
    # float64 dequantised reference: error bounded by the two quantisation steps
    approx = x.astype(np.float64) @ w.astype(np.float64).T + bias
    assert np.abs(y - approx).max() < 0.02 * np.abs(approx).max()
    qa, sa = oracle.quantize_rows_int8(x)
    exact = (qa.astype(np.float64) * sa[:, None]) @ (qw.astype(np.float64) * sw[:, None]).T + bias
    np.testing.assert_allclose(y, exact, rtol=1e-5, atol=1e-5)
