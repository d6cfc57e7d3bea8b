"""Pins the oracle of the bridge's approximate weight modes (``oracle/llama_approx.py``).

The reference's C prepare/submit code cannot be built here (it needs the QPU
runtime and generated program headers), so the oracle is pinned by
hand-worked known answers whose literal values separate the plausible
mistakes (round half to even or exact rounding instead of the fp32
``+ 0.5`` then truncation; multiplying by a reciprocal instead of dividing;
applying the column scale per block instead of once; dropping a scale), by
random columns re-derived in exact rational arithmetic with explicit
round-to-fp32 steps, and by power-of-two-scale cases whose results are exact.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

import oracle
from oracle.llama_approx import (
    column_w8_reference,
    requantize_q4_0_columns_w8,
    requantize_q8_0_rows_w8,
    round_half_away_w8,
    rowcol_w8a8_reference,
)
from q4_0_kats import _rn32


def test_rounding_rule_known_answers() -> None:
    s = np.array([0.5, 1.5, 2.5, -0.5, -2.5, 126.5, 127.6, -300.0, 0.0, -0.0, 1e-8,
                  np.float32(0.49999997), np.float32(-0.49999997), np.float32(0.4999999)], dtype=np.float32)
    # 2.5 -> 3 and -2.5 -> -3 (half away from zero, not to even); 0.49999997 + 0.5
    # rounds to 1.0 in fp32 before the truncation, so it gives 1, not 0;
    # 0.4999999 + 0.5 stays below 1.
    expected = [1, 2, 3, -1, -3, 127, 127, -127, 0, 0, 0, 1, -1, 0]
    np.testing.assert_array_equal(round_half_away_w8(s), expected)
    assert float(np.float32(0.49999997)) == 0.5 - 2.0**-25


def _q4_block(d: float, codes: list[int]) -> np.ndarray:
    return oracle.pack_q4_0_blocks(np.array([[d]], dtype=np.float16), np.array([[codes]], dtype=np.int64))[0, 0]


def test_column_requantisation_known_answers() -> None:
    # Block 0: d = 15.875, code 0 -> -8 * 15.875 = -127, the column's largest
    # magnitude, so the column scale is exactly 127 / 127 = 1.
    # Block 1: d = 0.5, so each value is (code - 8) / 2 and its code is that
    # value rounded half away from zero.
    b0 = [0] + [8] * 31
    b1 = [13, 3, 11, 5, 9, 7, 15, 1, 8] + [8] * 23
    column = np.stack([_q4_block(15.875, b0), _q4_block(0.5, b1)])[None]
    wq, cs = requantize_q4_0_columns_w8(column)
    assert cs.dtype == np.float32 and cs[0] == 1.0
    assert wq[0, 0] == -127 and not wq[0, 1:32].any()
    # 2.5 -> 3, -2.5 -> -3, 1.5 -> 2, -1.5 -> -2, 0.5 -> 1, -0.5 -> -1, 3.5 -> 4, -3.5 -> -4, 0 -> 0
    np.testing.assert_array_equal(wq[0, 32:41], [3, -3, 2, -2, 1, -1, 4, -4, 0])
    assert not wq[0, 41:].any()

    # A zero column keeps scale 0 and all-zero codes (no division).
    zero = np.stack([_q4_block(0.0, [3] * 32), _q4_block(1.0, [8] * 32)])[None]
    wq, cs = requantize_q4_0_columns_w8(zero)
    assert cs[0] == 0.0 and not wq.any()


def test_row_requantisation_known_answers() -> None:
    # Row max |q * d| = 127 * 1.0, so the row scale is 1; a second block with
    # d = 0.5 rounds its halves away from zero; a zero row keeps scale 0.
    vals = np.zeros((2, 2, 32), dtype=np.int64)
    vals[0, 0, 0] = 127
    vals[0, 1, :4] = [5, -5, 3, -3]
    act = oracle.pack_q8_0_blocks(np.array([[1.0, 0.5], [0.25, 0.25]], dtype=np.float16), vals)
    aq, rs = requantize_q8_0_rows_w8(act)
    assert rs[0] == 1.0 and rs[1] == 0.0
    assert aq[0, 0] == 127
    np.testing.assert_array_equal(aq[0, 32:36], [3, -3, 2, -2])
    assert not aq[1].any()


def _exact_codes(values: np.ndarray) -> tuple[list[int], float]:
    """The rounding rule in exact rational arithmetic with explicit fp32 steps."""
    maximum = max(Fraction(float(abs(v))) for v in values)
    scale = _rn32(maximum / 127) if maximum > 0 else Fraction(0)
    codes = []
    for v in values:
        if scale == 0:
            codes.append(0)
            continue
        s = _rn32(Fraction(float(v)) / scale)
        shifted = _rn32(s + Fraction(1, 2)) if s >= 0 else _rn32(s - Fraction(1, 2))
        q = int(shifted)  # int() of a Fraction truncates toward zero
        codes.append(max(-127, min(127, q)))
    return codes, float(scale)


def test_column_requantisation_matches_exact_arithmetic_on_random_columns() -> None:
    rng = np.random.default_rng(11)
    n, blocks = 6, 4
    scales = rng.uniform(0.001, 0.05, (n, blocks)).astype(np.float16)
    weights = oracle.pack_q4_0_blocks(scales, rng.integers(0, 16, (n, blocks, 32)))
    wq, cs = requantize_q4_0_columns_w8(weights)
    d, vals = oracle.unpack_q4_0_blocks(weights)
    separates_reciprocal = False
    for c in range(n):
        exact = (vals[c].astype(np.float32) * d[c][:, None]).astype(np.float32).reshape(-1)
        codes, scale = _exact_codes(exact)
        assert cs[c] == np.float32(scale)
        np.testing.assert_array_equal(wq[c], codes)
        # Multiplying by fl32(1 / scale) instead of dividing changes a code somewhere here.
        recip = np.float32(1.0) / np.float32(scale)
        alt = round_half_away_w8((exact * recip).astype(np.float32))
        separates_reciprocal |= bool((alt != wq[c]).any())
    assert separates_reciprocal


def test_row_requantisation_matches_exact_arithmetic_on_random_rows() -> None:
    rng = np.random.default_rng(12)
    m, blocks = 5, 3
    act = oracle.pack_q8_0_blocks(rng.uniform(0.001, 0.1, (m, blocks)).astype(np.float16),
                                  rng.integers(-128, 128, (m, blocks, 32)))
    aq, rs = requantize_q8_0_rows_w8(act)
    d, vals = oracle.unpack_q8_0_blocks(act)
    for r in range(m):
        exact = (vals[r].astype(np.float32) * d[r][:, None]).astype(np.float32).reshape(-1)
        codes, scale = _exact_codes(exact)
        assert rs[r] == np.float32(scale)
        np.testing.assert_array_equal(aq[r], codes)


def test_column_w8_linear_power_of_two_scales_is_exact() -> None:
    # Power-of-two activation and column scales with small codes: every fp32
    # step is exact, so the result equals the float64 dequantised dot.
    rng = np.random.default_rng(13)
    m, n, blocks = 3, 5, 4
    da = np.float16(2.0**-4) * np.ones((m, blocks), dtype=np.float16)
    da[1] = np.float16(2.0**-2)
    act = oracle.pack_q8_0_blocks(da, rng.integers(-20, 21, (m, blocks, 32)))
    wq = rng.integers(-20, 21, (n, blocks * 32)).astype(np.int8)
    cs = (2.0 ** rng.integers(-3, 3, n)).astype(np.float32)
    got = column_w8_reference(act, wq, cs)
    d, a = oracle.unpack_q8_0_blocks(act)
    deq = (a.astype(np.float64) * d[:, :, None].astype(np.float64)).reshape(m, -1)
    np.testing.assert_array_equal(got, (deq @ wq.astype(np.float64).T) * cs[None, :].astype(np.float64))


def test_column_w8_linear_applies_the_column_scale_once() -> None:
    # Two blocks with terms 1 and 2^-24 and column scale 3: the finished sum
    # fl32(1 + 2^-24) = 1 times 3 is 3, whereas scaling each term first gives
    # fl32(3 + fl32(3 * 2^-24)) = 3 + 2^-22.
    act = oracle.pack_q8_0_blocks(np.array([[1.0, 2.0**-24]], dtype=np.float16),
                                  np.array([[[1] + [0] * 31, [1] + [0] * 31]]))
    wq = np.zeros((1, 64), dtype=np.int8)
    wq[0, 0] = wq[0, 32] = 1
    got = column_w8_reference(act, wq, np.array([3.0], dtype=np.float32))
    assert got[0, 0] == np.float32(3.0)
    per_block = np.float32(3.0) + np.float32(np.float32(3.0) * np.float32(2.0**-24))
    assert per_block != np.float32(3.0)


def test_column_w8_linear_uses_each_blocks_activation_scale() -> None:
    # Block b of the row has da = 2^-b and a single product 1 * (b + 1).
    blocks = 4
    da = np.array([[2.0**-b for b in range(blocks)]], dtype=np.float16)
    vals = np.zeros((1, blocks, 32), dtype=np.int64)
    vals[0, :, 7] = 1
    act = oracle.pack_q8_0_blocks(da, vals)
    wq = np.zeros((1, blocks * 32), dtype=np.int8)
    for b in range(blocks):
        wq[0, b * 32 + 7] = b + 1
    got = column_w8_reference(act, wq, np.array([1.0], dtype=np.float32))
    assert got[0, 0] == np.float32(1 + 2 * 0.5 + 3 * 0.25 + 4 * 0.125)


def test_rowcol_w8a8_linear_known_answer() -> None:
    # dot = 3 * 2 + (-4) * 5 = -14; y = fl32(fl32(-14 * 0.5) * 0.25) = -1.75.
    aq = np.zeros((1, 32), dtype=np.int8)
    wq = np.zeros((1, 32), dtype=np.int8)
    aq[0, :2] = [3, -4]
    wq[0, :2] = [2, 5]
    got = rowcol_w8a8_reference(aq, np.array([0.5], np.float32), wq, np.array([0.25], np.float32))
    assert got[0, 0] == np.float32(-1.75)


@pytest.mark.parametrize("seed", [0, 1])
def test_rowcol_w8a8_reduces_to_the_w8a8_epilogue(seed: int) -> None:
    rng = np.random.default_rng(seed)
    aq = rng.integers(-127, 128, (4, 64)).astype(np.int8)
    wq = rng.integers(-127, 128, (6, 64)).astype(np.int8)
    rs = rng.uniform(0.01, 1, 4).astype(np.float32)
    cs = rng.uniform(0.01, 1, 6).astype(np.float32)
    acc = (aq.astype(np.int64) @ wq.astype(np.int64).T)
    want = ((acc.astype(np.float32) * rs[:, None]).astype(np.float32) * cs[None, :]).astype(np.float32)
    np.testing.assert_array_equal(rowcol_w8a8_reference(aq, rs, wq, cs), want)
