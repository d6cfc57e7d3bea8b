"""The arithmetic identity behind the prefill kernels' biased block dots (CPU).

The Q4_0 x Q8_0 prefill kernels give the matrix core an accumulator input of
the bit pattern 0x4B400000 (the float 1.5 * 2^23) in every output, read the
int32 result as a float f = 1.5 * 2^23 + dot, and form fl32(float(dot) * dw)
as one fma(f, dw, -1.5 * 2^23 * dw) when dw is finite.  These checks run
over every finite fp16 scale and dots across the whole int8 x int8 block
range; the fma is emulated in float64, where f * dw (24 x 11 significant
bits) and the sum dot * dw (at most 20 x 11 bits) are exact, so one rounding
to float32 is the fma's.
"""

from __future__ import annotations

import numpy as np

BIAS_BITS = 0x4B400000
BIAS = 12582912.0


def _dots() -> np.ndarray:
    rng = np.random.default_rng(5)
    edges = [0, 1, -1, 2, -2, 3, 127, -128, 1023, -1024, 32767, -32768, 32768, 2**19 - 1, -(2**19)]
    return np.concatenate([np.array(edges), rng.integers(-(2**19), 2**19, 240)]).astype(np.int64)


def _finite_fp16_scales() -> np.ndarray:
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    values = bits.view(np.float16)
    return values[np.isfinite(values)].astype(np.float32)


def test_biased_int32_result_reads_as_bias_plus_dot() -> None:
    dots = _dots()
    assert np.abs(dots).max() <= 32 * 128 * 128  # any two int8 blocks of 32
    f = (BIAS_BITS + dots).astype(np.uint32).view(np.float32)
    np.testing.assert_array_equal(f.astype(np.float64), BIAS + dots.astype(np.float64))
    # f - 1.5 * 2^23 in float32 is the exact conversion (the slow form).
    np.testing.assert_array_equal(f - np.float32(BIAS), dots.astype(np.float32))


def test_fma_of_biased_dot_equals_convert_then_multiply_for_every_finite_fp16_scale() -> None:
    dw = _finite_fp16_scales()
    assert dw.size == 63488
    c = (np.float32(-BIAS) * dw).astype(np.float32)
    # The addend is exact: 1.5 * 2^23 * dw needs 13 significant bits.
    np.testing.assert_array_equal(c.astype(np.float64), -BIAS * dw.astype(np.float64))
    for dot in _dots():
        f = np.float64(BIAS + float(dot))
        fused = (f * dw.astype(np.float64) + c.astype(np.float64)).astype(np.float32)
        want = (np.float32(dot) * dw).astype(np.float32)
        # Equal as values; only a zero's sign may differ (the fma's exact zero
        # is +0 where dot * dw is -0), which the +0-started accumulator absorbs.
        assert np.array_equal(fused, want), dot
        nonzero = want != 0
        np.testing.assert_array_equal(np.signbit(fused[nonzero]), np.signbit(want[nonzero]))
        assert not np.signbit(fused[~nonzero]).any()


def test_a_plausible_slip_fails_the_identity() -> None:
    # Rounding the addend's product (e.g. a bias of 1.5 * 2^23 + 1) or
    # multiplying the biased value first and subtracting after each changes results.
    dw = _finite_fp16_scales()
    dot = np.int64(12345)
    f = np.float64(BIAS + float(dot))
    want = (np.float32(dot) * dw).astype(np.float32)
    off_by_one = (f * dw.astype(np.float64) - (BIAS + 1.0) * dw.astype(np.float64)).astype(np.float32)
    assert not np.array_equal(off_by_one, want)
    two_roundings = ((np.float32(f) * dw).astype(np.float32) - (np.float32(BIAS) * dw).astype(np.float32)).astype(np.float32)
    assert not np.array_equal(two_roundings, want)
