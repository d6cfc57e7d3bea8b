"""Pins of the GEGLU -> Q8_0 oracle and the library's host GELU table (CPU only).

The reference's only CPU test of this producer is the layout check at
tests/test_qpu_xla_ggml_geglu_q8.py:24-30; the rest of the pinning comes from
an independent erf, textbook normal-CDF values, identities of GELU and cases
that reduce to the already pinned Q8_0 quantiser.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import scipy.special
import torch

import oracle

FP16_BITS = np.arange(1 << 16, dtype=np.uint16)
FP16_VALUES = FP16_BITS.view(np.float16).astype(np.float64)
FINITE = np.isfinite(FP16_VALUES)


def test_reference_layout_case() -> None:
    # tests/test_qpu_xla_ggml_geglu_q8.py:24-30 of the reference.
    gate = np.linspace(-2.0, 2.0, 64, dtype=np.float32).reshape(1, 64)
    up = np.linspace(0.5, 1.5, 64, dtype=np.float32).reshape(1, 64)
    packed = oracle.geglu_q8_0_reference(gate, up)
    assert packed.shape == (1, 2, 34)
    assert packed.dtype == np.uint8
    assert np.any(packed[..., 2:].view(np.int8) != 0)


def test_table_matches_an_independent_erf() -> None:
    # SciPy's erf (Cephes) is an implementation independent of the C library's
    # erf that Python's math.erf uses; after the fp32 and fp16 roundings every
    # finite entry agrees.
    table = oracle.gelu_fp16_table()
    with np.errstate(invalid="ignore"):
        gelu = 0.5 * FP16_VALUES * (1.0 + scipy.special.erf(FP16_VALUES / math.sqrt(2.0)))
    independent = gelu.astype(np.float32).astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(table[FINITE], independent[FINITE])


@pytest.mark.parametrize("x,phi", [
    (1.0, 0.8413447460685429), (-1.0, 0.15865525393145707),
    (2.0, 0.9772498680518208), (-2.0, 0.022750131948179195),
    (3.0, 0.9986501019683699), (-3.0, 0.0013498980316301035),
])
def test_table_textbook_values(x: float, phi: float) -> None:
    # gelu(x) = x * Phi(x), Phi the standard normal CDF (tabulated values).
    table = oracle.gelu_fp16_table().view(np.float16)
    assert table[np.float16(x).view(np.uint16)] == np.float16(np.float32(x * phi))


def test_table_identities() -> None:
    table = oracle.gelu_fp16_table().view(np.float16).astype(np.float64)
    # gelu(x) = x exactly once Phi(x) rounds to 1 (x >= 6 is far past that in fp16).
    big = FINITE & (FP16_VALUES >= 6.0)
    np.testing.assert_array_equal(table[big], FP16_VALUES[big])
    # gelu(x) - gelu(-x) = x; each entry carries at most half an fp16 ulp of its own
    # magnitude (<= |x|), so the identity holds to one ulp of x.
    positive = FINITE & (FP16_VALUES > 0) & (FP16_VALUES < 60000)
    x = FP16_VALUES[positive]
    negative_bits = (FP16_BITS[positive] | 0x8000)
    residual = table[FP16_BITS[positive]] - table[negative_bits] - x
    ulp = np.spacing(x.astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(residual) <= ulp)
    assert table[0] == 0.0


def test_closed_forms_outside_the_lds_band() -> None:
    # The band kernel keeps fp16 magnitudes in [2^-10, 8) in LDS and uses
    # closed forms beyond: gelu(x) = x for finite x >= 8, -0 for finite x <= -8.
    table = oracle.gelu_fp16_table()
    magnitude = FP16_BITS & 0x7FFF
    beyond = (magnitude >= 0x4800) & (magnitude < 0x7C00)
    positive = beyond & (FP16_BITS < 0x8000)
    negative = beyond & (FP16_BITS >= 0x8000)
    np.testing.assert_array_equal(table[positive], FP16_BITS[positive])
    assert np.all(table[negative] == 0x8000)


def test_library_table_equals_oracle() -> None:
    from qpu_xla_amd import _lib
    from qpu_xla_amd.kernels import ggml_gelu_fp16_table

    raw = np.zeros(1 << 16, dtype=np.uint16)
    _lib.call("qxt_ggml_gelu_fp16_table", raw.ctypes.data_as(ctypes.c_void_p))
    np.testing.assert_array_equal(raw, oracle.gelu_fp16_table())
    mirrored = ggml_gelu_fp16_table()
    assert mirrored.dtype == torch.uint16 and tuple(mirrored.shape) == (1 << 16,)
    np.testing.assert_array_equal(mirrored.view(torch.int16).numpy().view(np.uint16), raw)


def test_table_index_is_round_to_nearest_even() -> None:
    # fp32 gates exactly half-way between neighbouring fp16 values: the index is
    # the even neighbour (torch's half conversion is an independent RNE).
    rng = np.random.default_rng(5001)
    lows = rng.integers(0x0001, 0x7BFF, size=4096).astype(np.uint16)
    low = lows.view(np.float16).astype(np.float64)
    high = (lows + 1).view(np.float16).astype(np.float64)
    mid = ((low + high) / 2).astype(np.float32)
    assert np.all(mid.astype(np.float64) == (low + high) / 2)  # exact in fp32
    signs = np.where(rng.random(4096) < 0.5, -1.0, 1.0).astype(np.float32)
    gate = (mid * signs)[: 4096 // 32 * 32].reshape(-1, 32)
    up = np.ones_like(gate)
    expected_index = torch.from_numpy(gate).half().view(torch.int16).numpy().view(np.uint16)
    table = oracle.gelu_fp16_table()
    activated = oracle.geglu_activate(gate, up)
    np.testing.assert_array_equal(activated, table[expected_index].view(np.float16).astype(np.float32))


def test_identity_and_zero_cases_reduce_to_the_q8_0_quantiser() -> None:
    rng = np.random.default_rng(5002)
    # gelu(x) = x for fp16 gates >= 6: the producer equals the Q8_0 quantiser of up * gate.
    gate = rng.uniform(6.0, 2000.0, size=(3, 96)).astype(np.float16).astype(np.float32)
    up = rng.normal(0.0, 1.0, size=(3, 96)).astype(np.float32)
    np.testing.assert_array_equal(oracle.geglu_q8_0_reference(gate, up), oracle.quantize_q8_0_blocks(gate * up))
    # gelu(x) = -0 for x <= -12 (x Phi(x) underflows fp16): all-zero blocks with d = 0.
    gate = rng.uniform(-60000.0, -12.0, size=(2, 64)).astype(np.float32)
    packed = oracle.geglu_q8_0_reference(gate, up[:2, :64])
    assert np.all(packed == 0)


def test_dequantised_blocks_track_float64_geglu() -> None:
    rng = np.random.default_rng(5003)
    gate = rng.normal(0.0, 1.5, size=(8, 256)).astype(np.float32)
    up = rng.normal(0.0, 1.5, size=(8, 256)).astype(np.float32)
    packed = oracle.geglu_q8_0_reference(gate, up)
    scales, values = oracle.unpack_q8_0_blocks(packed)
    d = scales.astype(np.float64)[..., None]
    decoded = (d * values.astype(np.float64)).reshape(8, 256)
    g = gate.astype(np.float64)
    gelu = 0.5 * g * (1.0 + scipy.special.erf(g / math.sqrt(2.0)))
    exact = gelu * up.astype(np.float64)
    step = np.repeat(scales.astype(np.float64), 32, axis=1)
    # Error budget: rint to half a step; the fp16 scale (at most 127 codes x half an
    # fp16 ulp of d, < 0.07 step); fp16 rounding of the gate index (|gelu'| < 1.13)
    # and of the table entry, each half an fp16 ulp, scaled by |up|.
    tolerance = 0.57 * step + np.abs(up) * (2.0 ** -11 * (1.13 * np.abs(g) + np.abs(gelu)) + 2.0 ** -24)
    assert np.all(np.abs(decoded - exact) <= tolerance)


def test_split_planes_match_native_blocks() -> None:
    rng = np.random.default_rng(5004)
    gate = rng.normal(0.0, 0.8, size=(5, 160)).astype(np.float32)
    up = rng.normal(0.0, 0.8, size=(5, 160)).astype(np.float32)
    packed = oracle.geglu_q8_0_reference(gate, up)
    scale_words, values = oracle.geglu_q8_0_split_reference(gate, up)
    assert scale_words.dtype == np.uint32 and values.dtype == np.int8
    np.testing.assert_array_equal(scale_words.astype(np.uint16), packed[..., :2].copy().view(np.uint16)[..., 0])
    np.testing.assert_array_equal(values.view(np.uint8).reshape(5, 5, 32), packed[..., 2:])
    assert np.all(scale_words >> 16 == 0)


def test_producer_input_checks() -> None:
    with pytest.raises(ValueError):
        oracle.geglu_q8_0_reference(np.zeros((2, 32), np.float32), np.zeros((2, 64), np.float32))
    with pytest.raises(ValueError):
        oracle.geglu_q8_0_reference(np.zeros((2, 48), np.float32), np.zeros((2, 48), np.float32))
