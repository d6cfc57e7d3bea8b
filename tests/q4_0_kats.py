"""Known-answer blocks for the GGML Q4_0 weight quantiser.

ggml's published reference quantiser (``quantize_row_q4_0_ref`` in llama.cpp's
``ggml-quants.c``; the reference calls it as ``quantize_row_q4_0`` from
``integrations/llama_cpp/tests/qpu_ggml_backend_smoke.cpp:119``) does, per
32-element block, in fp32:

* ``max`` = the first element of largest magnitude (strict ``amax < |v|``
  scan, so a later element of equal magnitude never replaces it; +0.0 when
  every element is zero),
* ``d = max / -8`` and ``id = d ? 1/d : 0``,
* ``code = MIN(15, (int8_t)(x * id + 8.5f))``, stored with ``d`` as fp16 (RNE).

Each block below is built so that one plausible mistake changes at least one
code or scale bit, and its expected codes are written out as literals worked
by hand from that rule (comments give the arithmetic).  ``exact_codes``
re-derives a block in exact rational arithmetic with explicit round-to-fp32
steps, an implementation independent of NumPy's float32 kernels.
"""

from __future__ import annotations

from fractions import Fraction
import math

import numpy as np


def f32_bits(bits: int) -> np.float32:
    return np.array([bits], dtype=np.uint32).view(np.float32)[0]


def _block(entries: dict[int, float], fill: float = 0.0) -> np.ndarray:
    block = np.full(32, fill, dtype=np.float32)
    for index, value in entries.items():
        block[index] = np.float32(value)
    return block


# (name, 32 fp32 values, expected fp16 scale bits, expected codes by index; other indexes -> fill code)
def kat_blocks() -> list[tuple[str, np.ndarray, int, dict[int, int], int]]:
    kats = []

    # d = -8 / -8 = 1, id = 1: the code is floor(x + 8.5) exactly, so every
    # half-way value k + 0.5 rounds UP (round-half-even would send 0.5 -> 8 and
    # -7.5 -> 0; trunc(x + 8) would send -7.5 -> 0; half away from zero sends
    # -0.5 -> 7).  7.5 -> 16 is clamped to 15.
    halves = [-7.5, -6.5, -5.5, -4.5, -3.5, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, 7.5]
    whole = [0.0, 1.0, -1.0, 2.0, -2.0, 3.0, -3.0, 4.0, -4.0, 5.0, -5.0, 6.0, -6.0, 7.0, -7.0]
    values = [-8.0] + halves + whole
    codes = [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 15,
             8, 9, 7, 10, 6, 11, 5, 12, 4, 13, 3, 14, 2, 15, 1]
    kats.append(("half_way_values_round_up", np.array(values, np.float32), 0x3C00, dict(enumerate(codes)), 8))

    # Largest element positive (+4 at index 5): d = -0.5 (0xB800), id = -2.
    # 4 -> -8 + 8.5 -> 0; -3 -> 6 + 8.5 -> 14; 1 -> 6.5 -> 6; -1 -> 10.5 -> 10;
    # 0.25 -> 8.0 -> 8; -0.25 -> 9.0 -> 9; 0.75 -> 7.0 -> 7; 3.75 -> 1.0 -> 1;
    # -3.75 -> 16.0 -> 15; -3.5 -> 15.5 -> 15.
    kats.append((
        "largest_positive",
        _block({5: 4.0, 0: -3.0, 1: 1.0, 2: -1.0, 3: 0.25, 4: -0.25, 6: 0.75, 7: 3.75, 8: -3.75, 9: -3.5}),
        0xB800,
        {5: 0, 0: 14, 1: 6, 2: 10, 3: 8, 4: 9, 6: 7, 7: 1, 8: 15, 9: 15},
        8,
    ))

    # Largest element negative (-4 at index 2): d = 0.5 (0x3800), id = 2.
    # -4 -> 0; 3 -> 14.5 -> 14; 1 -> 10.5 -> 10; -1 -> 6.5 -> 6; -0.25 -> 8.0 -> 8;
    # 3.75 -> 16.0 -> 15.
    kats.append((
        "largest_negative",
        _block({2: -4.0, 0: 3.0, 1: 1.0, 3: -1.0, 4: -0.25, 5: 3.75}),
        0x3800,
        {2: 0, 0: 14, 1: 10, 3: 6, 4: 8, 5: 15},
        8,
    ))

    # Tie in magnitude, negative first (-2 at 3, +2 at 7): the first wins,
    # d = 0.25 (0x3400), id = 4: -2 -> 0, 2 -> 15, 0.5 -> 10.5 -> 10.
    kats.append(("tie_negative_first", _block({0: 0.5, 3: -2.0, 7: 2.0}), 0x3400, {0: 10, 3: 0, 7: 15}, 8))
    # The same tie, positive first: d = -0.25 (0xB400), id = -4:
    # 2 -> 0, -2 -> 15, 0.5 -> -2 + 8.5 -> 6.
    kats.append(("tie_positive_first", _block({0: 0.5, 3: 2.0, 7: -2.0}), 0xB400, {0: 6, 3: 0, 7: 15}, 8))

    # All zero (and all -0.0): max stays +0.0, d = 0 / -8 = -0.0 (0x8000),
    # id = 0, every code 8.
    kats.append(("all_zero", np.zeros(32, np.float32), 0x8000, {}, 8))
    kats.append(("all_negative_zero", np.full(32, -0.0, np.float32), 0x8000, {}, 8))

    # fp16-subnormal scale: max = 2^-17 -> d = -2^-20 = -16 * 2^-24 (0x8010),
    # id = -2^20 exactly.  2^-17 -> 0; -2^-17 -> 15; 2^-18 -> -4 + 8.5 -> 4;
    # -2^-19 -> 2 + 8.5 -> 10; 3 * 2^-20 -> -3 + 8.5 -> 5.
    kats.append((
        "fp16_subnormal_scale",
        _block({0: 2.0**-17, 1: -(2.0**-17), 2: 2.0**-18, 3: -(2.0**-19), 4: 3 * 2.0**-20}),
        0x8010,
        {0: 0, 1: 15, 2: 4, 3: 10, 4: 5},
        8,
    ))

    # Multiply by fl32(1/d), not divide by d: max = 0xBFD51F87, x = 0xBFAD299E.
    # fl32(x * fl32(1/d)) = -6.50000048 -> + 8.5 -> 1.99999952 -> code 1, whereas
    # fl32(x / d) = -6.5 exactly would give code 2 (checked by exact_codes).
    separator = np.zeros(32, np.float32)
    separator[0] = f32_bits(0xBFD51F87)
    separator[1] = f32_bits(0xBFAD299E)
    kats.append(("reciprocal_not_division", separator, None, {0: 0, 1: 1}, 8))

    # The codes use the fp32 d, not its fp16 rounding: max = 0x3F699697,
    # x = 0x3F5AFD2E gives code 0 with id = fl32(1 / fl32(max / -8)); with the
    # fp16-rounded d the same element would get code 1.
    rounding = np.zeros(32, np.float32)
    rounding[0] = f32_bits(0x3F699697)
    rounding[1] = f32_bits(0x3F5AFD2E)
    kats.append(("fp32_scale_not_fp16", rounding, None, {0: 0, 1: 0}, 8))
    return kats


def kat_matrix() -> tuple[np.ndarray, list[tuple[str, int | None, np.ndarray]]]:
    """All KAT blocks as one [1, 32 * n] weight row plus (name, scale bits, 32 codes) per block."""
    rows, expected = [], []
    for name, values, scale_bits, codes, fill in kat_blocks():
        full = np.full(32, fill, dtype=np.int64)
        for index, code in codes.items():
            full[index] = code
        rows.append(values)
        expected.append((name, scale_bits, full))
    return np.concatenate(rows)[None, :].astype(np.float32), expected


# ----------------------------------------------------------- exact arithmetic


def _rn32(value: Fraction) -> Fraction:
    """Round an exact rational to the nearest fp32 value, ties to even (normal and subnormal range)."""
    if value == 0:
        return Fraction(0)
    sign = -1 if value < 0 else 1
    a = abs(value)
    exponent = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # Correct the float estimate of floor(log2(a)).
    while Fraction(2) ** exponent > a:
        exponent -= 1
    while Fraction(2) ** (exponent + 1) <= a:
        exponent += 1
    exponent = max(exponent, -126)
    ulp = Fraction(2) ** (exponent - 23)
    scaled = a / ulp
    low = math.floor(scaled)
    rest = scaled - low
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and low % 2 == 1):
        low += 1
    return sign * low * ulp


def exact_codes(block: np.ndarray) -> tuple[Fraction, list[int]]:
    """(d, codes) of one block by ggml's rule, each fp32 operation rounded explicitly."""
    values = [Fraction(float(v)) for v in block.astype(np.float32)]
    amax, maximum = Fraction(0), Fraction(0)
    for v in values:
        if amax < abs(v):
            amax, maximum = abs(v), v
    d = _rn32(maximum / -8)
    inverse = _rn32(1 / d) if d != 0 else Fraction(0)
    codes = []
    for v in values:
        shifted = _rn32(_rn32(v * inverse) + Fraction(17, 2))
        codes.append(min(15, math.floor(shifted)))  # shifted >= 0: (int8_t) truncation == floor
    return d, codes
