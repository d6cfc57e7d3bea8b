"""Known-answer vectors for the Q8_0 activation quantiser and the per-row int8 quantiser.

The two quantisers differ in one step, and these vectors are built around it:

* Q8_0 (reference ``examples/benchmark_llama_cpp_qpu_persistent_q4.py:42-53``),
  per 32-element block in fp32: ``d = absmax / 127``, ``inv = 1 / d`` (0 when
  d == 0), ``code = clip(rint(x * inv), -127, 127)`` -- a multiply by the
  rounded reciprocal -- with ``d`` stored as fp16 (round to nearest even);
* per-row int8 (reference ``src/qpu_xla/models/tinyllama/quantization.py:156-171``
  and ``:1085-1092``): ``s = max(absmax / 127, fl32(1 / 127))``,
  ``q = clip(rint(x / s), -127, 127)`` -- a true division.

``rint`` rounds half-way values to even in both.  Every vector holds elements
for which one plausible mistake changes a code: dividing instead of
multiplying by ``fl32(1/d)`` (or the reverse for the row quantiser), rounding
half away from zero, or quantising with the fp16-rounded ``d``.  The expected
codes are literals; the comments give the fp32 quotients they round, and
``exact_q8_0`` / ``exact_row`` re-derive them in exact rational arithmetic
with explicit round-to-fp32 steps (independent of NumPy's float32 kernels).

The separator elements share one absmax, ``M = 0x408AD652`` (4.338662):
``d = fl32(M / 127) = 0x3D0BEE2E`` (0.034162693), ``fl32(1 / d) = 0x41EA2C70``
(29.271698), fp16 ``d`` = ``0x285F`` (0.03414917).
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np

from q4_0_kats import _rn32, f32_bits

M_BITS = 0x408AD652

# Separator elements: fp32 bits -> (fl32(x * fl32(1/d)), fl32(x / d)) for the
# shared absmax M, and the code each rounding gives.
#   0x3DAEE9BA: x*inv = 2.50000024 -> 3;    x/d = 2.5 exactly -> 2 (half to even)
#   0x3E63630B: x*inv = 6.50000048 -> 7;    x/d = 6.5 exactly -> 6
#   0x3EA62AD6: x*inv = 9.5 exactly -> 10;  x/d = 9.49999905 -> 9
#   0x3F44C6F1: x*inv = 22.5000019 -> 23;   x/d = 22.5 exactly -> 22
#   0x3DAEE9B9: x*inv = x/d = 2.5 exactly -> 2 (half away from zero would give 3)
#   0x3E1D6BF4: x*inv = x/d = 4.5 exactly -> 4 (half away from zero: 5)
#   0x3C8BEE2E: x*inv = 0.5 exactly -> 0; with the fp16 d, x * fl32(1/d16) = 0.500198 -> 1
#   0x3D51E541: x*inv = 1.49999964 -> 1;   with the fp16 d, 1.5005935 -> 2
#   0x408AD652 (M itself): x*inv = 127.0000076 -> 127 (the clip to +-127 is never reached:
#   the absmax element lands within a few ulp of 127)


def _values(entries: dict[int, int], size: int = 32) -> np.ndarray:
    out = np.zeros(size, dtype=np.float32)
    for index, bits in entries.items():
        out[index] = f32_bits(bits)
    return out


# (name, 32 fp32 values, fp16 scale bits, expected codes by index (others 0))
def q8_0_kat_blocks() -> list[tuple[str, np.ndarray, int, dict[int, int]]]:
    kats = []
    separators = {0: M_BITS, 1: 0x3DAEE9BA, 2: 0x3E63630B, 3: 0x3EA62AD6, 4: 0x3F44C6F1, 5: 0x3DAEE9B9,
                  6: 0x3E1D6BF4, 7: 0x3C8BEE2E, 8: 0x3D51E541, 9: 0xBDAEE9BA, 10: 0xBEA62AD6}
    kats.append(("reciprocal_product", _values(separators), 0x285F,
                 {0: 127, 1: 3, 2: 7, 3: 10, 4: 23, 5: 2, 6: 4, 7: 0, 8: 1, 9: -3, 10: -10}))
    # The largest element is negative: d comes from |x| (a signed maximum would
    # store the negative scale 0xA85F and flip every code).
    kats.append(("largest_negative", _values({3: 0xC08AD652, 20: 0x3EA62AD6, 31: 0xBF44C6F1}), 0x285F,
                 {3: -127, 20: 10, 31: -23}))
    # All zero: d = 0 and inv = 0 (the reference's guard), every code 0 (1/0
    # would make x * inv = 0 * inf = NaN).
    kats.append(("all_zero", np.zeros(32, np.float32), 0x0000, {}))
    # absmax = 127 * 2^-17: d = 2^-17 exactly, an fp16 subnormal (0x0080),
    # inv = 2^17 and every product exact: 2^-18 -> 0.5 -> 0; 3 * 2^-18 -> 1.5 -> 2;
    # -5 * 2^-18 -> -2.5 -> -2; 100 * 2^-17 -> 100.
    tiny = np.zeros(32, np.float32)
    tiny[0] = np.float32(127 * 2.0**-17)
    tiny[1] = np.float32(2.0**-18)
    tiny[2] = np.float32(3 * 2.0**-18)
    tiny[3] = np.float32(-5 * 2.0**-18)
    tiny[4] = np.float32(100 * 2.0**-17)
    kats.append(("fp16_subnormal_scale", tiny, 0x0080, {0: 127, 1: 0, 2: 2, 3: -2, 4: 100}))
    return kats


# (name, fp32 row, floor, fp32 scale bits, expected codes by index (others 0))
def row_kats() -> list[tuple[str, np.ndarray, bool, int, dict[int, int]]]:
    kats = []
    separators = {0: M_BITS, 1: 0x3DAEE9BA, 2: 0x3E63630B, 3: 0x3EA62AD6, 4: 0x3F44C6F1, 5: 0x3DAEE9B9,
                  6: 0x3E1D6BF4, 7: 0x3C8BEE2E, 8: 0x3D51E541, 9: 0xBDAEE9BA, 10: 0xBEA62AD6}
    # s = d = 0x3D0BEE2E (above the floor); the codes round x / s, so each
    # separator gets the division's code from the table above.
    kats.append(("true_division", _values(separators, 48), True, 0x3D0BEE2E,
                 {0: 127, 1: 2, 2: 6, 3: 9, 4: 22, 5: 2, 6: 4, 7: 0, 8: 1, 9: -2, 10: -9}))
    # absmax 0.5 < 1: the floor s = fl32(1/127) = 0x3C010204 (0.007874016) is
    # active.  fl32(x / s): 0.5 -> 63.5 -> 64 (half to even); 0.25 -> 31.75 -> 32;
    # -0.0625 -> -7.9375 -> -8; 2^-8 -> 0.49609375 -> 0.  (absmax / 127 as the
    # scale would give 127, 64, -16 and 1, the next row.)
    floor_row = np.zeros(48, np.float32)
    floor_row[[0, 1, 2, 3]] = [0.5, 0.25, -0.0625, 2.0**-8]
    kats.append(("scale_floor", floor_row, True, 0x3C010204, {0: 64, 1: 32, 2: -8, 3: 0}))
    # The same row without the floor (the library's QXT_QUANT_NO_SCALE_FLOOR
    # mode): s = fl32(0.5 / 127) = 0x3B810204; 0.5 -> 127; 0.25 -> 63.5 -> 64
    # (half to even); -0.0625 -> -15.875 -> -16; 2^-8 -> 0.9921875 -> 1.
    kats.append(("no_scale_floor", floor_row, False, 0x3B810204, {0: 127, 1: 64, 2: -16, 3: 1}))
    return kats


# ----------------------------------------------------------- exact arithmetic


def rint_even(value: Fraction) -> int:
    """Round an exact rational to the nearest integer, half-way values to even."""
    low = math.floor(value)
    rest = value - low
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and low % 2 == 1):
        low += 1
    return low


def _clip127(code: int) -> int:
    return max(-127, min(127, code))


def exact_q8_0(block: np.ndarray, *, divide: bool = False, fp16_scale: bool = False,
               half_away: bool = False) -> tuple[Fraction, list[int]]:
    """(d, codes) of one Q8_0 block, every fp32 operation rounded explicitly.

    The keyword arguments switch in the plausible mistakes the known answers
    must reject: ``divide`` rounds ``x / d`` instead of ``x * fl32(1/d)``;
    ``fp16_scale`` quantises with the stored fp16 ``d``; ``half_away`` rounds
    half-way values away from zero.
    """
    values = [Fraction(float(v)) for v in block.astype(np.float32)]
    d = _rn32(max(abs(v) for v in values) / 127)
    if fp16_scale:
        d = Fraction(float(np.float16(float(d))))
    inverse = _rn32(1 / d) if d != 0 else Fraction(0)
    codes = []
    for v in values:
        quotient = (_rn32(v / d) if d != 0 else Fraction(0)) if divide else _rn32(v * inverse)
        codes.append(_clip127(_round(quotient, half_away)))
    return d, codes


def exact_row(row: np.ndarray, *, floor: bool = True, reciprocal: bool = False,
              half_away: bool = False) -> tuple[Fraction, list[int]]:
    """(s, codes) of one per-row int8 row in exact arithmetic.

    ``reciprocal`` rounds ``x * fl32(1/s)`` instead of the true quotient
    ``x / s`` (the mistake the row known answers must reject).
    """
    values = [Fraction(float(v)) for v in row.astype(np.float32)]
    s = _rn32(max(abs(v) for v in values) / 127)
    if floor:
        s = max(s, Fraction(float(np.float32(1.0 / 127.0))))
    codes = []
    for v in values:
        if s == 0:
            codes.append(0)
            continue
        quotient = _rn32(v * _rn32(1 / s)) if reciprocal else _rn32(v / s)
        codes.append(_clip127(_round(quotient, half_away)))
    return s, codes


def _round(value: Fraction, half_away: bool) -> int:
    if not half_away:
        return rint_even(value)
    magnitude = math.floor(abs(value) + Fraction(1, 2))
    return magnitude if value >= 0 else -magnitude


def expected_codes(codes: dict[int, int], size: int) -> list[int]:
    return [codes.get(i, 0) for i in range(size)]
