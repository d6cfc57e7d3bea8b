"""The row quantisers' division by a row scale, restated in exact rational arithmetic.

The GPU kernels compute x / s for a whole row as q0 = fl(x r), e = fma(-q0, s, x),
fl(e r + q0) with r = fl(1 / s) (``quant_recip`` in ``csrc/qxt_common.h``).  This
checks, with every fp32 rounding made explicit on exact rationals, that the
sequence equals IEEE division at the inputs where a mistake would show: quotients
at and beside the half-integers where ``rint`` changes, scales with all-ones and
power-of-two significands, and scales down to the sequence's lower limit 2^-70.
The GPU tests compare the kernels themselves with the NumPy oracle.
"""

from __future__ import annotations

import random
from fractions import Fraction

from q4_0_kats import _rn32

SCALE_MIN_EXPONENT = -70  # kRecipScaleMin = 2^-70


def _recip_quotient(x: Fraction, s: Fraction) -> Fraction:
    r = _rn32(Fraction(1) / s)
    q0 = _rn32(x * r)
    e = _rn32(x - q0 * s)  # fma: one rounding of the exact value
    return _rn32(e * r + q0)


def _ulp(x: Fraction) -> Fraction:
    a = abs(x)
    e = -126
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    return Fraction(2) ** (e - 23)


def test_reciprocal_quotient_equals_ieee_division_at_rounding_ties() -> None:
    rng = random.Random(20)
    for case in range(3000):
        kind = case % 10
        sig = (1 << 24) - 1 if kind == 0 else (1 << 23) if kind == 1 else rng.randrange(1 << 23, 1 << 24)
        s = Fraction(sig) * Fraction(2) ** (rng.randrange(SCALE_MIN_EXPONENT, 20) - 23)
        if rng.random() < 0.8:
            x = _rn32((Fraction(rng.randrange(-128, 128)) + Fraction(1, 2)) * s)
            x = _rn32(x + rng.randrange(-3, 4) * _ulp(x)) if x != 0 else x
        else:
            x = _rn32(Fraction(rng.uniform(-127.5, 127.5)) * s)
        assert _recip_quotient(x, s) == _rn32(x / s), (float(x), float(s))


def test_a_plain_reciprocal_product_is_not_ieee_division() -> None:
    # The correction step matters: fl(x * fl(1/s)) alone differs somewhere here.
    rng = random.Random(21)
    differs = False
    for _ in range(3000):
        s = Fraction(rng.randrange(1 << 23, 1 << 24)) * Fraction(2) ** -30
        x = _rn32((Fraction(rng.randrange(-128, 128)) + Fraction(1, 2)) * s)
        differs |= _rn32(x * _rn32(Fraction(1) / s)) != _rn32(x / s)
    assert differs
