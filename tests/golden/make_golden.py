"""Regenerate the golden fixtures under ``tests/golden/``.

Two kinds of fixtures:

* ``kat_*.npz`` -- closed-form known-answer tests restated from the
  reference's native smokes.  Inputs are the smokes' formulas; expected
  values are computed here with plain Python integers (exact), independently
  of the oracle:
    - ``qpu_llama_q4_0_smoke.c:15-36``    M=1, K=32, N=32, scales 1.0
    - ``qpu_llama_q4_0_m4_smoke.c:17-40`` M=4, K=32, N=32, scales 1.0
    - ``qpu_llama_q4_0_mx_smoke.c:50-88`` M=5, K=64, N=32, scales 1.0 / 0.5
    - ``qpu_llama_w8a8_smoke.c:58-66``    K=16, N=16, a_r = r-8, w_rc = ((3r+5c)%15)-7
  plus the codec extremes of ``tests/test_qpu_xla_ggml_q4_0.py:25-44``.
* ``oracle_*.npz`` -- seeded inputs (the reference tests' seeds and shapes)
  with expected outputs from the NumPy oracle, used as regression vectors.

Run: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import sys
from fractions import Fraction
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402

ONE_FP16 = 0x3C00
HALF_FP16 = 0x3800


def _le16(value: int) -> list[int]:
    return [value & 0xFF, value >> 8]


def kat_q4_0_m1() -> dict[str, np.ndarray]:
    inputs, outputs = 32, 32
    activation = _le16(ONE_FP16) + [(i - 16) & 0xFF for i in range(inputs)]
    weights, expected = [], []
    for column in range(outputs):
        row = _le16(ONE_FP16)
        acc = 0
        for index in range(inputs // 2):
            low = (index + column) % 16
            high = (index * 3 + column) % 16
            row.append(low | (high << 4))
            acc += (low - 8) * (index - 16)
            acc += (high - 8) * (index + 16 - 16)
        weights.append(row)
        expected.append(acc)
    return {
        "activation": np.array(activation, dtype=np.uint8).reshape(1, 1, 34),
        "weight": np.array(weights, dtype=np.uint8).reshape(outputs, 1, 18),
        "expected": np.array(expected, dtype=np.float32).reshape(1, outputs),
        "resident_start": np.int64(16),
        "resident_count": np.int64(16),
    }


def kat_q4_0_m4() -> dict[str, np.ndarray]:
    inputs, outputs, rows = 32, 32, 4
    act = [[*_le16(ONE_FP16), *[(i - 12 - r) & 0xFF for i in range(inputs)]] for r in range(rows)]
    weights = []
    expected = [[0] * outputs for _ in range(rows)]
    for column in range(outputs):
        wrow = _le16(ONE_FP16)
        for index in range(inputs // 2):
            low = (index + column) % 16
            high = (index * 3 + column) % 16
            wrow.append(low | (high << 4))
            for r in range(rows):
                expected[r][column] += (low - 8) * (index - 12 - r)
                expected[r][column] += (high - 8) * (index + 16 - 12 - r)
        weights.append(wrow)
    return {
        "activation": np.array(act, dtype=np.uint8).reshape(rows, 1, 34),
        "weight": np.array(weights, dtype=np.uint8).reshape(outputs, 1, 18),
        "expected": np.array(expected, dtype=np.float32),
        "resident_start": np.int64(16),
        "resident_count": np.int64(16),
    }


def kat_q4_0_mx() -> dict[str, np.ndarray]:
    blocks, outputs, rows = 2, 32, 5
    act = np.zeros((rows, blocks, 34), dtype=np.uint8)
    a_val = {}
    for r in range(rows):
        for b in range(blocks):
            scale = ONE_FP16 if (r + b) % 2 == 0 else HALF_FP16
            act[r, b, 0:2] = _le16(scale)
            for i in range(32):
                v = i - 12 - r + b * 3
                a_val[(r, b, i)] = v
                act[r, b, 2 + i] = v & 0xFF
    weight = np.zeros((outputs, blocks, 18), dtype=np.uint8)
    expected = [[Fraction(0)] * outputs for _ in range(rows)]
    for c in range(outputs):
        for b in range(blocks):
            scale = ONE_FP16 if (c + b) % 2 == 0 else HALF_FP16
            weight[c, b, 0:2] = _le16(scale)
            for i in range(16):
                low = (i + c + b) % 16
                high = (i * 3 + c + b * 2) % 16
                weight[c, b, 2 + i] = low | (high << 4)
                for r in range(rows):
                    cs = Fraction(1 if (r + b) % 2 == 0 else 1, 1 if (r + b) % 2 == 0 else 2)
                    cs *= Fraction(1, 1 if (c + b) % 2 == 0 else 2)
                    expected[r][c] += cs * ((low - 8) * a_val[(r, b, i)] + (high - 8) * a_val[(r, b, 16 + i)])
    return {
        "activation": act,
        "weight": weight,
        "expected": np.array([[float(v) for v in row] for row in expected], dtype=np.float32),
        "resident_start": np.int64(16),
        "resident_count": np.int64(16),
    }


def kat_w8a8() -> dict[str, np.ndarray]:
    reduction, outputs = 16, 16
    a = [r - 8 for r in range(reduction)]
    w = [[((3 * r + 5 * c) % 15) - 7 for c in range(outputs)] for r in range(reduction)]  # [K][N]
    expected = [sum(a[r] * w[r][c] for r in range(reduction)) for c in range(outputs)]
    return {
        "activation": np.array(a, dtype=np.int8).reshape(1, reduction),
        "weight_kn": np.array(w, dtype=np.int8),
        "expected": np.array(expected, dtype=np.int32).reshape(1, outputs),
    }


def codec_extremes() -> dict[str, np.ndarray]:
    q4_scales = np.array([0.0, -0.5, np.float16(2**-14)], dtype=np.float16)
    q4_codes = np.stack(
        (np.zeros(32, np.uint8), np.full(32, 15, np.uint8), np.arange(32, dtype=np.uint8) % 16)
    )
    q8_scales = np.array([0.0, 0.125], dtype=np.float16)
    q8_values = np.stack((np.full(32, -128, np.int16), np.full(32, 127, np.int16)))
    return {"q4_scales": q4_scales, "q4_codes": q4_codes, "q8_scales": q8_scales, "q8_values": q8_values}


def oracle_q4_0_linear() -> dict[str, np.ndarray]:
    # Seed and shape of tests/test_qpu_xla_ggml_q4_0.py:47-80 (rows=4 -> seed 4404).
    rows, blocks, outputs = 4, 5, 32
    rng = np.random.default_rng(4400 + rows)
    a_scales = rng.uniform(0.0001, 0.2, size=(rows, blocks)).astype(np.float32)
    a_values = rng.integers(-128, 128, size=(rows, blocks, 32), dtype=np.int16)
    w_scales = rng.uniform(-0.2, 0.2, size=(outputs, blocks)).astype(np.float16)
    w_codes = rng.integers(0, 16, size=(outputs, blocks, 32), dtype=np.uint8)
    act = oracle.pack_q8_0_blocks(a_scales, a_values)
    wt = oracle.pack_q4_0_blocks(w_scales, w_codes)
    return {
        "activation": act,
        "weight": wt,
        "expected": oracle.q4_0_q8_0_reference(act, wt),
        "dots": oracle.q4_0_q8_0_block_dots(act, wt),
    }


def oracle_w8a8_fused() -> dict[str, np.ndarray]:
    # Seed and shape of tests/test_qpu_xla_gemm_int8.py:57-92.
    p, q, r = 32, 64, 48
    rng = np.random.default_rng(1765)
    left = rng.integers(-127, 128, size=(p, q), dtype=np.int8)
    right = rng.integers(-127, 128, size=(q, r), dtype=np.int8)
    sa = rng.uniform(0.001, 0.1, size=p).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, size=r).astype(np.float32)
    acc = oracle.int8_gemm_i32(left, np.ascontiguousarray(right.T))
    return {
        "left": left,
        "right": right,
        "row_scales": sa,
        "column_scales": sw,
        "acc": acc,
        "expected": oracle.dequantize_epilogue(acc, sa, sw),
    }


def oracle_quantizers() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(2024)
    x = rng.standard_normal((3, 256), dtype=np.float32)
    x[1, 32:64] = 0.0  # an all-zero Q8_0 block (d = 0, inv = 0)
    x[2] *= np.float32(1e-4)  # tiny row: per-row scale floor is active
    w = (rng.standard_normal((4, 128), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    q8 = oracle.quantize_q8_0_blocks(x)
    qa, sa = oracle.quantize_rows_int8(x)
    q4 = oracle.quantize_q4_0_blocks(w)
    return {"x": x, "q8_0_blocks": q8, "rows_q": qa, "rows_scale": sa, "w": w, "q4_0_blocks": q4}


FIXTURES = {
    "kat_q4_0_m1": kat_q4_0_m1,
    "kat_q4_0_m4": kat_q4_0_m4,
    "kat_q4_0_mx": kat_q4_0_mx,
    "kat_w8a8": kat_w8a8,
    "codec_extremes": codec_extremes,
    "oracle_q4_0_linear_seed4404": oracle_q4_0_linear,
    "oracle_w8a8_fused_seed1765": oracle_w8a8_fused,
    "oracle_quantizers_seed2024": oracle_quantizers,
}


def main() -> None:
    for name, make in FIXTURES.items():
        np.savez(HERE / f"{name}.npz", **make())
        print(f"wrote tests/golden/{name}.npz")


if __name__ == "__main__":
    main()
