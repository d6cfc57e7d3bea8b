"""NumPy oracle for the dynamic W8A8 int8 linear.

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py`` for who may import it.

Contract (reference ``src/qpu_xla/models/tinyllama/quantization.py``):

* quantiser, for weights (per output channel) and activations (per row):
  ``scale = max(fl32(absmax / 127), fl32(1 / 127))``;
  ``q = clip(rint(fl32(x / scale)), -127, 127)`` (true division, half-even);
* int32 accumulation of int8 x int8 products;
* epilogue ``y = fl32(fl32(float(acc) * sa[m]) * sw[n])`` followed by a
  separate fp32 ``y + bias[n]``.
"""

from __future__ import annotations

import numpy as np

SCALE_FLOOR = np.float32(1.0 / 127.0)
INT32_MAX = np.iinfo(np.int32).max


def _quantize_rows(values: np.ndarray, floor: bool) -> tuple[np.ndarray, np.ndarray]:
    row_max = np.max(np.abs(values), axis=1)
    scales = (row_max / np.float32(127.0)).astype(np.float32)
    if floor:
        scales = np.maximum(scales, SCALE_FLOOR).astype(np.float32)
    safe = np.where(scales > 0, scales, np.float32(1.0)).astype(np.float32)
    q = np.rint(values / safe[:, None]).clip(-127, 127).astype(np.int8)
    q[scales == 0] = 0
    return np.ascontiguousarray(q), np.ascontiguousarray(scales)


def quantize_rows_int8(values: np.ndarray, *, floor: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """Per-row dynamic activation quantisation -> (int8 [M, K], fp32 scales [M]).

    Follows ``_prepare_values`` (``quantization.py:156-171``), the CPU oracle
    ``cpu_reference`` (``quantization.py:1065-1072``) and
    ``_dynamic_int8_reference`` (``tests/test_qpu_xla_quantization.py:50-54``).
    ``floor=False`` drops the 1/127 floor; that mode is NOT the reference's
    contract (a zero row then gets scale 0 and codes 0).
    """
    values = np.asarray(values, dtype=np.float32)
    if values.ndim != 2:
        raise ValueError("per-row quantisation needs a rank-2 float32 matrix")
    return _quantize_rows(values, floor)


def quantize_per_output_channel_int8(weight: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel weight quantisation -> (int8 [N, K], fp32 scales [N]).

    Follows ``quantize_per_output_channel_int8`` (``quantization.py:1085-1092``).
    """
    weight = np.asarray(weight)
    if weight.ndim != 2 or weight.dtype != np.float32:
        raise ValueError("per-channel quantisation needs a rank-2 float32 matrix")
    return _quantize_rows(weight, True)


def pack_int8_quads(values: np.ndarray) -> np.ndarray:
    """Pack four adjacent int8 along the last axis into little-endian uint32.

    Follows ``src/qpu_xla/kernels/gemm_int8.py:23-29``.
    """
    values = np.asarray(values)
    if values.ndim != 2 or values.dtype != np.int8 or values.shape[1] % 4:
        raise ValueError("packing needs rank-2 int8 whose last extent is a multiple of 4")
    u = values.view(np.uint8).astype(np.uint32)
    return np.ascontiguousarray(u[:, 0::4] | (u[:, 1::4] << 8) | (u[:, 2::4] << 16) | (u[:, 3::4] << 24))


def pack_int8_gemm_operands(left: np.ndarray, right: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Logical (P, Q) @ (Q, R) -> (left u32 [P, Q/4], right u32 [Q/4, R]).

    Follows ``src/qpu_xla/kernels/gemm_int8.py:32-40``.
    """
    if left.ndim != 2 or right.ndim != 2 or left.dtype != np.int8 or right.dtype != np.int8:
        raise ValueError("W8A8 operands must be rank-2 int8")
    if left.shape[1] != right.shape[0] or left.shape[1] % 4:
        raise ValueError("reduction extents must match and be a multiple of 4")
    return pack_int8_quads(left), np.ascontiguousarray(pack_int8_quads(np.ascontiguousarray(right.T)).T)


def check_accumulation_range(reduction: int) -> None:
    """Overflow guard ``K * 127 * 127 <= INT32_MAX`` (``gemm_int8.py:296-298``)."""
    if reduction * 127 * 127 > INT32_MAX:
        raise ValueError("W8A8 accumulation can overflow int32")


def int8_gemm_i32(qa: np.ndarray, qw: np.ndarray) -> np.ndarray:
    """Exact int32 ``acc[m, n] = sum_k qa[m, k] * qw[n, k]`` for int8 qa [M, K], qw [N, K].

    The reference computes ``q_a @ q_w.T`` in int32 (``quantization.py:1073``).
    Here small problems use int64 matmul; large ones use float64 BLAS, which is
    exact because every partial sum is an integer of magnitude at most
    ``K * 128 * 128 < 2**53`` (K <= 2**38).
    """
    if qa.dtype != np.int8 or qw.dtype != np.int8 or qa.ndim != 2 or qw.ndim != 2:
        raise ValueError("int8_gemm_i32 needs rank-2 int8 operands")
    if qa.shape[1] != qw.shape[1]:
        raise ValueError("reduction extents differ")
    check_accumulation_range(qa.shape[1])
    m, k = qa.shape
    n = qw.shape[0]
    if m * n * k <= (1 << 24):
        return (qa.astype(np.int64) @ qw.astype(np.int64).T).astype(np.int32)
    return (qa.astype(np.float64) @ qw.astype(np.float64).T).astype(np.int32)


def dequantize_epilogue(
    acc: np.ndarray, row_scales: np.ndarray, column_scales: np.ndarray, bias: np.ndarray | None = None
) -> np.ndarray:
    """``y = fl32(fl32(float(acc) * sa[m]) * sw[n])``, then ``y += bias[n]`` as a separate add.

    Follows ``quantization.py:1073-1075`` (and the fused QPU store order at
    ``src/qpu_xla/kernels/gemm_int8.py:176-178``); bias as a separate fp32
    add per ``models/smolvla/accelerated.py:259-261``.
    """
    y = acc.astype(np.float32) * row_scales.astype(np.float32)[:, None]
    y *= column_scales.astype(np.float32)[None, :]
    if bias is not None:
        y += bias.astype(np.float32)[None, :]
    return np.ascontiguousarray(y, dtype=np.float32)


def w8a8_linear_reference(
    values: np.ndarray,
    weight_codes: np.ndarray,
    weight_scales: np.ndarray,
    bias: np.ndarray | None = None,
    *,
    floor: bool = True,
) -> np.ndarray:
    """Whole dynamic W8A8 linear: row quantise, int32 GEMM, dequant, bias.

    Follows ``_StagedW8A8Linear._cpu`` (``models/smolvla/accelerated.py:248-262``).
    """
    qa, sa = quantize_rows_int8(values, floor=floor)
    acc = int8_gemm_i32(qa, weight_codes)
    return dequantize_epilogue(acc, sa, weight_scales, bias)
