"""NumPy oracle for the llama.cpp bridge's approximate Q4_0 weight modes.

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py`` for who may import it.

Two modes of ``qpu_llama_q4_0_linear_prepare`` (reference
``integrations/llama_cpp/src/qpu_llama_q4_0.c:205-460``) replace the Q4_0
block scales of a linear with more than four rows by one fp32 scale per
output column, re-quantising the weights to int8 at prepare time:

* ``COLUMN_W8``: int8 weights [N, K] with column scales; the activation
  stays Q8_0 (int8 values + an fp16 scale per block).  Per block an exact
  int32 dot, ``acc = fl32(acc + fl32(float(dot) * da_b))`` in block order,
  then ``y = fl32(acc * cs[n])`` (the ``column_weight_scale`` variant of the
  tiled program, ``src/qpu_xla/kernels/ggml_q4_0.py:377-525``, restated on the
  CPU by ``qpu_llama_q4_0.c:862-911``).
* ``ROWCOL_W8A8``: the activation row is re-quantised to int8 with one fp32
  row scale as well; one int32 dot over the whole row, then
  ``y = fl32(fl32(float(dot) * rs[m]) * cs[n])`` (the tiled W8A8 GEMM with
  fused scaling, ``qpu_llama_q4_0.c:879-906``).

Both re-quantisers share one rounding rule (``qpu_llama_q4_0.c:352-380`` and
``:548-568``): ``scale = max|v| / 127`` in fp32 (0 when the maximum is 0),
``s = fl32(v / scale)``, ``q = trunc(fl32(s + 0.5))`` for ``s >= 0`` else
``trunc(fl32(s - 0.5))``, clamped to [-127, 127].  The fp32 addition of 0.5
is part of the rule: ``s = 0.49999997`` gives 1, not 0.
"""

from __future__ import annotations

import numpy as np

from oracle.ggml import QK, unpack_q4_0_blocks, unpack_q8_0_blocks
from oracle.w8a8 import dequantize_epilogue, int8_gemm_i32

_HALF = np.float32(0.5)


def round_half_away_w8(scaled: np.ndarray) -> np.ndarray:
    """``(long)(s >= 0 ? s + 0.5f : s - 0.5f)`` clamped to [-127, 127] (``qpu_llama_q4_0.c:377-380``)."""
    scaled = np.asarray(scaled, dtype=np.float32)
    shifted = np.where(scaled >= 0, scaled + _HALF, scaled - _HALF).astype(np.float32)
    return np.clip(np.trunc(shifted), -127, 127).astype(np.int8)


def _requantize(values: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Rows of exact fp32 values [R, K] -> (int8 [R, K], fp32 scales [R])."""
    maximum = np.abs(values).max(axis=1).astype(np.float32)
    scales = np.where(maximum > 0, maximum / np.float32(127.0), np.float32(0.0)).astype(np.float32)
    safe = np.where(scales > 0, scales, np.float32(1.0)).astype(np.float32)
    scaled = (values / safe[:, None]).astype(np.float32)
    scaled = np.where(scales[:, None] > 0, scaled, np.float32(0.0)).astype(np.float32)
    return round_half_away_w8(scaled), scales


def requantize_q4_0_columns_w8(weight_blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Q4_0 weights [N, B, 18] -> (int8 [N, K], fp32 column scales [N]).

    Follows ``qpu_llama_q4_0.c:332-386``: ``v = fl32((code - 8) * d_b)`` (exact:
    a 4-bit integer times an fp16 value), column scale ``max|v| / 127``, then
    the shared rounding rule.  The device keeps the codes as uint32 words of
    four consecutive k (``qword = block * 8 + index / 4``), i.e.
    ``oracle.pack_int8_quads(wq).T``.
    """
    scales, values = unpack_q4_0_blocks(weight_blocks)
    n, blocks = scales.shape
    exact = (values.astype(np.float32) * scales[:, :, None]).astype(np.float32).reshape(n, blocks * QK)
    return _requantize(exact)


def requantize_q8_0_rows_w8(activation_blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Q8_0 activations [M, B, 34] -> (int8 [M, K], fp32 row scales [M]).

    Follows ``qpu_llama_q4_0.c:526-571``: ``v = fl32(q * d_b)`` (exact: an 8-bit
    integer times an fp16 value), row scale ``max|v| / 127``, then the shared
    rounding rule.
    """
    scales, values = unpack_q8_0_blocks(activation_blocks)
    m, blocks = scales.shape
    exact = (values.astype(np.float32) * scales[:, :, None]).astype(np.float32).reshape(m, blocks * QK)
    return _requantize(exact)


def column_w8_reference(activation_blocks: np.ndarray, weight_q: np.ndarray,
                        column_scales: np.ndarray) -> np.ndarray:
    """COLUMN_W8 linear: ``y[m, n] = fl32(sum_b fl32(float(dot_b) * da[m, b]) * cs[n])``.

    ``dot_b`` is the exact int32 dot of the Q8_0 block with the int8 weights
    of that block; the sum runs in block order in fp32
    (``ggml_q4_0.py:497-525``, ``qpu_llama_q4_0.c:862-911``).
    """
    da, aq = unpack_q8_0_blocks(activation_blocks)
    m, blocks = da.shape
    wq = np.asarray(weight_q, dtype=np.int8)
    n = wq.shape[0]
    if wq.shape != (n, blocks * QK):
        raise ValueError("weight codes must be int8 [N, blocks * 32]")
    w = wq.reshape(n, blocks, QK).astype(np.int32)
    a = aq.astype(np.int32)
    acc = np.zeros((m, n), dtype=np.float32)
    for b in range(blocks):
        dots = a[:, b] @ w[:, b].T
        acc = (acc + (dots.astype(np.float32) * da[:, b, None]).astype(np.float32)).astype(np.float32)
    return (acc * np.asarray(column_scales, dtype=np.float32)[None, :]).astype(np.float32)


def rowcol_w8a8_reference(activation_q: np.ndarray, row_scales: np.ndarray, weight_q: np.ndarray,
                          column_scales: np.ndarray) -> np.ndarray:
    """ROWCOL_W8A8 linear: ``y = fl32(fl32(float(sum_k a * w) * rs[m]) * cs[n])`` (``qpu_llama_q4_0.c:879-906``)."""
    acc = int8_gemm_i32(np.asarray(activation_q, dtype=np.int8), np.asarray(weight_q, dtype=np.int8))
    return dequantize_epilogue(acc, np.asarray(row_scales, dtype=np.float32),
                               np.asarray(column_scales, dtype=np.float32), None)
