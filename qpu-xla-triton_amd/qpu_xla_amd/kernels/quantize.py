"""GPU quantisers: Q8_0 activations, per-row int8 activations, Q4_0 weights.

* ``quantize_q8_0`` -- arithmetic of the reference's own quantiser
  ``quantize_q8_0_split`` (examples/benchmark_llama_cpp_qpu_persistent_q4.py:42-53),
  emitting native 34-byte blocks (src/qpu_xla/kernels/ggml_q4_0.py:43-55).
* ``quantize_rows_int8`` -- ``PreparedW8A8Linear._prepare_values``
  (src/qpu_xla/models/tinyllama/quantization.py:156-171), including the
  fl32(1/127) scale floor; ``floor=False`` is a labelled non-reference mode.
* ``quantize_q4_0`` -- ggml's reference Q4_0 rule for weight preparation
  (called by the reference at integrations/llama_cpp/tests/qpu_ggml_backend_smoke.cpp:119).
"""

from __future__ import annotations

from typing import Any

import torch

from qpu_xla_amd import _lib
from qpu_xla_amd._tensors import ptr, require_gpu, row_stride, rows_are_dense, stream_handle

QK = 32
Q4_0_BLOCK_BYTES = 18
Q8_0_BLOCK_BYTES = 34


def _check_f32_rows(name: str, x: torch.Tensor) -> None:
    if x.dtype != torch.float32 or x.dim() != 2 or not rows_are_dense(x):
        raise ValueError(f"{name}: expects a rank-2 float32 tensor with contiguous rows")


def quantize_q8_0(x: torch.Tensor, out: torch.Tensor | None = None, *, stream: Any = None) -> torch.Tensor:
    """fp32 [M, K] -> native Q8_0 blocks uint8 [M, K/32, 34]."""
    _check_f32_rows("quantize_q8_0", x)
    rows, columns = x.shape
    if columns % QK:
        raise ValueError("quantize_q8_0: K must be a multiple of 32")
    if out is None:
        out = torch.empty((rows, columns // QK, Q8_0_BLOCK_BYTES), dtype=torch.uint8, device=x.device)
    elif out.dtype != torch.uint8 or tuple(out.shape) != (rows, columns // QK, Q8_0_BLOCK_BYTES) or not out[0].is_contiguous():
        raise ValueError("quantize_q8_0: out must be uint8 [M, K/32, 34] with contiguous rows")
    require_gpu("quantize_q8_0", x, out)
    _lib.call("qxt_quantize_q8_0", ptr(x), row_stride(x), ptr(out), row_stride(out), rows, columns, stream_handle(stream))
    return out


def quantize_rows_int8(
    x: torch.Tensor,
    *,
    floor: bool = True,
    padded_columns: int | None = None,
    out: torch.Tensor | None = None,
    scales: torch.Tensor | None = None,
    stream: Any = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 [M, K] -> (int8 [M, padded_columns], fp32 scales [M]); padding columns are 0."""
    _check_f32_rows("quantize_rows_int8", x)
    rows, columns = x.shape
    padded = columns if padded_columns is None else int(padded_columns)
    if padded < columns:
        raise ValueError("quantize_rows_int8: padded_columns < K")
    if out is None:
        out = torch.empty((rows, padded), dtype=torch.int8, device=x.device)
    if scales is None:
        scales = torch.empty((rows,), dtype=torch.float32, device=x.device)
    if out.dtype != torch.int8 or out.dim() != 2 or out.shape[0] < rows or out.shape[1] < padded or not rows_are_dense(out):
        raise ValueError("quantize_rows_int8: out must be int8 [>= M, >= padded_columns] with contiguous rows")
    if scales.dtype != torch.float32 or scales.dim() != 1 or scales.shape[0] < rows or not scales.is_contiguous():
        raise ValueError("quantize_rows_int8: scales must be contiguous float32 [>= M]")
    require_gpu("quantize_rows_int8", x, out, scales)
    flags = 0 if floor else _lib.QUANT_NO_SCALE_FLOOR
    _lib.call(
        "qxt_quantize_rows_int8",
        ptr(x), row_stride(x), ptr(out), row_stride(out), ptr(scales),
        rows, columns, padded, flags, stream_handle(stream),
    )
    return out, scales


def quantize_q4_0(w: torch.Tensor, out: torch.Tensor | None = None, *, stream: Any = None) -> torch.Tensor:
    """fp32 [N, K] -> native Q4_0 blocks uint8 [N, K/32, 18]."""
    _check_f32_rows("quantize_q4_0", w)
    rows, columns = w.shape
    if columns % QK:
        raise ValueError("quantize_q4_0: K must be a multiple of 32")
    if out is None:
        out = torch.empty((rows, columns // QK, Q4_0_BLOCK_BYTES), dtype=torch.uint8, device=w.device)
    elif out.dtype != torch.uint8 or tuple(out.shape) != (rows, columns // QK, Q4_0_BLOCK_BYTES) or not out[0].is_contiguous():
        raise ValueError("quantize_q4_0: out must be uint8 [N, K/32, 18] with contiguous rows")
    require_gpu("quantize_q4_0", w, out)
    _lib.call("qxt_quantize_q4_0", ptr(w), row_stride(w), ptr(out), row_stride(out), rows, columns, stream_handle(stream))
    return out
