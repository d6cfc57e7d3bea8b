"""Standalone int32 -> fp32 W8A8 epilogue.

Contract of the reference's ``src/qpu_xla/kernels/w8a8_epilogue.py:108-174``:
args ``(source, row_scales, column_scales, destination[, bias])``, source
int32 [M, N], grid ``(N // 16, M // 16, 1)``, result
``fl32(fl32(float(acc) * sa[m]) * sw[n])`` (+ ``bias[n]`` as a separate add).
"""

from __future__ import annotations

from typing import Any

import torch

from qpu_xla_amd import _lib
from qpu_xla_amd._tensors import ptr, row_stride, rows_are_dense, stream_handle
from qpu_xla_amd.errors import KernelError
from qpu_xla_amd.kernel import Kernel


def supports_w8a8_dequantize(
    source: torch.Tensor,
    row_scales: torch.Tensor,
    column_scales: torch.Tensor,
    destination: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> bool:
    floats = [row_scales, column_scales, destination] + ([bias] if bias is not None else [])
    tensors = [source, *floats]
    if not all(isinstance(t, torch.Tensor) for t in tensors):
        return False
    if source.dtype != torch.int32 or any(t.dtype != torch.float32 for t in floats):
        return False
    if source.dim() != 2 or tuple(destination.shape) != tuple(source.shape):
        return False
    rows, columns = source.shape
    if rows % 16 or columns % 16 or tuple(row_scales.shape) != (rows,) or tuple(column_scales.shape) != (columns,):
        return False
    if bias is not None and tuple(bias.shape) != (columns,):
        return False
    if any(t.device.type != "cuda" for t in tensors) or len({t.device for t in tensors}) != 1:
        return False
    return all(t.is_contiguous() for t in tensors)


def _execute_w8a8_dequantize(stream: Any, args: tuple[Any, ...], grid: tuple[int, int, int]) -> None:
    if len(args) not in (4, 5) or not all(isinstance(a, torch.Tensor) for a in args):
        raise KernelError("W8A8 dequantization expects (source, row_scales, column_scales, destination[, bias])")
    source, row_scales, column_scales, destination = args[:4]
    bias = args[4] if len(args) == 5 else None
    if not supports_w8a8_dequantize(source, row_scales, column_scales, destination, bias):
        raise KernelError("W8A8 dequantization requires contiguous 16x16-aligned INT32-to-FP32 tensors")
    want = (source.shape[1] // 16, source.shape[0] // 16, 1)
    if tuple(grid) != want:
        raise KernelError(f"W8A8 dequantization grid must be {want}, got {tuple(grid)}")
    _lib.call(
        "qxt_w8a8_dequantize",
        ptr(source), row_stride(source), ptr(row_scales), ptr(column_scales), ptr(bias),
        ptr(destination), row_stride(destination), source.shape[0], source.shape[1], stream_handle(stream),
    )


W8A8_DEQUANTIZE_KERNEL = Kernel("gfx950.w8a8_dequantize", _execute_w8a8_dequantize)


def w8a8_dequantize(
    acc: torch.Tensor,
    row_scales: torch.Tensor,
    column_scales: torch.Tensor,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    *,
    stream: Any = None,
) -> torch.Tensor:
    """Functional form for any shape (no 16-alignment)."""
    if acc.dtype != torch.int32 or acc.dim() != 2 or not rows_are_dense(acc):
        raise ValueError("w8a8_dequantize: int32 [M, N] with contiguous rows required")
    m, n = acc.shape
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=acc.device)
    _lib.call(
        "qxt_w8a8_dequantize",
        ptr(acc), row_stride(acc), ptr(row_scales), ptr(column_scales), ptr(bias), ptr(out), row_stride(out),
        m, n, stream_handle(stream),
    )
    return out
