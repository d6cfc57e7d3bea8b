"""M = 1 packed W8A8 GEMV to int32.

Contract of the reference's ``src/qpu_xla/kernels/gemv_int8.py:93-153``:
args ``(source, weight, destination)`` with source words [1, K/4], weight
``pack_int8_quads(W).T`` words [K/4, N], destination int32 [1, N], grid
``(N // 16, 1, 1)``.  On gfx950 the same MFMA GEMM runs it with M = 1.
"""

from __future__ import annotations

from typing import Any

import torch

from qpu_xla_amd import _lib
from qpu_xla_amd._tensors import PACKED_WORD_DTYPES, ptr, row_stride, rows_are_dense, stream_handle
from qpu_xla_amd.errors import KernelError
from qpu_xla_amd.kernel import Kernel


def supports_w8a8_gemv(source: torch.Tensor, weight: torch.Tensor, destination: torch.Tensor) -> bool:
    tensors = (source, weight, destination)
    if not all(isinstance(t, torch.Tensor) and t.dim() == 2 for t in tensors):
        return False
    if source.dtype not in PACKED_WORD_DTYPES or weight.dtype not in PACKED_WORD_DTYPES:
        return False
    if destination.dtype != torch.int32 or source.shape[0] != 1 or destination.shape[0] != 1:
        return False
    q_words = source.shape[1]
    if weight.shape[0] != q_words or destination.shape[1] != weight.shape[1] or weight.shape[1] % 16 or q_words % 4:
        return False
    if any(t.device.type != "cuda" for t in tensors) or len({t.device for t in tensors}) != 1:
        return False
    return all(rows_are_dense(t) for t in tensors)


def _execute_w8a8_gemv(stream: Any, args: tuple[Any, ...], grid: tuple[int, int, int]) -> None:
    if len(args) != 3 or not all(isinstance(a, torch.Tensor) for a in args):
        raise KernelError("packed W8A8 GEMV expects (source, weight, destination)")
    source, weight, destination = args
    if not supports_w8a8_gemv(source, weight, destination):
        raise KernelError("packed W8A8 GEMV requires one packed source row and 16-aligned output columns")
    want = (weight.shape[1] // 16, 1, 1)
    if tuple(grid) != want:
        raise KernelError(f"packed W8A8 GEMV grid must be {want}, got {tuple(grid)}")
    if source.shape[1] * 4 * 127 * 127 > 2**31 - 1:
        raise ValueError("packed W8A8 GEMV accumulation can overflow int32")
    _lib.call(
        "qxt_w8a8_gemm_i32",
        ptr(source), row_stride(source), ptr(weight), row_stride(weight), ptr(destination), row_stride(destination),
        1, weight.shape[1], source.shape[1] * 4, _lib.WEIGHT_K4N, stream_handle(stream),
    )


W8A8_GEMV_KERNEL = Kernel("gfx950.w8a8_gemv", _execute_w8a8_gemv)
