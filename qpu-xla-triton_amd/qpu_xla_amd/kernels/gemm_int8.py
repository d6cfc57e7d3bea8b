"""Dynamic-W8A8 int8 GEMM on gfx950 (MFMA, exact int32 accumulation).

Kernel-level contract of the reference's ``src/qpu_xla/kernels/gemm_int8.py``:

* ``TILED_W8A8_GEMM_KERNEL`` -- args ``(left, right, destination)``: left
  packed-K4 words [P, Q/4] (byte-identical to int8 [P, Q]), right
  ``pack_int8_quads(W).T`` words [Q/4, R], destination int32 [P, R];
  grid ``(R // 16, P // 16, 1)``; P, R multiples of 16, Q of 16.
* ``TILED_W8A8_GEMM_DEQUANTIZE_KERNEL`` -- args ``(left, right, row_scales,
  column_scales, destination[, bias])`` writing
  ``fl32(fl32(float(acc) * sa[p]) * sw[r])`` (``gemm_int8.py:176-178``), plus
  ``+ bias[r]`` as a separate add when the optional sixth argument is given.

Packed words may be ``torch.int32`` or ``torch.uint32`` tensors.  The
functional helpers take the natural layouts instead: activations int8
[M, K] and weights int8 [N, K] (``QuantizedMatrixInt8.values``), which is the
layout the MFMA kernel reads best.
"""

from __future__ import annotations

from typing import Any

import torch

from qpu_xla_amd import _lib
from qpu_xla_amd._tensors import PACKED_WORD_DTYPES, ptr, require_gpu, row_stride, rows_are_dense, stream_handle
from qpu_xla_amd.errors import KernelError
from qpu_xla_amd.kernel import Kernel

INT32_MAX = 2**31 - 1


def pack_int8_quads(values: torch.Tensor) -> torch.Tensor:
    """int8 [R, C] -> int32 words [R, C/4], four adjacent bytes per word (gemm_int8.py:23-29)."""
    if values.dtype != torch.int8 or values.dim() != 2 or values.shape[1] % 4:
        raise ValueError("packed INT8 matrices must be rank-2 int8 with a final dimension divisible by four")
    return values.contiguous().view(torch.int32)


def pack_int8_gemm_operands(left: torch.Tensor, right: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Logical (P, Q) @ (Q, R) int8 -> (left words [P, Q/4], right words [Q/4, R]) (gemm_int8.py:32-40)."""
    if left.dim() != 2 or right.dim() != 2 or left.dtype != torch.int8 or right.dtype != torch.int8:
        raise ValueError("W8A8 GEMM operands must be rank-2 int8 matrices")
    if left.shape[1] != right.shape[0] or left.shape[1] % 4:
        raise ValueError("W8A8 GEMM reduction dimensions must align and be divisible by four")
    return pack_int8_quads(left), pack_int8_quads(right.t().contiguous()).t().contiguous()


def _check_accumulation(reduction: int) -> None:
    if reduction * 127 * 127 > INT32_MAX:
        raise ValueError("packed W8A8 GEMM accumulation can overflow int32")


def _words(t: Any) -> bool:
    return isinstance(t, torch.Tensor) and t.dtype in PACKED_WORD_DTYPES and t.dim() == 2


def supports_tiled_w8a8_gemm(left: torch.Tensor, right: torch.Tensor, destination: torch.Tensor) -> bool:
    """Packed-operand contract of the int32 GEMM (gemm_int8.py:224-236)."""
    if not (_words(left) and _words(right) and isinstance(destination, torch.Tensor)):
        return False
    if destination.dtype != torch.int32 or destination.dim() != 2:
        return False
    p, q_words = left.shape
    right_q_words, r = right.shape
    if q_words != right_q_words or tuple(destination.shape) != (p, r) or p % 16 or q_words % 4 or r % 16:
        return False
    if not all(rows_are_dense(t) for t in (left, right, destination)):
        return False
    return all(t.device.type == "cuda" for t in (left, right, destination)) and len(
        {t.device for t in (left, right, destination)}
    ) == 1


def supports_tiled_w8a8_gemm_dequantize(
    left: torch.Tensor,
    right: torch.Tensor,
    row_scales: torch.Tensor,
    column_scales: torch.Tensor,
    destination: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> bool:
    """Packed-operand contract of the fused dequant GEMM (gemm_int8.py:239-268)."""
    if not (_words(left) and _words(right)):
        return False
    floats = [row_scales, column_scales, destination] + ([bias] if bias is not None else [])
    if any(not isinstance(t, torch.Tensor) or t.dtype != torch.float32 for t in floats):
        return False
    if destination.dim() != 2:
        return False
    rows, q_words = left.shape
    right_q_words, columns = right.shape
    if (
        q_words != right_q_words
        or tuple(destination.shape) != (rows, columns)
        or rows % 16
        or q_words % 4
        or columns % 16
        or tuple(row_scales.shape) != (rows,)
        or tuple(column_scales.shape) != (columns,)
        or (bias is not None and tuple(bias.shape) != (columns,))
    ):
        return False
    tensors = [left, right, *floats]
    if not all(rows_are_dense(t) for t in tensors):
        return False
    return all(t.device.type == "cuda" for t in tensors) and len({t.device for t in tensors}) == 1


def _execute_tiled_w8a8_gemm(stream: Any, args: tuple[Any, ...], grid: tuple[int, int, int]) -> None:
    if len(args) != 3 or not all(isinstance(a, torch.Tensor) for a in args):
        raise KernelError("packed W8A8 GEMM expects (left, right, destination)")
    left, right, destination = args
    if not supports_tiled_w8a8_gemm(left, right, destination):
        raise KernelError("packed W8A8 GEMM requires packed word inputs, int32 output, and 16x16x16 logical tiles")
    want = (right.shape[1] // 16, left.shape[0] // 16, 1)
    if tuple(grid) != want:
        raise KernelError(f"packed W8A8 GEMM grid must be {want}, got {tuple(grid)}")
    _check_accumulation(left.shape[1] * 4)
    _lib.call(
        "qxt_w8a8_gemm_i32",
        ptr(left), row_stride(left), ptr(right), row_stride(right), ptr(destination), row_stride(destination),
        left.shape[0], right.shape[1], left.shape[1] * 4, _lib.WEIGHT_K4N, stream_handle(stream),
    )


TILED_W8A8_GEMM_KERNEL = Kernel("gfx950.tiled_w8a8_gemm", _execute_tiled_w8a8_gemm)


def _execute_tiled_w8a8_gemm_dequantize(stream: Any, args: tuple[Any, ...], grid: tuple[int, int, int]) -> None:
    if len(args) not in (5, 6) or not all(isinstance(a, torch.Tensor) for a in args):
        raise KernelError("fused W8A8 GEMM expects (left, right, row_scales, column_scales, destination[, bias])")
    left, right, row_scales, column_scales, destination = args[:5]
    bias = args[5] if len(args) == 6 else None
    if not supports_tiled_w8a8_gemm_dequantize(left, right, row_scales, column_scales, destination, bias):
        raise KernelError("fused W8A8 GEMM requires packed inputs, aligned FP32 output, and matching scales")
    want = (right.shape[1] // 16, left.shape[0] // 16, 1)
    if tuple(grid) != want:
        raise KernelError(f"fused W8A8 GEMM grid must be {want}, got {tuple(grid)}")
    _check_accumulation(left.shape[1] * 4)
    _lib.call(
        "qxt_w8a8_gemm_dequantize",
        ptr(left), row_stride(left), ptr(right), row_stride(right),
        ptr(row_scales), ptr(column_scales), ptr(bias), ptr(destination), row_stride(destination),
        left.shape[0], right.shape[1], left.shape[1] * 4, _lib.WEIGHT_K4N, stream_handle(stream),
    )


TILED_W8A8_GEMM_DEQUANTIZE_KERNEL = Kernel("gfx950.tiled_w8a8_gemm_dequantize", _execute_tiled_w8a8_gemm_dequantize)


# ------------------------------------------------------- natural-layout helpers


def _check_nk(name: str, a: torch.Tensor, w: torch.Tensor) -> tuple[int, int, int]:
    if a.dtype != torch.int8 or w.dtype != torch.int8 or a.dim() != 2 or w.dim() != 2:
        raise ValueError(f"{name}: int8 activations [M, K] and int8 weights [N, K] are required")
    m, k = a.shape
    n, k2 = w.shape
    if k != k2 or k % 16:
        raise ValueError(f"{name}: K must match and be a multiple of 16")
    if not (rows_are_dense(a) and rows_are_dense(w)):
        raise ValueError(f"{name}: operands need contiguous rows")
    _check_accumulation(k)
    return m, n, k


def w8a8_gemm_i32(a: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None, *, stream: Any = None) -> torch.Tensor:
    """Exact int32 ``a @ w.T`` for int8 a [M, K], w [N, K]."""
    m, n, k = _check_nk("w8a8_gemm_i32", a, w)
    if out is None:
        out = torch.empty((m, n), dtype=torch.int32, device=a.device)
    require_gpu("w8a8_gemm_i32", a, w, out)
    _lib.call(
        "qxt_w8a8_gemm_i32", ptr(a), row_stride(a), ptr(w), row_stride(w), ptr(out), row_stride(out),
        m, n, k, _lib.WEIGHT_NK, stream_handle(stream),
    )
    return out


def w8a8_gemm_dequantize(
    a: torch.Tensor,
    w: torch.Tensor,
    row_scales: torch.Tensor,
    column_scales: torch.Tensor,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    *,
    stream: Any = None,
) -> torch.Tensor:
    """``fl32(fl32(float(a @ w.T) * sa) * sw) (+ bias)`` in one fused kernel."""
    m, n, k = _check_nk("w8a8_gemm_dequantize", a, w)
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    for t, shape in ((row_scales, (m,)), (column_scales, (n,))):
        if t.dtype != torch.float32 or t.shape[0] < shape[0] or not t.is_contiguous():
            raise ValueError("w8a8_gemm_dequantize: scales must be contiguous float32")
    if bias is not None and (bias.dtype != torch.float32 or tuple(bias.shape) != (n,) or not bias.is_contiguous()):
        raise ValueError("w8a8_gemm_dequantize: bias must be contiguous float32 [N]")
    require_gpu("w8a8_gemm_dequantize", a, w, row_scales, column_scales, bias, out)
    _lib.call(
        "qxt_w8a8_gemm_dequantize", ptr(a), row_stride(a), ptr(w), row_stride(w),
        ptr(row_scales), ptr(column_scales), ptr(bias), ptr(out), row_stride(out),
        m, n, k, _lib.WEIGHT_NK, stream_handle(stream),
    )
    return out
