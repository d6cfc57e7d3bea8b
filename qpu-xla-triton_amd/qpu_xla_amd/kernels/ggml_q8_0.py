"""Native GGML Q8_0 x Q8_0 linear on gfx950.

Mirrors ``src/qpu_xla/kernels/ggml_q8_0.py``: a ``supports_*`` predicate, an
executor that re-validates and checks the grid, and
``GGML_Q8_0_Q8_0_LINEAR_M4_KERNEL`` submitted as
``Queue.submit(kernel, (activation, weight, destination, wcol0, ocol0, ncols),
grid=(ncols // 16, 1, 1))`` with four activation rows.  The result equals
``ggml_q8_0_q8_0_reference`` (``:26-51``) bit for bit: per block an exact
int32 dot, scaled by the activation scale, then the weight scale, summed in
block order.

Widened contract: the functional form takes any row count and column range;
the ``Kernel`` keeps the reference's exact M=4, 16-aligned contract.
"""

from __future__ import annotations

from typing import Any

import torch

from qpu_xla_amd import _lib
from qpu_xla_amd._tensors import ptr, require_gpu, row_stride, rows_are_dense, stream_handle
from qpu_xla_amd.errors import KernelError
from qpu_xla_amd.kernel import Kernel

QK8_0 = 32
Q8_0_BLOCK_BYTES = 34
OUTPUT_TILE = 16


def supports_ggml_q8_0_q8_0_linear_m4(
    activation: Any, weight: Any, destination: Any, weight_column_start: int, output_column_start: int,
    column_count: int,
) -> bool:
    """Exact M=4 contract of the reference kernel (``ggml_q8_0.py:183-217``) on HIP tensors."""
    if not all(isinstance(t, torch.Tensor) for t in (activation, weight, destination)):
        return False
    if activation.dtype != torch.uint8 or weight.dtype != torch.uint8 or destination.dtype != torch.float32:
        return False
    if activation.dim() != 3 or weight.dim() != 3 or destination.dim() != 2:
        return False
    rows, blocks, a_bytes = activation.shape
    outputs, w_blocks, w_bytes = weight.shape
    if rows != 4 or a_bytes != Q8_0_BLOCK_BYTES or w_bytes != Q8_0_BLOCK_BYTES:
        return False
    if blocks != w_blocks or destination.shape[0] != rows:
        return False
    if weight_column_start < 0 or output_column_start < 0:
        return False
    if weight_column_start % OUTPUT_TILE or output_column_start % OUTPUT_TILE:
        return False
    if column_count <= 0 or column_count % OUTPUT_TILE:
        return False
    if weight_column_start + column_count > outputs or output_column_start + column_count > destination.shape[1]:
        return False
    if not (activation.is_contiguous() and weight.is_contiguous() and destination.is_contiguous()):
        return False
    return activation.is_cuda and weight.is_cuda and destination.is_cuda


def _launch(activation, weight, destination, wcol0, ocol0, ncols, stream) -> None:
    rows, blocks, _ = activation.shape
    _lib.call(
        "qxt_ggml_q8_0_q8_0_linear",
        ptr(activation), row_stride(activation), ptr(weight), row_stride(weight),
        ptr(destination), row_stride(destination), rows, blocks, wcol0, ocol0, ncols, stream_handle(stream),
    )


def _execute_ggml_q8_0_q8_0_linear_m4(stream: Any, args: tuple[Any, ...], grid: tuple[int, int, int]) -> None:
    if len(args) != 6 or not all(isinstance(a, torch.Tensor) for a in args[:3]):
        raise KernelError(
            "GGML Q8_0 linear expects "
            "(activation, weight, destination, weight_column_start, output_column_start, column_count)"
        )
    activation, weight, destination, wcol0, ocol0, ncols = args
    if not all(isinstance(v, int) for v in (wcol0, ocol0, ncols)):
        raise KernelError("GGML Q8_0 column bounds must be integers")
    if not supports_ggml_q8_0_q8_0_linear_m4(activation, weight, destination, wcol0, ocol0, ncols):
        raise KernelError("GGML Q8_0 linear requires contiguous native M=4 blocks and aligned columns")
    want = (ncols // OUTPUT_TILE, 1, 1)
    if tuple(grid) != want:
        raise KernelError(f"GGML Q8_0 linear grid must be {want}, got {tuple(grid)}")
    _launch(activation, weight, destination, wcol0, ocol0, ncols, stream)


GGML_Q8_0_Q8_0_LINEAR_M4_KERNEL = Kernel("gfx950.ggml_q8_0_q8_0_linear_m4", _execute_ggml_q8_0_q8_0_linear_m4)


def ggml_q8_0_q8_0_linear(
    activation: torch.Tensor,
    weight: torch.Tensor,
    destination: torch.Tensor | None = None,
    *,
    weight_column_start: int = 0,
    output_column_start: int = 0,
    column_count: int | None = None,
    stream: Any = None,
) -> torch.Tensor:
    """Functional form: any row count and column range; returns ``destination``."""
    if activation.dim() != 3 or weight.dim() != 3:
        raise ValueError("activation [M, B, 34] and weight [N, B, 34] blocks are required")
    rows = activation.shape[0]
    if column_count is None:
        column_count = weight.shape[0] - weight_column_start
    if destination is None:
        destination = torch.empty((rows, output_column_start + column_count), dtype=torch.float32, device=weight.device)
    require_gpu("ggml_q8_0_q8_0_linear", activation, weight, destination)
    if activation.dtype != torch.uint8 or weight.dtype != torch.uint8 or destination.dtype != torch.float32:
        raise ValueError("ggml_q8_0_q8_0_linear: uint8 blocks and a float32 destination are required")
    if not (activation.is_contiguous() and weight.is_contiguous() and rows_are_dense(destination)):
        raise ValueError("ggml_q8_0_q8_0_linear: tensors need contiguous rows")
    if activation.shape[2] != Q8_0_BLOCK_BYTES or weight.shape[2] != Q8_0_BLOCK_BYTES or activation.shape[1] != weight.shape[1]:
        raise ValueError("ggml_q8_0_q8_0_linear: block extents or counts do not match")
    if weight_column_start < 0 or weight_column_start + column_count > weight.shape[0]:
        raise ValueError("ggml_q8_0_q8_0_linear: weight column range out of bounds")
    if output_column_start < 0 or output_column_start + column_count > destination.shape[1] or destination.shape[0] != rows:
        raise ValueError("ggml_q8_0_q8_0_linear: destination too small")
    _launch(activation, weight, destination, weight_column_start, output_column_start, column_count, stream)
    return destination


__all__ = [
    "GGML_Q8_0_Q8_0_LINEAR_M4_KERNEL",
    "ggml_q8_0_q8_0_linear",
    "supports_ggml_q8_0_q8_0_linear_m4",
]
