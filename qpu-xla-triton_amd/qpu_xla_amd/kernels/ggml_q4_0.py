"""Native GGML Q4_0 x Q8_0 linear on gfx950.

Mirrors the operator surface of the reference's
``src/qpu_xla/kernels/ggml_q4_0.py``: the same block constants and codec
helpers, a ``supports_ggml_q4_0_q8_0_linear`` predicate, an executor that
re-validates and checks the grid, and a ``Kernel`` constant submitted through
``Queue.submit(kernel, (activation, weight, destination, wcol0, ocol0, ncols),
grid=(ncols // 16, ceil(rows / 4), 1))``.  Tensors are torch tensors on the
HIP device; the kernel writes only ``destination[:, ocol0:ocol0 + ncols]``.

Differences from the reference contract, all widening it: any ``rows >= 1``
(the reference QPU program needs 4 or a multiple of 16 and its native runtime
replicates M=1 four times), and the grid's row extent is ``ceil(rows / 4)``.
"""

from __future__ import annotations

from typing import Any

import torch

from qpu_xla_amd import _lib
from qpu_xla_amd._tensors import PACKED_WORD_DTYPES, ptr, require_gpu, row_stride, rows_are_dense, stream_handle
from qpu_xla_amd.errors import KernelError
from qpu_xla_amd.kernel import Kernel

Q4_0_BLOCK_ELEMENTS = 32
Q4_0_BLOCK_BYTES = 18
Q8_0_BLOCK_BYTES = 34
OUTPUT_TILE = 16
ROW_TILE = 4
MX_ROW_TILE = 16  # row tile of the tiled (prefill) kernel's grid, as the reference's


# ----------------------------------------------------------------- block codec
# Same byte layouts as the reference codec (ggml_q4_0.py:28-78), on torch tensors
# of any device.


def pack_ggml_q4_0_blocks(scales: torch.Tensor, codes: torch.Tensor) -> torch.Tensor:
    """fp16-representable scales [...] and 0..15 codes [..., 32] -> uint8 [..., 18]."""
    codes = torch.as_tensor(codes)
    scales = torch.as_tensor(scales).to(torch.float16)
    if tuple(codes.shape) != (*scales.shape, Q4_0_BLOCK_ELEMENTS) or bool(((codes < 0) | (codes > 15)).any()):
        raise ValueError("Q4_0 codes must have scales.shape + (32,) and values in 0..15")
    out = torch.empty((*scales.shape, Q4_0_BLOCK_BYTES), dtype=torch.uint8, device=codes.device)
    out[..., 0:2] = scales.contiguous().view(torch.uint8).reshape(*scales.shape, 2).to(codes.device)
    c = codes.to(torch.uint8)
    out[..., 2:] = c[..., :16] | (c[..., 16:] << 4)
    return out


def pack_ggml_q8_0_blocks(scales: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
    """fp16-representable scales [...] and int8 values [..., 32] -> uint8 [..., 34]."""
    values = torch.as_tensor(values)
    scales = torch.as_tensor(scales).to(torch.float16)
    if tuple(values.shape) != (*scales.shape, Q4_0_BLOCK_ELEMENTS) or bool(((values < -128) | (values > 127)).any()):
        raise ValueError("Q8_0 values must have scales.shape + (32,) and values in -128..127")
    out = torch.empty((*scales.shape, Q8_0_BLOCK_BYTES), dtype=torch.uint8, device=values.device)
    out[..., 0:2] = scales.contiguous().view(torch.uint8).reshape(*scales.shape, 2).to(values.device)
    out[..., 2:] = values.to(torch.int8).view(torch.uint8)
    return out


def unpack_ggml_q4_0_blocks(blocks: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """uint8 [..., 18] -> (float32 scales [...], int8 values [..., 32] in -8..7)."""
    if blocks.dtype != torch.uint8 or blocks.dim() < 1 or blocks.shape[-1] != Q4_0_BLOCK_BYTES:
        raise ValueError("Q4_0 blocks must be uint8 with a final extent of 18 bytes")
    scales = blocks[..., 0:2].contiguous().view(torch.float16).squeeze(-1).to(torch.float32)
    qs = blocks[..., 2:]
    values = torch.cat(((qs & 0x0F).to(torch.int8) - 8, (qs >> 4).to(torch.int8) - 8), dim=-1)
    return scales, values


def unpack_ggml_q8_0_blocks(blocks: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """uint8 [..., 34] -> (float32 scales [...], int8 values [..., 32])."""
    if blocks.dtype != torch.uint8 or blocks.dim() < 1 or blocks.shape[-1] != Q8_0_BLOCK_BYTES:
        raise ValueError("Q8_0 blocks must be uint8 with a final extent of 34 bytes")
    scales = blocks[..., 0:2].contiguous().view(torch.float16).squeeze(-1).to(torch.float32)
    return scales, blocks[..., 2:].contiguous().view(torch.int8)


# ------------------------------------------------------------------- operator


def supports_ggml_q4_0_q8_0_linear(
    activation: torch.Tensor,
    weight: torch.Tensor,
    destination: torch.Tensor,
    weight_column_start: int,
    output_column_start: int,
    column_count: int,
) -> bool:
    """Whether native block tensors meet the small-M contract (ggml_q4_0.py:725-761)."""
    tensors = (activation, weight, destination)
    if not all(isinstance(t, torch.Tensor) for t in tensors):
        return False
    if any(t.device.type != "cuda" for t in tensors) or len({t.device for t in tensors}) != 1:
        return False
    if activation.dtype != torch.uint8 or weight.dtype != torch.uint8 or destination.dtype != torch.float32:
        return False
    if activation.dim() != 3 or weight.dim() != 3 or destination.dim() != 2:
        return False
    rows, blocks, activation_bytes = activation.shape
    outputs, weight_blocks, weight_bytes = weight.shape
    if rows <= 0 or activation_bytes != Q8_0_BLOCK_BYTES or weight_bytes != Q4_0_BLOCK_BYTES:
        return False
    if blocks <= 0 or blocks != weight_blocks or destination.shape[0] != rows:
        return False
    starts = (weight_column_start, output_column_start)
    if any(s < 0 or s % OUTPUT_TILE for s in starts) or column_count <= 0 or column_count % OUTPUT_TILE:
        return False
    if weight_column_start + column_count > outputs or output_column_start + column_count > destination.shape[1]:
        return False
    return activation.is_contiguous() and weight.is_contiguous() and rows_are_dense(destination)


def expected_grid(rows: int, column_count: int) -> tuple[int, int, int]:
    return (column_count // OUTPUT_TILE, (rows + ROW_TILE - 1) // ROW_TILE, 1)


def _launch_linear(activation, weight, destination, wcol0, ocol0, ncols, stream) -> None:
    rows, blocks, _ = activation.shape
    _lib.call(
        "qxt_ggml_q4_0_q8_0_linear",
        ptr(activation), row_stride(activation), ptr(weight), row_stride(weight),
        ptr(destination), row_stride(destination),
        rows, blocks, wcol0, ocol0, ncols, stream_handle(stream),
    )


def _execute_ggml_q4_0_q8_0_linear(stream: Any, args: tuple[Any, ...], grid: tuple[int, int, int]) -> None:
    if len(args) != 6 or not all(isinstance(a, torch.Tensor) for a in args[:3]):
        raise KernelError(
            "GGML Q4_0 linear expects "
            "(activation, weight, destination, weight_column_start, output_column_start, column_count)"
        )
    activation, weight, destination, wcol0, ocol0, ncols = args
    if not all(isinstance(v, int) for v in (wcol0, ocol0, ncols)):
        raise KernelError("GGML Q4_0 column bounds must be integers")
    if not supports_ggml_q4_0_q8_0_linear(activation, weight, destination, wcol0, ocol0, ncols):
        raise KernelError("GGML Q4_0 linear requires native contiguous Q8_0/Q4_0 blocks and aligned columns")
    want = expected_grid(activation.shape[0], ncols)
    if tuple(grid) != want:
        raise KernelError(f"GGML Q4_0 linear grid must be {want}, got {tuple(grid)}")
    _launch_linear(activation, weight, destination, wcol0, ocol0, ncols, stream)


GGML_Q4_0_Q8_0_LINEAR_KERNEL = Kernel("gfx950.ggml_q4_0_q8_0_linear", _execute_ggml_q4_0_q8_0_linear)


def ggml_q4_0_q8_0_linear(
    activation: torch.Tensor,
    weight: torch.Tensor,
    destination: torch.Tensor | None = None,
    *,
    weight_column_start: int = 0,
    output_column_start: int = 0,
    column_count: int | None = None,
    stream: Any = None,
) -> torch.Tensor:
    """Functional form: any column range (no 16-alignment), returns ``destination``."""
    if activation.dim() != 3 or weight.dim() != 3:
        raise ValueError("activation [M, B, 34] and weight [N, B, 18] blocks are required")
    rows = activation.shape[0]
    if column_count is None:
        column_count = weight.shape[0] - weight_column_start
    if destination is None:
        destination = torch.empty((rows, output_column_start + column_count), dtype=torch.float32, device=weight.device)
    require_gpu("ggml_q4_0_q8_0_linear", activation, weight, destination)
    if not (activation.is_contiguous() and weight.is_contiguous() and rows_are_dense(destination)):
        raise ValueError("ggml_q4_0_q8_0_linear: tensors need contiguous rows")
    if activation.dtype != torch.uint8 or weight.dtype != torch.uint8 or destination.dtype != torch.float32:
        raise ValueError("ggml_q4_0_q8_0_linear: uint8 blocks and a float32 destination are required")
    if activation.shape[2] != Q8_0_BLOCK_BYTES or weight.shape[2] != Q4_0_BLOCK_BYTES or activation.shape[1] != weight.shape[1]:
        raise ValueError("ggml_q4_0_q8_0_linear: block extents or counts do not match")
    if weight_column_start < 0 or weight_column_start + column_count > weight.shape[0]:
        raise ValueError("ggml_q4_0_q8_0_linear: weight column range out of bounds")
    if output_column_start < 0 or output_column_start + column_count > destination.shape[1] or destination.shape[0] != rows:
        raise ValueError("ggml_q4_0_q8_0_linear: destination too small")
    _launch_linear(activation, weight, destination, weight_column_start, output_column_start, column_count, stream)
    return destination


# ------------------------------------------------------------- lane layout
# Decode-path weight layout (qxt_q4_0_pack_lanes): the native rows' 144-byte
# units (8 blocks of one column) in groups of 64, chunk v of unit l of a group
# at (v * 64 + l) * 16, so every 16-byte load instruction of a wave reads one
# contiguous kilobyte.  Same bytes, prepared once like the reference's
# prepared-linear weight upload (qpu_llama_q4_0.c:343-395).

LANE_GROUP_UNITS = 64
LANE_UNIT_BYTES = 144


class Q4_0LaneWeights:
    """A Q4_0 matrix [columns, blocks, 18] held in the lane layout (uint8 device tensor)."""

    def __init__(self, packed: torch.Tensor, columns: int, blocks: int) -> None:
        need = lanes_bytes(columns, blocks)
        if packed.dtype != torch.uint8 or packed.dim() != 1 or packed.numel() < need or not packed.is_contiguous():
            raise ValueError("lane weights must be a contiguous uint8 tensor of qxt_q4_0_lanes_bytes bytes")
        self.packed = packed
        self.columns = int(columns)
        self.blocks = int(blocks)

    @property
    def device(self) -> torch.device:
        return self.packed.device

    @property
    def shape(self) -> tuple[int, int, int]:
        """Shape of the native matrix this holds."""
        return (self.columns, self.blocks, Q4_0_BLOCK_BYTES)


def lanes_bytes(columns: int, blocks: int) -> int:
    """Bytes of the lane layout (whole 64-unit groups); needs blocks % 8 == 0."""
    if columns <= 0 or blocks <= 0 or blocks % 8:
        raise ValueError("the lane layout needs columns > 0 and blocks % 8 == 0")
    units = columns * (blocks // 8)
    return -(-units // LANE_GROUP_UNITS) * LANE_GROUP_UNITS * LANE_UNIT_BYTES


def pack_ggml_q4_0_lane_weights(weight: torch.Tensor, *, stream: Any = None) -> Q4_0LaneWeights:
    """Repack native Q4_0 blocks uint8 [N, B, 18] (B % 8 == 0) into the lane layout on the GPU."""
    if weight.dtype != torch.uint8 or weight.dim() != 3 or weight.shape[2] != Q4_0_BLOCK_BYTES or not weight.is_contiguous():
        raise ValueError("pack_ggml_q4_0_lane_weights: contiguous uint8 [N, B, 18] blocks are required")
    columns, blocks, _ = weight.shape
    packed = torch.empty(lanes_bytes(columns, blocks), dtype=torch.uint8, device=weight.device)
    require_gpu("pack_ggml_q4_0_lane_weights", weight, packed)
    _lib.call("qxt_q4_0_pack_lanes", ptr(weight), row_stride(weight), ptr(packed), packed.numel(), columns, blocks,
              stream_handle(stream))
    return Q4_0LaneWeights(packed, columns, blocks)


def ggml_q4_0_q8_0_lane_linear(
    activation: torch.Tensor,
    weight: Q4_0LaneWeights,
    destination: torch.Tensor | None = None,
    *,
    weight_column_start: int = 0,
    output_column_start: int = 0,
    column_count: int | None = None,
    stream: Any = None,
) -> torch.Tensor:
    """``ggml_q4_0_q8_0_linear`` over lane-layout weights (same result bit for bit)."""
    if activation.dim() != 3 or activation.dtype != torch.uint8 or activation.shape[2] != Q8_0_BLOCK_BYTES:
        raise ValueError("ggml_q4_0_q8_0_lane_linear: activation must be uint8 [M, B, 34]")
    rows, blocks = activation.shape[0], activation.shape[1]
    if blocks != weight.blocks or not activation.is_contiguous():
        raise ValueError("ggml_q4_0_q8_0_lane_linear: contiguous activation with the weight's block count required")
    if column_count is None:
        column_count = weight.columns - weight_column_start
    if destination is None:
        destination = torch.empty((rows, output_column_start + column_count), dtype=torch.float32, device=weight.device)
    if destination.dtype != torch.float32 or not rows_are_dense(destination):
        raise ValueError("ggml_q4_0_q8_0_lane_linear: float32 destination with contiguous rows required")
    if weight_column_start < 0 or weight_column_start + column_count > weight.columns:
        raise ValueError("ggml_q4_0_q8_0_lane_linear: weight column range out of bounds")
    if output_column_start < 0 or output_column_start + column_count > destination.shape[1] or destination.shape[0] != rows:
        raise ValueError("ggml_q4_0_q8_0_lane_linear: destination too small")
    require_gpu("ggml_q4_0_q8_0_lane_linear", activation, weight.packed, destination)
    _lib.call(
        "qxt_ggml_q4_0_q8_0_linear_lanes",
        ptr(activation), row_stride(activation), ptr(weight.packed), weight.columns,
        ptr(destination), row_stride(destination),
        rows, blocks, weight_column_start, output_column_start, column_count, stream_handle(stream),
    )
    return destination


def ggml_q4_0_q8_0_block_dots(
    activation: torch.Tensor,
    weight: torch.Tensor,
    *,
    weight_column_start: int = 0,
    column_count: int | None = None,
    stream: Any = None,
) -> torch.Tensor:
    """Debug path: exact int32 block dots [M, column_count, B]."""
    rows, blocks, _ = activation.shape
    if column_count is None:
        column_count = weight.shape[0] - weight_column_start
    if weight_column_start < 0 or weight_column_start + column_count > weight.shape[0]:
        raise ValueError("block dots: weight column range out of bounds")
    dots = torch.empty((rows, column_count, blocks), dtype=torch.int32, device=weight.device)
    require_gpu("ggml_q4_0_q8_0_block_dots", activation, weight, dots)
    if not (activation.is_contiguous() and weight.is_contiguous()):
        raise ValueError("block dots: contiguous block tensors required")
    _lib.call(
        "qxt_ggml_q4_0_q8_0_block_dots",
        ptr(activation), row_stride(activation), ptr(weight), row_stride(weight), ptr(dots),
        rows, blocks, weight_column_start, column_count, stream_handle(stream),
    )
    return dots


# ------------------------------------------------------- tiled (prefill) layout
# The split operands of the reference's GGML_Q4_0_Q8_0_TILED_LINEAR_KERNEL
# (ggml_q4_0.py:844-967): activation int8 [M, K] + fp16 scale bits [M, B]
# (2-byte halves, or 4-byte words when the reference's activation_scale_word
# program is used); weight uint32 words [B * 8, N] of signed int8 quads + fp16
# scale bits [B, N].  Word dtypes: int32/uint32; half dtypes: int16/uint16.

_HALF_DTYPES = (torch.int16, torch.uint16)


def pack_ggml_q4_0_tiled_weights(blocks: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Native Q4_0 weights uint8 [N, B, 18] -> (scale bits int16 [B, N], words int32 [B * 8, N]).

    Same layout as the reference's ``pack_ggml_q4_0_tiled_weights``
    (ggml_q4_0.py:844-855): word ``(8 b + g, n)`` holds the signed values
    ``code - 8`` of elements ``4 g .. 4 g + 3`` of block ``b`` of output ``n``.
    """
    if blocks.dtype != torch.uint8 or blocks.dim() != 3 or blocks.shape[2] != Q4_0_BLOCK_BYTES:
        raise ValueError("native Q4_0 weights must be uint8 [outputs, blocks, 18]")
    outputs, nblocks, _ = blocks.shape
    scale_bits = blocks[..., 0:2].contiguous().view(torch.int16).reshape(outputs, nblocks).t().contiguous()
    qs = blocks[..., 2:]
    values = torch.cat(((qs & 0x0F).to(torch.int8) - 8, (qs >> 4).to(torch.int8) - 8), dim=-1)
    groups = values.reshape(outputs, nblocks, 8, 4).permute(1, 2, 0, 3).contiguous()
    return scale_bits, groups.view(torch.int32).reshape(nblocks * 8, outputs)


def split_ggml_q8_0_blocks(blocks: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Native Q8_0 activations uint8 [M, B, 34] -> (scale bits int16 [M, B], values uint8 [M, B * 32])."""
    if blocks.dtype != torch.uint8 or blocks.dim() != 3 or blocks.shape[2] != Q8_0_BLOCK_BYTES:
        raise ValueError("native Q8_0 activations must be uint8 [rows, blocks, 34]")
    rows, nblocks, _ = blocks.shape
    scales = blocks[..., 0:2].contiguous().view(torch.int16).reshape(rows, nblocks)
    values = blocks[..., 2:].contiguous().reshape(rows, nblocks * Q4_0_BLOCK_ELEMENTS)
    return scales, values


def supports_ggml_q4_0_q8_0_tiled_linear(
    activation_q: torch.Tensor,
    activation_scales: torch.Tensor,
    weight_q: torch.Tensor,
    weight_scales: torch.Tensor,
    destination: torch.Tensor,
) -> bool:
    """Whether split tensors meet the tiled contract (ggml_q4_0.py:886-920), widened to any M and N."""
    tensors = (activation_q, activation_scales, weight_q, weight_scales, destination)
    if not all(isinstance(t, torch.Tensor) and t.dim() == 2 for t in tensors):
        return False
    if any(t.device.type != "cuda" for t in tensors) or len({t.device for t in tensors}) != 1:
        return False
    if activation_q.dtype not in (torch.uint8, torch.int8) or weight_q.dtype not in PACKED_WORD_DTYPES:
        return False
    if activation_scales.dtype not in _HALF_DTYPES + PACKED_WORD_DTYPES or weight_scales.dtype not in _HALF_DTYPES:
        return False
    if destination.dtype != torch.float32:
        return False
    rows, columns = activation_q.shape
    if rows <= 0 or columns <= 0 or columns % Q4_0_BLOCK_ELEMENTS:
        return False
    blocks = columns // Q4_0_BLOCK_ELEMENTS
    outputs = weight_q.shape[1]
    shapes_ok = (
        outputs > 0
        and tuple(activation_scales.shape) == (rows, blocks)
        and tuple(weight_q.shape) == (blocks * 8, outputs)
        and tuple(weight_scales.shape) == (blocks, outputs)
        and tuple(destination.shape) == (rows, outputs)
    )
    return shapes_ok and all(t.is_contiguous() for t in tensors)


def tiled_grid(rows: int, outputs: int) -> tuple[int, int, int]:
    return ((outputs + OUTPUT_TILE - 1) // OUTPUT_TILE, (rows + MX_ROW_TILE - 1) // MX_ROW_TILE, 1)


def _launch_tiled(activation_q, activation_scales, weight_q, weight_scales, destination, stream) -> None:
    rows, columns = activation_q.shape
    _lib.call(
        "qxt_ggml_q4_0_q8_0_tiled_linear",
        ptr(activation_q), row_stride(activation_q), ptr(activation_scales), row_stride(activation_scales),
        activation_scales.element_size(), ptr(weight_q), row_stride(weight_q), ptr(weight_scales),
        row_stride(weight_scales), ptr(destination), row_stride(destination),
        rows, columns // Q4_0_BLOCK_ELEMENTS, weight_q.shape[1], stream_handle(stream),
    )


def _execute_ggml_q4_0_q8_0_tiled_linear(stream: Any, args: tuple[Any, ...], grid: tuple[int, int, int]) -> None:
    if len(args) != 5 or not all(isinstance(a, torch.Tensor) for a in args):
        raise KernelError("tiled Q4_0 linear expects split activation/weight scales, values, and output")
    if not supports_ggml_q4_0_q8_0_tiled_linear(*args):
        raise KernelError("tiled Q4_0 linear requires aligned contiguous split tensors")
    activation_q, _, weight_q, _, destination = args
    want = tiled_grid(activation_q.shape[0], weight_q.shape[1])
    if tuple(grid) != want:
        raise KernelError(f"tiled Q4_0 linear grid must be {want}, got {tuple(grid)}")
    _launch_tiled(*args, stream)


GGML_Q4_0_Q8_0_TILED_LINEAR_KERNEL = Kernel("gfx950.ggml_q4_0_q8_0_tiled_linear", _execute_ggml_q4_0_q8_0_tiled_linear)


def ggml_q4_0_q8_0_tiled_linear(
    activation_q: torch.Tensor,
    activation_scales: torch.Tensor,
    weight_q: torch.Tensor,
    weight_scales: torch.Tensor,
    destination: torch.Tensor | None = None,
    *,
    stream: Any = None,
) -> torch.Tensor:
    """Functional form of the tiled linear; returns the fp32 [M, N] destination."""
    if destination is None:
        destination = torch.empty((activation_q.shape[0], weight_q.shape[1]), dtype=torch.float32, device=weight_q.device)
    if not supports_ggml_q4_0_q8_0_tiled_linear(activation_q, activation_scales, weight_q, weight_scales, destination):
        raise ValueError("ggml_q4_0_q8_0_tiled_linear: operands do not meet the tiled layout contract")
    _launch_tiled(activation_q, activation_scales, weight_q, weight_scales, destination, stream)
    return destination


class Q4_0LinearBatch:
    """Independent Q4_0 x Q8_0 linears computed by one kernel launch.

    Each task is a dict with ``weight`` (uint8 [N, B, 18], or a
    ``Q4_0LaneWeights`` from ``pack_ggml_q4_0_lane_weights``), ``destination``
    (float32 [rows, >= N]) and exactly one of ``x`` (float32 [rows, B*32]:
    quantised to Q8_0 inside the kernel, same rule as ``quantize_q8_0``) or
    ``activation`` (native Q8_0 uint8 [rows, B, 34]); optional
    ``weight_column_start``, ``output_column_start`` and ``column_count``.
    The batch keeps references to every tensor; their storage must not be
    reallocated while the batch is alive (launches read the pointers
    captured at construction).  This is the prepared-handle shape of the
    reference's ``qpu_llama_q4_0_linear_prepare`` / ``_submit``
    (integrations/llama_cpp/include/qpu_llama_q4_0.h:63-75).
    """

    def __init__(self, tasks: list[dict]) -> None:
        import ctypes

        if not tasks:
            raise ValueError("Q4_0LinearBatch needs at least one task")
        self._tensors = []
        table = (_lib.Q4Task * len(tasks))()
        for i, spec in enumerate(tasks):
            weight = spec["weight"]
            destination = spec["destination"]
            x = spec.get("x")
            activation = spec.get("activation")
            if (x is None) == (activation is None):
                raise ValueError("each task needs exactly one of 'x' and 'activation'")
            lanes = isinstance(weight, Q4_0LaneWeights)
            if lanes:
                weight_tensor = weight.packed
            else:
                weight_tensor = weight
                if weight.dtype != torch.uint8 or weight.dim() != 3 or weight.shape[2] != Q4_0_BLOCK_BYTES:
                    raise ValueError("task weight must be uint8 [N, B, 18] or Q4_0LaneWeights")
                if not weight.is_contiguous():
                    raise ValueError("task weight must be contiguous")
            if destination.dtype != torch.float32 or not rows_are_dense(destination):
                raise ValueError("task destination must be float32 with contiguous rows")
            blocks = weight.shape[1]
            source = x if x is not None else activation
            rows = source.shape[0]
            wcol0 = int(spec.get("weight_column_start", 0))
            ocol0 = int(spec.get("output_column_start", 0))
            ncols = int(spec.get("column_count", weight.shape[0] - wcol0))
            if wcol0 < 0 or wcol0 + ncols > weight.shape[0] or ocol0 < 0 or ocol0 + ncols > destination.shape[1]:
                raise ValueError("task column range out of bounds")
            if destination.shape[0] != rows:
                raise ValueError("task destination rows differ from the activation rows")
            if x is not None:
                if x.dtype != torch.float32 or x.dim() != 2 or x.shape[1] != blocks * Q4_0_BLOCK_ELEMENTS or not rows_are_dense(x):
                    raise ValueError("task x must be float32 [rows, K] with contiguous rows")
                table[i].x = x.data_ptr()
                table[i].x_row_stride = row_stride(x)
            else:
                if activation.dtype != torch.uint8 or tuple(activation.shape[1:]) != (blocks, Q8_0_BLOCK_BYTES) or not activation.is_contiguous():
                    raise ValueError("task activation must be contiguous uint8 [rows, B, 34]")
                table[i].activation = activation.data_ptr()
                table[i].activation_row_stride = row_stride(activation)
            require_gpu("Q4_0LinearBatch", source, weight_tensor, destination)
            table[i].weight = weight_tensor.data_ptr()
            table[i].weight_row_stride = 0 if lanes else row_stride(weight_tensor)
            table[i].weight_layout = _lib.Q4_0_LAYOUT_LANES if lanes else _lib.Q4_0_LAYOUT_NATIVE
            table[i].destination = destination.data_ptr()
            table[i].destination_row_stride = row_stride(destination)
            table[i].rows = rows
            table[i].blocks = blocks
            table[i].weight_column_start = wcol0
            table[i].output_column_start = ocol0
            table[i].column_count = ncols
            self._tensors.extend(t for t in (x, activation, weight_tensor, destination) if t is not None)
        handle = ctypes.c_void_p()
        _lib.check(_lib.load().qxt_q4_0_batch_prepare(table, len(tasks), ctypes.byref(handle)))
        self._handle = handle
        self.task_count = len(tasks)
        self.work_items = int(_lib.load().qxt_q4_0_batch_work_items(handle))

    def launch(self, stream: Any = None) -> None:
        if self._handle is None:
            raise RuntimeError("Q4_0LinearBatch is closed")
        _lib.call("qxt_q4_0_batch_launch", self._handle, stream_handle(stream))

    def close(self) -> None:
        if self._handle is not None:
            _lib.load().qxt_q4_0_batch_destroy(self._handle)
            self._handle = None
            self._tensors = []

    def __enter__(self) -> "Q4_0LinearBatch":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass
