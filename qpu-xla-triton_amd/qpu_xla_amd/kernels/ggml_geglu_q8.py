"""Fused GGML GEGLU -> native Q8_0 activation producer on gfx950.

Mirrors ``src/qpu_xla/kernels/ggml_geglu_q8.py``:

* ``ggml_gelu_fp16_table()`` -- the exact-GELU fp16 lookup table (``:26-34``),
  built by the library's host routine ``qxt_ggml_gelu_fp16_table``.
* ``GGML_GEGLU_Q8_0_KERNEL`` submitted as ``Queue.submit(kernel, (gate, up,
  destination, gelu_table), grid=(K // 32, M, 1))`` writes native 34-byte
  Q8_0 blocks [M, K/32, 34] (``:262-308``).
* ``GGML_GEGLU_Q8_0_SPLIT_KERNEL`` with ``(gate, up, scales, values,
  gelu_table)`` writes the split planes the tiled Q4_0 linear reads: fp16
  scale bits zero-extended in uint32 [M, K/32] and int8 values [M, K]
  (``:311-385``).

Both equal ``ggml_geglu_q8_0_reference`` (``:37-59``) bit for bit: the gate
is rounded to fp16 (nearest even) to index the table, the table value times
``up`` in fp32 is quantised per 32-element block with ``d = absmax / 127``,
``inverse = 1 / d`` (0 when d is 0), ``q = clip(rint(v * inverse), +-127)``.

Widened contract: the functional forms take rows with any stride (dense
within a row) and 2-byte scale planes as well; the ``Kernel`` objects keep
the reference's contiguous shapes and grid.
"""

from __future__ import annotations

import ctypes
import threading
from functools import lru_cache
from typing import Any

import numpy as np
import torch

from qpu_xla_amd import _lib
from qpu_xla_amd._tensors import PACKED_WORD_DTYPES, ptr, require_gpu, row_stride, rows_are_dense, stream_handle
from qpu_xla_amd.errors import KernelError
from qpu_xla_amd.kernel import Kernel

Q8_0_BLOCK_ELEMENTS = 32
Q8_0_BLOCK_BYTES = 34
TABLE_ENTRIES = 1 << 16

_TABLE_DTYPES = (torch.uint16, torch.int16)
_HALF_SCALE_DTYPES = (torch.uint16, torch.int16)


@lru_cache(maxsize=1)
def _host_table() -> np.ndarray:
    table = np.empty(TABLE_ENTRIES, dtype=np.uint16)
    _lib.call("qxt_ggml_gelu_fp16_table", table.ctypes.data_as(ctypes.c_void_p))
    table.flags.writeable = False
    return table


def ggml_gelu_fp16_table(device: torch.device | str | None = None) -> torch.Tensor:
    """The exact-GELU fp16 table as uint16 [65536] on ``device`` (CPU by default).

    Entry ``i`` is ``fp16(fl32(0.5 x (1 + erf(x / sqrt 2))))`` for ``x`` the
    fp16 value with bits ``i`` (``ggml_geglu_q8.py:26-34``).
    """
    host = torch.from_numpy(_host_table().view(np.int16).copy())
    if device is not None and torch.device(device).type != "cpu":
        host = host.to(device)
    return host.view(torch.uint16)


_device_tables: dict[torch.device, torch.Tensor] = {}
_device_lock = threading.Lock()


def _device_table(device: torch.device) -> torch.Tensor:
    with _device_lock:
        table = _device_tables.get(device)
        if table is None:
            table = ggml_gelu_fp16_table(device)
            _device_tables[device] = table
        return table


def _is_table(t: Any) -> bool:
    return (
        isinstance(t, torch.Tensor)
        and t.dtype in _TABLE_DTYPES
        and tuple(t.shape) == (TABLE_ENTRIES,)
        and t.is_contiguous()
    )


def _gate_up_shape(gate: Any, up: Any) -> tuple[int, int] | None:
    if not all(isinstance(t, torch.Tensor) for t in (gate, up)):
        return None
    if gate.dtype != torch.float32 or up.dtype != torch.float32 or gate.dim() != 2 or gate.shape != up.shape:
        return None
    rows, columns = gate.shape
    if rows <= 0 or columns <= 0 or columns % Q8_0_BLOCK_ELEMENTS:
        return None
    return int(rows), int(columns)


def supports_ggml_geglu_q8_0(gate: Any, up: Any, destination: Any, gelu_table: Any) -> bool:
    """Contract of the fused producer (``ggml_geglu_q8.py:239-259``) on HIP tensors."""
    shape = _gate_up_shape(gate, up)
    if shape is None or not isinstance(destination, torch.Tensor) or not _is_table(gelu_table):
        return False
    rows, columns = shape
    expected = (rows, columns // Q8_0_BLOCK_ELEMENTS, Q8_0_BLOCK_BYTES)
    if destination.dtype != torch.uint8 or tuple(destination.shape) != expected:
        return False
    tensors = (gate, up, destination, gelu_table)
    if not all(t.is_contiguous() for t in tensors):
        return False
    return all(t.is_cuda for t in tensors) and len({t.device for t in tensors}) == 1


def supports_ggml_geglu_q8_0_split(gate: Any, up: Any, scales: Any, values: Any, gelu_table: Any) -> bool:
    """Contract of the split producer (``ggml_geglu_q8.py:311-335``) on HIP tensors.

    Scales are uint32/int32 words as in the reference, or 2-byte halves.
    """
    shape = _gate_up_shape(gate, up)
    if shape is None or not all(isinstance(t, torch.Tensor) for t in (scales, values)) or not _is_table(gelu_table):
        return False
    rows, columns = shape
    if scales.dtype not in PACKED_WORD_DTYPES + _HALF_SCALE_DTYPES or values.dtype not in (torch.uint8, torch.int8):
        return False
    if tuple(scales.shape) != (rows, columns // Q8_0_BLOCK_ELEMENTS) or tuple(values.shape) != (rows, columns):
        return False
    tensors = (gate, up, scales, values, gelu_table)
    if not all(t.is_contiguous() for t in tensors):
        return False
    return all(t.is_cuda for t in tensors) and len({t.device for t in tensors}) == 1


def _launch(gate, up, destination, table, stream) -> None:
    rows, columns = gate.shape
    _lib.call(
        "qxt_ggml_geglu_q8_0",
        ptr(gate), row_stride(gate), ptr(up), row_stride(up), ptr(table), ptr(destination), row_stride(destination),
        rows, columns, stream_handle(stream),
    )


def _launch_split(gate, up, scales, values, table, stream) -> None:
    rows, columns = gate.shape
    _lib.call(
        "qxt_ggml_geglu_q8_0_split",
        ptr(gate), row_stride(gate), ptr(up), row_stride(up), ptr(table), ptr(scales), row_stride(scales),
        scales.element_size(), ptr(values), row_stride(values), rows, columns, stream_handle(stream),
    )


def _execute_ggml_geglu_q8_0(stream: Any, args: tuple[Any, ...], grid: tuple[int, int, int]) -> None:
    if len(args) != 4 or not all(isinstance(a, torch.Tensor) for a in args):
        raise KernelError("fused GEGLU-Q8_0 expects (gate, up, destination, gelu_table)")
    gate, up, destination, table = args
    if not supports_ggml_geglu_q8_0(gate, up, destination, table):
        raise KernelError("fused GEGLU-Q8_0 requires contiguous MxK F32 and Mx(K/32)x34 output")
    want = (destination.shape[1], destination.shape[0], 1)
    if tuple(grid) != want:
        raise KernelError(f"fused GEGLU-Q8_0 grid must be {want}, got {tuple(grid)}")
    _launch(gate, up, destination, table, stream)


GGML_GEGLU_Q8_0_KERNEL = Kernel("gfx950.ggml_geglu_q8_0", _execute_ggml_geglu_q8_0)


def _execute_ggml_geglu_q8_0_split(stream: Any, args: tuple[Any, ...], grid: tuple[int, int, int]) -> None:
    if len(args) != 5 or not all(isinstance(a, torch.Tensor) for a in args):
        raise KernelError("split GEGLU-Q8_0 expects gate, up, scales, values, and table")
    gate, up, scales, values, table = args
    if not supports_ggml_geglu_q8_0_split(gate, up, scales, values, table):
        raise KernelError("split GEGLU-Q8_0 requires contiguous MxK tensors")
    want = (scales.shape[1], scales.shape[0], 1)
    if tuple(grid) != want:
        raise KernelError(f"split GEGLU-Q8_0 grid must be {want}, got {tuple(grid)}")
    _launch_split(gate, up, scales, values, table, stream)


GGML_GEGLU_Q8_0_SPLIT_KERNEL = Kernel("gfx950.ggml_geglu_q8_0_split", _execute_ggml_geglu_q8_0_split)


def _check_inputs(name: str, gate: torch.Tensor, up: torch.Tensor) -> tuple[int, int]:
    shape = _gate_up_shape(gate, up)
    if shape is None:
        raise ValueError(f"{name}: gate/up must be equal rank-two float32 tensors with K divisible by 32")
    if not (rows_are_dense(gate) and rows_are_dense(up)):
        raise ValueError(f"{name}: gate/up rows must be contiguous")
    return shape


def _resolve_table(name: str, gelu_table: torch.Tensor | None, device: torch.device) -> torch.Tensor:
    if gelu_table is None:
        return _device_table(device)
    if not _is_table(gelu_table):
        raise ValueError(f"{name}: gelu_table must be a contiguous uint16 [65536] tensor")
    return gelu_table


def ggml_geglu_q8_0(
    gate: torch.Tensor,
    up: torch.Tensor,
    gelu_table: torch.Tensor | None = None,
    destination: torch.Tensor | None = None,
    *,
    stream: Any = None,
) -> torch.Tensor:
    """Functional form: native Q8_0 blocks uint8 [M, K/32, 34] of GEGLU(gate, up)."""
    rows, columns = _check_inputs("ggml_geglu_q8_0", gate, up)
    table = _resolve_table("ggml_geglu_q8_0", gelu_table, gate.device)
    shape = (rows, columns // Q8_0_BLOCK_ELEMENTS, Q8_0_BLOCK_BYTES)
    if destination is None:
        destination = torch.empty(shape, dtype=torch.uint8, device=gate.device)
    elif destination.dtype != torch.uint8 or tuple(destination.shape) != shape or not rows_are_dense(destination):
        raise ValueError("ggml_geglu_q8_0: destination must be uint8 [M, K/32, 34] with contiguous rows")
    require_gpu("ggml_geglu_q8_0", gate, up, table, destination)
    _launch(gate, up, destination, table, stream)
    return destination


def ggml_geglu_q8_0_split(
    gate: torch.Tensor,
    up: torch.Tensor,
    gelu_table: torch.Tensor | None = None,
    scales: torch.Tensor | None = None,
    values: torch.Tensor | None = None,
    *,
    stream: Any = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Functional form: (fp16 scale bits [M, K/32] as uint32 words by default, int8 values [M, K])."""
    rows, columns = _check_inputs("ggml_geglu_q8_0_split", gate, up)
    table = _resolve_table("ggml_geglu_q8_0_split", gelu_table, gate.device)
    blocks = columns // Q8_0_BLOCK_ELEMENTS
    if scales is None:
        scales = torch.empty((rows, blocks), dtype=torch.int32, device=gate.device)
    elif scales.dtype not in PACKED_WORD_DTYPES + _HALF_SCALE_DTYPES or tuple(scales.shape) != (rows, blocks):
        raise ValueError("ggml_geglu_q8_0_split: scales must be 2- or 4-byte integers [M, K/32]")
    if values is None:
        values = torch.empty((rows, columns), dtype=torch.int8, device=gate.device)
    elif values.dtype not in (torch.uint8, torch.int8) or tuple(values.shape) != (rows, columns):
        raise ValueError("ggml_geglu_q8_0_split: values must be int8/uint8 [M, K]")
    if not (rows_are_dense(scales) and rows_are_dense(values)):
        raise ValueError("ggml_geglu_q8_0_split: scales/values rows must be contiguous")
    require_gpu("ggml_geglu_q8_0_split", gate, up, table, scales, values)
    _launch_split(gate, up, scales, values, table, stream)
    return scales, values


__all__ = [
    "GGML_GEGLU_Q8_0_KERNEL",
    "GGML_GEGLU_Q8_0_SPLIT_KERNEL",
    "ggml_geglu_q8_0",
    "ggml_geglu_q8_0_split",
    "ggml_gelu_fp16_table",
    "supports_ggml_geglu_q8_0",
    "supports_ggml_geglu_q8_0_split",
]
