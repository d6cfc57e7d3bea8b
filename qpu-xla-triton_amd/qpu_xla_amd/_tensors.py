"""Small helpers turning torch device tensors into C-ABI arguments."""

from __future__ import annotations

import ctypes
from typing import Any

import torch

PACKED_WORD_DTYPES = (torch.int32, torch.uint32)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def row_stride(t: torch.Tensor) -> int:
    """Byte distance between consecutive rows (dimension 0).

    A tensor with a single row may carry any stride for dimension 0 (torch and
    NumPy report 1 for transposed single-row views); its dense row length is
    the stride then, which is what the C ABI's stride checks expect.
    """
    stride = int(t.stride(0))
    if t.dim() >= 2 and t.shape[0] == 1:
        row = 1
        for extent in t.shape[1:]:
            row *= int(extent)
        stride = max(stride, row)
    return stride * t.element_size()


def rows_are_dense(t: torch.Tensor) -> bool:
    """Every row is contiguous in memory (the last dimensions are packed)."""
    if t.dim() <= 1:
        return t.dim() == 0 or t.stride(0) == 1
    return t[0].is_contiguous()


def stream_handle(stream: Any = None) -> ctypes.c_void_p:
    """HIP stream handle from a Queue, a torch stream, a raw int or None (current stream)."""
    if stream is None:
        return ctypes.c_void_p(int(torch.cuda.current_stream().cuda_stream))
    if hasattr(stream, "handle"):
        return ctypes.c_void_p(int(stream.handle))
    if isinstance(stream, torch.cuda.Stream):
        return ctypes.c_void_p(int(stream.cuda_stream))
    return ctypes.c_void_p(int(stream))


def on_gpu(*tensors: torch.Tensor | None) -> bool:
    devices = {t.device for t in tensors if t is not None}
    return len(devices) == 1 and next(iter(devices)).type == "cuda"


def require_gpu(name: str, *tensors: torch.Tensor | None) -> None:
    if not on_gpu(*tensors):
        raise ValueError(f"{name}: all tensors must live on one HIP device (no CPU fallback)")
