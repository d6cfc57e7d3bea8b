"""Dynamic W8A8 linear on the GPU placement.

Host-side mirror of the reference's W8A8 contract owner,
``src/qpu_xla/models/tinyllama/quantization.py``:

* ``QuantizedMatrixInt8`` (``:31-54``) -- int8 values [N, K] plus one fp32
  scale per output channel, here as HIP device tensors;
* ``quantize_per_output_channel_int8`` (``:1085-1092``) -- same rule
  (``scale = max(absmax/127, 1/127)``, ``rint(w / scale)`` clipped to +-127),
  run by the per-row GPU quantiser;
* ``w8a8_linear`` -- the whole dynamic operator (per-row activation
  quantisation, int8 MFMA GEMM, fused dequant + bias) as two kernels;
* ``PreparedW8A8Linear`` (``:57-330``) -- a persistent plan owning the
  device weights and the activation workspace, bound to its first queue and
  allowing one in-flight invocation, as the reference plan does.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from qpu_xla_amd import _lib
from qpu_xla_amd._tensors import ptr, require_gpu, row_stride, rows_are_dense, stream_handle
from qpu_xla_amd.errors import DependencyError
from qpu_xla_amd.kernels.quantize import quantize_rows_int8
from qpu_xla_amd.queue import Event, Queue

INT32_MAX = 2**31 - 1


@dataclass(frozen=True)
class QuantizedMatrixInt8:
    """Row-wise symmetric int8 matrix [N, K] plus one fp32 scale per row (device tensors)."""

    values: torch.Tensor
    scales: torch.Tensor

    def __post_init__(self) -> None:
        if self.values.dim() != 2 or self.scales.dim() != 1 or self.scales.shape[0] != self.values.shape[0]:
            raise ValueError("quantized matrix values must be rank-2 with one scale per output row")
        if self.values.dtype != torch.int8 or self.scales.dtype != torch.float32:
            raise ValueError("quantized matrix values must be int8 and scales float32")
        if not self.values.is_contiguous() or not self.scales.is_contiguous():
            raise ValueError("quantized matrix values and scales must be contiguous")

    @property
    def shape(self) -> tuple[int, int]:
        return (int(self.values.shape[0]), int(self.values.shape[1]))

    def dequantize(self) -> torch.Tensor:
        return self.values.to(torch.float32) * self.scales[:, None]


def quantize_per_output_channel_int8(weight: torch.Tensor, *, stream: Any = None) -> QuantizedMatrixInt8:
    """Symmetrically quantise fp32 ``(output, input)`` weights to int8 rows on the GPU."""
    if weight.dim() != 2 or weight.dtype != torch.float32:
        raise ValueError("quantize_per_output_channel_int8 requires a rank-2 float32 matrix")
    values, scales = quantize_rows_int8(weight.contiguous(), floor=True, stream=stream)
    return QuantizedMatrixInt8(values, scales)


def _padded(k: int) -> int:
    return (k + 15) // 16 * 16


def w8a8_linear(
    x: torch.Tensor,
    weight: QuantizedMatrixInt8,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    *,
    floor: bool = True,
    workspace: tuple[torch.Tensor, torch.Tensor] | None = None,
    stream: Any = None,
) -> torch.Tensor:
    """Dynamic W8A8 linear ``y = dequant(quant_rows(x) @ W.T) + bias`` (fp32 [M, N]).

    ``workspace`` = (int8 [>= M, >= K], fp32 [>= M]) avoids allocating the
    quantised activation; K must be a multiple of 16 (pad the weight
    otherwise, as the reference plan does).
    """
    if x.dtype != torch.float32 or x.dim() != 2 or not rows_are_dense(x):
        raise ValueError("w8a8_linear: float32 [M, K] activations with contiguous rows are required")
    m, k = x.shape
    n, k2 = weight.shape
    if k != k2:
        raise ValueError("w8a8_linear: activation and weight reduction extents differ")
    if k % 16:
        raise ValueError("w8a8_linear: K must be a multiple of 16 (pad the weight, as PreparedW8A8Linear does)")
    if k * 127 * 127 > INT32_MAX:
        raise ValueError("w8a8_linear: accumulation can overflow int32")
    if bias is not None and (bias.dtype != torch.float32 or tuple(bias.shape) != (n,) or not bias.is_contiguous()):
        raise ValueError("w8a8_linear: bias must be contiguous float32 [N]")
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=x.device)
    if workspace is None:
        qa = torch.empty((m, k), dtype=torch.int8, device=x.device)
        sa = torch.empty((m,), dtype=torch.float32, device=x.device)
    else:
        qa, sa = workspace
        if qa.dtype != torch.int8 or qa.shape[0] < m or qa.shape[1] < k or sa.dtype != torch.float32 or sa.shape[0] < m:
            raise ValueError("w8a8_linear: workspace too small")
    require_gpu("w8a8_linear", x, weight.values, weight.scales, bias, out, qa, sa)
    flags = 0 if floor else _lib.QUANT_NO_SCALE_FLOOR
    _lib.call(
        "qxt_w8a8_linear",
        ptr(x), row_stride(x), ptr(qa), row_stride(qa), ptr(sa),
        ptr(weight.values), row_stride(weight.values), ptr(weight.scales), ptr(bias),
        ptr(out), row_stride(out), m, n, k, _lib.WEIGHT_NK, flags, stream_handle(stream),
    )
    return out


class PreparedW8A8Linear:
    """Persistent W8A8 projection plan on the GPU placement.

    Owns the weight (padded to a multiple of 16 along K, zero columns), an
    optional bias and the activation workspace for up to ``max_batch`` rows.
    ``execute`` quantises the fp32 source per row on the GPU and runs the
    fused MFMA GEMM + dequant (+ bias) epilogue on the queue's stream.  The
    plan binds to its first queue and allows one in-flight invocation
    (``quantization.py:288-295``), because the workspace is reused.
    """

    def __init__(self, weight: QuantizedMatrixInt8, *, max_batch: int, bias: torch.Tensor | None = None) -> None:
        if max_batch <= 0:
            raise ValueError("PreparedW8A8Linear max_batch must be positive")
        outputs, features = weight.shape
        self.max_batch = max_batch
        self.features = features
        self.outputs = outputs
        self.padded_features = _padded(features)
        if self.padded_features * 127 * 127 > INT32_MAX:
            raise ValueError("prepared W8A8 linear accumulation can overflow int32")
        device = weight.values.device
        if device.type != "cuda":
            raise ValueError("PreparedW8A8Linear requires weights on a HIP device (no CPU fallback)")
        values = torch.zeros((outputs, self.padded_features), dtype=torch.int8, device=device)
        values[:, :features] = weight.values
        self.weight = QuantizedMatrixInt8(values, weight.scales.contiguous())
        self.bias = None if bias is None else bias.to(device=device, dtype=torch.float32).contiguous()
        if self.bias is not None and tuple(self.bias.shape) != (outputs,):
            raise ValueError("bias must have one value per output channel")
        self._source = torch.zeros((max_batch, self.padded_features), dtype=torch.float32, device=device)
        self._qa = torch.zeros((max_batch, self.padded_features), dtype=torch.int8, device=device)
        self._sa = torch.zeros((max_batch,), dtype=torch.float32, device=device)
        self._queue: Queue | None = None
        self._last_event: Event | None = None
        self._closed = False

    def __enter__(self) -> "PreparedW8A8Linear":
        if self._closed:
            raise RuntimeError("prepared W8A8 linear plan is closed")
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def close(self) -> None:
        if self._closed:
            return
        if self._last_event is not None:
            self._last_event.wait()
        self._closed = True

    def execute(self, destination: torch.Tensor, source: torch.Tensor, *, queue: Queue, wait_for=()) -> Event:
        """Submit quantise + GEMM + epilogue; returns the completion event."""
        if self._closed:
            raise RuntimeError("prepared W8A8 linear plan is closed")
        if self._last_event is not None and not self._last_event.done:
            raise RuntimeError("prepared W8A8 linear plan already has an in-flight invocation")
        if self._queue is None:
            self._queue = queue
        elif self._queue is not queue:
            raise DependencyError("prepared W8A8 linear plan is bound to its first submission queue")
        if source.dtype != torch.float32 or destination.dtype != torch.float32:
            raise ValueError("prepared W8A8 linear requires float32 source and destination")
        if source.dim() != 2 or destination.dim() != 2:
            raise ValueError("prepared W8A8 linear requires rank-2 source and destination")
        batch, features = source.shape
        if batch > self.max_batch or features != self.features:
            raise ValueError("prepared W8A8 linear source exceeds the plan shape")
        if tuple(destination.shape) != (batch, self.outputs):
            raise ValueError("prepared W8A8 linear destination shape does not align")
        if source.device != self.weight.values.device or destination.device != self.weight.values.device:
            raise DependencyError("prepared W8A8 linear tensors must live on the plan device")
        queue._wait_dependencies(wait_for)
        with torch.cuda.stream(queue.stream):
            if self.padded_features != features or not rows_are_dense(source):
                staged = self._source[:batch]
                staged[:, :features].copy_(source)
                src = staged
            else:
                src = source
            w8a8_linear(
                src, self.weight, self.bias, destination,
                workspace=(self._qa, self._sa), stream=queue,
            )
            hip_event = torch.cuda.Event()
            hip_event.record(queue.stream)
        self._last_event = Event(queue, "gfx950.w8a8_linear", "gpu", hip_event)
        return self._last_event
