"""Dynamic W8A8 linear on the GPU placement.

Host-side mirror of the reference's W8A8 contract owner,
``src/qpu_xla/models/tinyllama/quantization.py``:

* ``QuantizedMatrixInt8`` (``:31-54``) -- int8 values [N, K] plus one fp32
  scale per output channel, here as HIP device tensors;
* ``quantize_per_output_channel_int8`` (``:1085-1092``) -- same rule
  (``scale = max(absmax/127, 1/127)``, ``rint(w / scale)`` clipped to +-127),
  run by the per-row GPU quantiser;
* ``w8a8_linear`` -- the whole dynamic operator (per-row activation
  quantisation, int8 MFMA GEMM or dot4 GEMV, fused dequant + bias);
* ``PreparedW8A8Linear`` (``:57-878``) -- a persistent plan owning the
  device weights and the activation workspace, bound to its first queue and
  allowing one in-flight invocation, as the reference plan does; its
  partitioned ("hybrid") forms split rows or output columns between two
  queues, both on the GPU;
* ``CalibratedW8A8Linear`` (``:881-1082``) -- dispatches only measured
  ``supported-win`` candidates of the exact shape class from a
  ``CandidateRegistry``.  There is no CPU reference path: a shape without a
  GPU or hybrid winner raises instead of running on the host.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from qpu_xla_amd import _lib
from qpu_xla_amd._tensors import ptr, require_gpu, row_stride, rows_are_dense, stream_handle
from qpu_xla_amd.candidates import CandidateRecord, CandidateRegistry
from qpu_xla_amd.errors import DependencyError
from qpu_xla_amd.kernels.gemm_int8 import w8a8_gemm_dequantize
from qpu_xla_amd.kernels.quantize import quantize_rows_int8
from qpu_xla_amd.placement import Placement
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


PARTITION_ALIGNMENT = 16
LINEAR_OPERATION = "linear"
W8A8_DTYPE = "w8a8-i32-fp32"
# int8 [N, K] rows are byte-identical to the reference's packed-K4 words.
W8A8_LAYOUT = "row-major-packed-k4"


def w8a8_shape_class(batch: int, features: int, outputs: int) -> str:
    """Shape-class key of a W8A8 linear record: ``"{M}x{K}x{N}"``."""
    return f"{batch}x{features}x{outputs}"


class PreparedW8A8Linear:
    """Persistent W8A8 projection plan on the GPU placement.

    Owns the weight (padded to a multiple of 16 along K, zero columns), an
    optional bias and the activation workspace for up to ``max_batch`` rows.
    ``execute`` quantises the fp32 source per row on the GPU and runs the
    int8 GEMM (dot4 GEMV for M <= 4) with the fused dequant (+ bias)
    epilogue on the queue's stream.  The plan binds to its first queue and
    allows one in-flight invocation (``quantization.py:288-295``), because
    the workspace is reused.

    ``execute_hybrid`` / ``execute_hybrid_rows`` keep the reference's
    partition contract (``quantization.py:350-662``): an aligned prefix of
    output columns or rows goes to ``qpu_queue`` and the disjoint tail to
    ``cpu_queue``.  Here both queues are HIP streams of the same GPU -- the
    tail is not computed on the host -- so each partition is exactly the
    work one device of a sharded deployment would run; results are
    bit-identical to ``execute``.
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
        self.device = device
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
        self._second_queue: Queue | None = None
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

    @property
    def activation_workspace(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(int8 [max_batch, padded K], fp32 [max_batch]) read by ``execute_prepared``."""
        return self._qa, self._sa

    # ------------------------------------------------------------ validation

    def _begin(self) -> None:
        if self._closed:
            raise RuntimeError("prepared W8A8 linear plan is closed")
        if self._last_event is not None and not self._last_event.done:
            raise RuntimeError("prepared W8A8 linear plan already has an in-flight invocation")

    def _bind(self, queue: Queue, second: Queue | None = None) -> None:
        if second is not None and second is queue:
            raise DependencyError("hybrid W8A8 linear requires two distinct queues")
        for q in (queue, second):
            if q is not None and q.device != self.device:
                raise DependencyError("prepared W8A8 linear queues must belong to the plan device")
        if self._queue is None:
            self._queue = queue
        elif self._queue is not queue:
            raise DependencyError("prepared W8A8 linear plan is bound to its first submission queue")
        if second is not None:
            if self._second_queue is None:
                self._second_queue = second
            elif self._second_queue is not second:
                raise DependencyError("prepared W8A8 linear plan is bound to its first partition queue")

    def _check_io(self, destination: torch.Tensor, source: torch.Tensor) -> int:
        if source.dtype != torch.float32 or destination.dtype != torch.float32:
            raise ValueError("prepared W8A8 linear requires float32 source and destination")
        if source.dim() != 2 or destination.dim() != 2:
            raise ValueError("prepared W8A8 linear requires rank-2 source and destination")
        batch, features = source.shape
        if batch <= 0 or batch > self.max_batch or features != self.features:
            raise ValueError("prepared W8A8 linear source exceeds the plan shape")
        if tuple(destination.shape) != (batch, self.outputs):
            raise ValueError("prepared W8A8 linear destination shape does not align")
        if source.device != self.device or destination.device != self.device:
            raise DependencyError("prepared W8A8 linear tensors must live on the plan device")
        return batch

    def _staged(self, source: torch.Tensor) -> tuple[torch.Tensor, bool]:
        """(rows the kernels read, whether ``source`` must first be copied into them).

        Rows already dense with the padded K are read in place; otherwise they
        are copied into the plan's source buffer (whose padding is zero).
        """
        if self.padded_features == self.features and rows_are_dense(source):
            return source, False
        return self._source[: source.shape[0]], True

    def _stage(self, staged: torch.Tensor, source: torch.Tensor) -> None:
        """Copy ``source`` into the plan's source buffer, on the current stream."""
        staged[:, : self.features].copy_(source)

    # ------------------------------------------------------------- execution
    #
    # Each step is one Queue.launch: it runs in the queue's order (held while
    # host work submitted earlier is pending), its event carries the step's
    # status and device timestamps, and a failure inside it fails the event.

    def execute(self, destination: torch.Tensor, source: torch.Tensor, *, queue: Queue, wait_for=()) -> Event:
        """Submit quantise + GEMM + epilogue; returns the completion event."""
        self._begin()
        self._bind(queue)
        self._check_io(destination, source)
        src, copy = self._staged(source)

        def issue() -> None:
            with torch.cuda.stream(queue.stream):
                if copy:
                    self._stage(src, source)
                w8a8_linear(src, self.weight, self.bias, destination, workspace=(self._qa, self._sa), stream=queue)

        self._last_event = queue.launch("gfx950.w8a8_linear", issue, tensors=(destination, source), wait_for=wait_for)
        return self._last_event

    def execute_prepared(self, destination: torch.Tensor, *, batch: int, queue: Queue, wait_for=()) -> Event:
        """GEMM + epilogue over an activation already quantised into ``activation_workspace``.

        Mirrors ``execute_prepared`` (``quantization.py:326-347``): an
        enclosing stage wrote ``batch`` int8 rows (zero-padded to the padded
        K) and their scales; ``wait_for`` orders this launch after it.
        """
        self._begin()
        self._bind(queue)
        if destination.dtype != torch.float32 or destination.dim() != 2:
            raise ValueError("prepared W8A8 linear destination must be rank-2 float32")
        if batch <= 0 or batch > self.max_batch or tuple(destination.shape) != (batch, self.outputs):
            raise ValueError("prepared W8A8 linear destination shape does not align")
        if destination.device != self.device:
            raise DependencyError("prepared W8A8 linear destination must live on the plan device")

        def issue() -> None:
            with torch.cuda.stream(queue.stream):
                w8a8_gemm_dequantize(
                    self._qa[:batch], self.weight.values, self._sa, self.weight.scales, self.bias, destination,
                    stream=queue,
                )

        self._last_event = queue.launch("gfx950.w8a8_gemm_dequantize", issue, tensors=(destination,),
                                        wait_for=wait_for)
        return self._last_event

    def execute_hybrid(
        self,
        destination: torch.Tensor,
        source: torch.Tensor,
        *,
        qpu_queue: Queue,
        cpu_queue: Queue,
        qpu_outputs: int,
        wait_for=(),
    ) -> Event:
        """Output columns [0, qpu_outputs) on ``qpu_queue``, the rest on ``cpu_queue`` (both GPU streams).

        The activation is quantised once on ``qpu_queue``; the second queue
        waits for it, then both run the fused GEMM over their column range.
        The returned event (on ``qpu_queue``) completes after both.
        """
        self._begin()
        batch = self._check_io(destination, source)
        if qpu_outputs <= 0 or qpu_outputs >= self.outputs or qpu_outputs % PARTITION_ALIGNMENT:
            raise ValueError("hybrid W8A8 qpu_outputs must be aligned and leave a non-empty tail")
        self._bind(qpu_queue, cpu_queue)
        split = int(qpu_outputs)
        src = source if rows_are_dense(source) else self._source[:batch, : self.features]

        def quantize() -> None:
            with torch.cuda.stream(qpu_queue.stream):
                if src is not source:
                    src.copy_(source)
                # The quantiser zero-fills the padded K columns of the workspace.
                quantize_rows_int8(src, padded_columns=self.padded_features, out=self._qa, scales=self._sa,
                                   stream=qpu_queue)

        def part(queue: Queue, cols: slice):
            def issue() -> None:
                with torch.cuda.stream(queue.stream):
                    w8a8_gemm_dequantize(
                        self._qa[:batch], self.weight.values[cols], self._sa, self.weight.scales[cols],
                        None if self.bias is None else self.bias[cols], destination[:, cols], stream=queue,
                    )
            return issue

        quantized = qpu_queue.launch("gfx950.quantize_rows_int8", quantize, tensors=(destination, source),
                                     wait_for=wait_for)
        qpu_queue.launch("gfx950.w8a8_gemm_dequantize", part(qpu_queue, slice(0, split)))
        tail = cpu_queue.launch("gfx950.w8a8_gemm_dequantize", part(cpu_queue, slice(split, self.outputs)),
                                tensors=(destination, source), wait_for=(quantized, *wait_for))
        self._last_event = qpu_queue.launch("gfx950.w8a8_linear.hybrid_join", lambda: None, wait_for=(tail,))
        return self._last_event

    def execute_hybrid_rows(
        self,
        destination: torch.Tensor,
        source: torch.Tensor,
        *,
        qpu_queue: Queue,
        cpu_queue: Queue,
        qpu_rows: int,
        wait_for=(),
    ) -> Event:
        """Rows [0, qpu_rows) on ``qpu_queue``, the rest on ``cpu_queue`` (both GPU streams).

        Per-row quantisation makes the row partitions independent: each
        queue runs the whole operator on its rows with its own slice of the
        workspace.  The returned event (on ``qpu_queue``) completes after both.
        """
        self._begin()
        batch = self._check_io(destination, source)
        if qpu_rows <= 0 or qpu_rows >= batch or qpu_rows % PARTITION_ALIGNMENT:
            raise ValueError("hybrid W8A8 qpu_rows must be aligned and leave a non-empty tail")
        self._bind(qpu_queue, cpu_queue)
        split = int(qpu_rows)
        src, copy = self._staged(source)

        def rows_of(queue: Queue, rows: slice):
            def issue() -> None:
                with torch.cuda.stream(queue.stream):
                    w8a8_linear(src[rows], self.weight, self.bias, destination[rows],
                                workspace=(self._qa[rows], self._sa[rows]), stream=queue)
            return issue

        ready = tuple(wait_for)
        if copy:
            # The staged copy is made once, on the first queue; the second waits for it.
            def stage() -> None:
                with torch.cuda.stream(qpu_queue.stream):
                    self._stage(src, source)

            ready = (qpu_queue.launch("gfx950.stage_source", stage, tensors=(destination, source),
                                      wait_for=wait_for),)
        qpu_queue.launch("gfx950.w8a8_linear", rows_of(qpu_queue, slice(0, split)), tensors=(destination, source),
                         wait_for=ready)
        tail = cpu_queue.launch("gfx950.w8a8_linear", rows_of(cpu_queue, slice(split, batch)),
                                tensors=(destination, source), wait_for=ready)
        self._last_event = qpu_queue.launch("gfx950.w8a8_linear.hybrid_join", lambda: None, wait_for=(tail,))
        return self._last_event


# --------------------------------------------------------- calibrated dispatch


@dataclass(frozen=True)
class W8A8Dispatch:
    """Outcome of candidate selection: where one call runs and on which record."""

    placement: Placement
    record: CandidateRecord

    @property
    def axis(self) -> str | None:
        return None if self.record.partition is None else self.record.partition.axis

    @property
    def units(self) -> int | None:
        return None if self.record.partition is None else self.record.partition.qpu_units


def _fastest(records: tuple[CandidateRecord, ...] | list[CandidateRecord]) -> CandidateRecord:
    def median_seconds(record: CandidateRecord) -> float:
        return float("inf") if record.performance is None else record.performance.candidate_median_seconds

    return min(records, key=median_seconds)


def select_w8a8_dispatch(
    candidates: CandidateRegistry,
    *,
    batch: int,
    features: int,
    outputs: int,
    placement: Placement = Placement.AUTO,
    qpu_rows: int | None = None,
    qpu_outputs: int | None = None,
    partition_queue: bool = False,
) -> W8A8Dispatch:
    """Pick the exact-shape ``supported-win`` record a W8A8 call runs on.

    Same rules as ``CalibratedW8A8Linear.execute`` (``quantization.py:966-1060``)
    with the GPU in the accelerator's place: ``Placement.GPU`` needs a
    ``"gpu"`` record, ``HYBRID`` a ``"hybrid"`` record whose partition matches
    the requested axis/size and a second queue, ``AUTO`` takes the fastest
    executable record by median candidate time.  ``"qpu"`` records are
    VideoCore measurements and never run here.  Where the reference falls
    back to its CPU reference, this raises ``ValueError``.
    """
    if qpu_rows is not None and qpu_outputs is not None:
        raise ValueError("qpu_rows and qpu_outputs are mutually exclusive")
    partitioned = qpu_rows is not None or qpu_outputs is not None
    if placement in {Placement.CPU, Placement.QPU, Placement.GPU} and partitioned:
        raise ValueError("hybrid partitions require HYBRID or AUTO placement")
    if placement is Placement.CPU:
        raise ValueError("the gfx950 library has no CPU placement for W8A8 linear; use GPU, HYBRID or AUTO")
    if placement is Placement.QPU:
        raise ValueError("the VideoCore QPU placement does not exist on gfx950; use Placement.GPU")
    exact = candidates.supported_for(
        operation=LINEAR_OPERATION, dtype=W8A8_DTYPE, layout=W8A8_LAYOUT,
        shape_class=w8a8_shape_class(batch, features, outputs),
    )
    gpu_records = tuple(r for r in exact if r.placement == Placement.GPU.value)

    def matches(record: CandidateRecord) -> bool:
        part = record.partition
        if part is None:
            return False
        if qpu_rows is not None:
            return part.axis == "rows" and part.qpu_units == qpu_rows
        if qpu_outputs is not None:
            return part.axis == "outputs" and part.qpu_units == qpu_outputs
        return part.axis in ("rows", "outputs")

    hybrid_records = tuple(r for r in exact if r.placement == Placement.HYBRID.value and matches(r))
    hybrid_ok = bool(hybrid_records) and partition_queue
    if placement is Placement.GPU:
        if not gpu_records:
            raise ValueError("no measured supported-win W8A8 GPU candidate exists for this exact shape")
        return W8A8Dispatch(Placement.GPU, _fastest(gpu_records))
    if placement is Placement.HYBRID:
        if not hybrid_ok:
            raise ValueError("no executable supported-win W8A8 hybrid candidate exists for this exact shape")
        return W8A8Dispatch(Placement.HYBRID, _fastest(hybrid_records))
    if partitioned and not hybrid_ok:
        raise ValueError("no supported W8A8 hybrid partition matches the requested axis and size")
    executable = [*(() if partitioned else gpu_records), *(hybrid_records if hybrid_ok else ())]
    if not executable:
        raise ValueError(
            f"no measured supported-win W8A8 GPU or hybrid candidate for shape "
            f"{w8a8_shape_class(batch, features, outputs)}; this library has no CPU reference fallback"
        )
    record = _fastest(executable)
    return W8A8Dispatch(Placement(record.placement), record)


class CalibratedW8A8Linear:
    """Dispatch a W8A8 linear only to measured GPU (or partitioned GPU) winners.

    Mirrors ``CalibratedW8A8Linear`` (``quantization.py:881-1062``):
    ``execute`` validates the call, picks the exact-shape winner with
    ``select_w8a8_dispatch`` and runs it through a ``PreparedW8A8Linear``,
    which is created only when the registry holds a GPU or hybrid winner for
    some batch size up to ``max_batch``.
    """

    def __init__(
        self,
        weight: QuantizedMatrixInt8,
        *,
        max_batch: int,
        candidates: CandidateRegistry,
        bias: torch.Tensor | None = None,
    ) -> None:
        if max_batch <= 0:
            raise ValueError("calibrated W8A8 linear max_batch must be positive")
        self.weight = weight
        self.max_batch = max_batch
        self.candidates = candidates
        outputs, features = weight.shape
        wanted = {w8a8_shape_class(b, features, outputs) for b in range(1, max_batch + 1)}
        executable = any(
            r.placement in (Placement.GPU.value, Placement.HYBRID.value)
            and (r.operation, r.dtype, r.layout) == (LINEAR_OPERATION, W8A8_DTYPE, W8A8_LAYOUT)
            and r.shape_class in wanted
            for r in candidates.supported
        )
        self._gpu = PreparedW8A8Linear(weight, max_batch=max_batch, bias=bias) if executable else None
        self.last_dispatch: W8A8Dispatch | None = None
        self._closed = False

    def __enter__(self) -> "CalibratedW8A8Linear":
        if self._closed:
            raise RuntimeError("calibrated W8A8 linear is closed")
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def close(self) -> None:
        if self._closed:
            return
        if self._gpu is not None:
            self._gpu.close()
        self._closed = True

    def execute(
        self,
        destination: torch.Tensor,
        source: torch.Tensor,
        *,
        queue: Queue,
        cpu_queue: Queue | None = None,
        placement: Placement = Placement.AUTO,
        qpu_rows: int | None = None,
        qpu_outputs: int | None = None,
        wait_for=(),
    ) -> Event:
        """Run the exact-shape winner; ``cpu_queue`` is the second (GPU) queue of a partitioned run."""
        if self._closed:
            raise RuntimeError("calibrated W8A8 linear is closed")
        if source.dtype != torch.float32 or destination.dtype != torch.float32:
            raise ValueError("calibrated W8A8 linear requires FP32 source and destination")
        if source.dim() != 2 or destination.dim() != 2:
            raise ValueError("calibrated W8A8 linear requires rank-2 tensors")
        outputs, features = self.weight.shape
        batch = int(source.shape[0])
        if batch > self.max_batch or int(source.shape[1]) != features:
            raise ValueError("calibrated W8A8 source exceeds its planned shape")
        if tuple(destination.shape) != (batch, outputs):
            raise ValueError("calibrated W8A8 destination shape does not align")
        dispatch = select_w8a8_dispatch(
            self.candidates, batch=batch, features=features, outputs=outputs, placement=placement,
            qpu_rows=qpu_rows, qpu_outputs=qpu_outputs, partition_queue=cpu_queue is not None,
        )
        assert self._gpu is not None  # a winner for this batch exists, so the plan was prepared
        self.last_dispatch = dispatch
        if dispatch.placement is Placement.GPU:
            return self._gpu.execute(destination, source, queue=queue, wait_for=wait_for)
        assert cpu_queue is not None and dispatch.units is not None
        if dispatch.axis == "rows":
            return self._gpu.execute_hybrid_rows(
                destination, source, qpu_queue=queue, cpu_queue=cpu_queue, qpu_rows=dispatch.units, wait_for=wait_for,
            )
        return self._gpu.execute_hybrid(
            destination, source, qpu_queue=queue, cpu_queue=cpu_queue, qpu_outputs=dispatch.units, wait_for=wait_for,
        )
