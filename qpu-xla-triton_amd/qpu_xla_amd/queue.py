"""In-order submission queue over one HIP stream.

The reference's ``Queue`` (``src/qpu_xla/queue.py:150-260``) is a single
worker thread that runs kernel executors and host tasks in order and returns
an ``Event`` per submission.  On the GPU the stream already is that in-order
worker, so this ``Queue`` enqueues each kernel on its HIP stream (through the
C ABI, no thread hop) and records a HIP event after it.  ``wait_for`` events
from other queues become stream waits.  ``host_task`` runs its callable on
the calling thread once its dependencies have completed.

Tensors cross from the caller's stream to the queue's the way torch expects
of a side stream: every submission first makes the queue's stream wait for
the caller's current stream (so an argument still being written there by
asynchronous work is complete before the queue reads it), and every tensor
argument is marked as used on the queue's stream (``record_stream``), so the
caching allocator does not hand its memory out again while the queue's work
on it is pending -- the caller may drop its references right after submit.
"""

from __future__ import annotations

import time
from collections.abc import Callable, Iterable
from typing import Any

import torch

from qpu_xla_amd._lib import call
from qpu_xla_amd.errors import DependencyError, EventTimeoutError
from qpu_xla_amd.kernel import Kernel, LaunchConfig


class Event:
    """Completion of one submission (kernel or host task)."""

    def __init__(self, queue: "Queue", name: str, category: str, hip_event: torch.cuda.Event | None) -> None:
        self.queue = queue
        self.name = name
        self.category = category
        self._hip_event = hip_event
        self.submitted_ns = time.perf_counter_ns()

    @property
    def done(self) -> bool:
        return True if self._hip_event is None else bool(self._hip_event.query())

    def wait(self, timeout: float | None = None) -> None:
        """Block until the submission finished (``timeout`` seconds at most)."""
        if self._hip_event is None:
            return
        if timeout is None:
            self._hip_event.synchronize()
            return
        deadline = time.monotonic() + timeout
        while not self._hip_event.query():
            if time.monotonic() > deadline:
                raise EventTimeoutError(f"event {self.name!r} did not complete within {timeout} s")
            time.sleep(20e-6)

    def hip_event(self) -> torch.cuda.Event | None:
        return self._hip_event


class Queue:
    """In-order queue bound to one device and one HIP stream."""

    def __init__(self, device: torch.device | int | str | None = None, stream: torch.cuda.Stream | None = None):
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
        self.stream = stream if stream is not None else torch.cuda.Stream(device=self.device)
        self._closed = False

    def __enter__(self) -> "Queue":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def close(self) -> None:
        if not self._closed:
            self.stream.synchronize()
            self._closed = True

    @property
    def handle(self) -> int:
        """The raw ``hipStream_t`` of this queue."""
        return int(self.stream.cuda_stream)

    def order_after_caller(self, tensors: Iterable[Any] = ()) -> None:
        """Order this queue after the caller's current stream; keep ``tensors`` alive for it.

        Called by every submission (and by the plans that launch on a queue):
        the queue's stream waits for the work already issued on the caller's
        current stream of this device, and each CUDA tensor in ``tensors`` is
        recorded as used by the queue's stream.
        """
        current = torch.cuda.current_stream(self.device)
        if current.cuda_stream != self.stream.cuda_stream:
            self.stream.wait_stream(current)
        for tensor in tensors:
            if isinstance(tensor, torch.Tensor) and tensor.is_cuda:
                tensor.record_stream(self.stream)

    def _wait_dependencies(self, wait_for: Iterable[Event]) -> None:
        for event in wait_for:
            if not isinstance(event, Event):
                raise DependencyError("wait_for accepts Events of this library only")
            hip_event = event.hip_event()
            if hip_event is not None and event.queue is not self:
                self.stream.wait_event(hip_event)

    def submit(
        self,
        kernel: Kernel,
        args: tuple[Any, ...] = (),
        *,
        grid: tuple[int, int, int] = (1, 1, 1),
        wait_for: Iterable[Event] = (),
        buffers: Iterable[Any] = (),
    ) -> Event:
        """Enqueue ``kernel`` on this queue's stream and return its completion event.

        ``buffers`` is accepted for signature compatibility with the
        reference; stream order already serialises hazards on one queue.
        """
        if self._closed:
            raise DependencyError("queue is closed")
        launch = LaunchConfig(tuple(int(g) for g in grid))  # type: ignore[arg-type]
        self.order_after_caller(args)
        self._wait_dependencies(wait_for)
        with torch.cuda.device(self.device):
            kernel.execute(self.handle, args, launch)
            hip_event = torch.cuda.Event()
            hip_event.record(self.stream)
        return Event(self, kernel.name, "gpu", hip_event)

    def host_task(
        self,
        fn: Callable[[], None],
        *,
        wait_for: Iterable[Event] = (),
        buffers: Iterable[Any] = (),
        name: str | None = None,
    ) -> Event:
        """Run ``fn`` on the calling thread after this queue and ``wait_for`` complete."""
        if self._closed:
            raise DependencyError("queue is closed")
        for event in wait_for:
            event.wait()
        self.stream.synchronize()
        fn()
        return Event(self, name or getattr(fn, "__qualname__", "host_task"), "host", None)

    def synchronize(self) -> None:
        call("qxt_stream_wait", self.handle)
