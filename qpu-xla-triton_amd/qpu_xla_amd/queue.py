"""In-order submission queue over one HIP stream, with the reference's event lifecycle.

The reference's ``Queue`` (``src/qpu_xla/queue.py:150-423``) is one worker
thread that runs kernel executors and host tasks in submission order and
returns an ``Event`` per submission (``queue.py:23-147``): PENDING until the
worker takes it, then RUNNING, then SUCCEEDED or FAILED (the failure kept on
the event and re-raised by ``wait``); a PENDING event can be cancelled.  On
the GPU the HIP stream already is an in-order worker, so this ``Queue``
launches a kernel on its stream from the submitting thread (no thread hop)
whenever nothing submitted earlier is still held on the host, bracketing the
launch with two timing events: the event is RUNNING from the launch on and
SUCCEEDED when the stream passes the second one, and its start and finish
timestamps are the device times of the two, on the host's monotonic clock.
Host tasks run on the queue's worker thread after the GPU work submitted
before them has finished; a submission made while host work is held (or that
waits for an event still held on another queue's worker) is held too, PENDING
and cancellable, until the worker issues it in order.  A launch whose
executor raises (validation, an injected submission failure) leaves nothing
on the stream: its event is FAILED and ``wait`` raises the ``KernelError``.

Tensors cross from the caller's stream to the queue's the way torch expects
of a side stream: every submission first makes the queue's stream wait for
the caller's current stream (so an argument still being written there by
asynchronous work is complete before the queue reads it), and every tensor
argument is marked as used on the queue's stream (``record_stream``), so the
caching allocator does not hand its memory out again while the queue's work
on it is pending -- the caller may drop its references right after submit.

``chrome_trace`` / ``write_chrome_trace`` export the reference's Chrome
Trace Event payload (``queue.py:275-374``): a queue-delay slice and an
execution slice per started event and a flow arrow per dependency;
``consume_completed_event_counts`` releases completed events by category.
"""

from __future__ import annotations

import json
import threading
import time
from collections.abc import Callable, Iterable
from enum import Enum
from os import PathLike
from queue import SimpleQueue
from typing import Any

import torch

from qpu_xla_amd._lib import call
from qpu_xla_amd.errors import DependencyError, DeviceClosedError, EventCancelledError, EventTimeoutError
from qpu_xla_amd.kernel import Kernel, LaunchConfig

TRACE_PROCESS = "qpu-xla"  # the reference's trace process label (queue.py:303)


class EventStatus(Enum):
    """Lifecycle states of a submission (values as the reference's ``EventStatus``)."""

    PENDING = "pending"
    RUNNING = "running"
    SUCCEEDED = "succeeded"
    FAILED = "failed"
    CANCELLED = "cancelled"


_TERMINAL = (EventStatus.SUCCEEDED, EventStatus.FAILED, EventStatus.CANCELLED)


class Event:
    """Completion state, failure and timestamps of one submission (kernel or host task).

    ``category`` is ``"gpu"`` for work on the queue's stream and ``"host"``
    for host tasks.  Timestamps are ``time.monotonic_ns`` values: submission
    on the host; start and finish on the host for host tasks, and the device
    times of the launch's bracketing HIP events for GPU work (None until the
    device has reached them).
    """

    def __init__(self, queue: "Queue", *, sequence: int, name: str, category: str,
                 dependencies: tuple["Event", ...]) -> None:
        self._queue = queue
        self._sequence = sequence
        self._name = name
        self._category = category
        self._dependencies = dependencies
        self._condition = threading.Condition()
        self._status = EventStatus.PENDING
        self._exception: BaseException | None = None
        self._submitted_ns = time.monotonic_ns()
        self._started_ns: int | None = None
        self._finished_ns: int | None = None
        self._start: torch.cuda.Event | None = None
        self._finish: torch.cuda.Event | None = None

    # ------------------------------------------------------------ properties

    @property
    def queue(self) -> "Queue":
        return self._queue

    @property
    def name(self) -> str:
        return self._name

    @property
    def category(self) -> str:
        return self._category

    @property
    def submitted_ns(self) -> int:
        return self._submitted_ns

    @property
    def status(self) -> EventStatus:
        with self._condition:
            if self._status is EventStatus.RUNNING and self._finish is not None and self._finish.query():
                self._status = EventStatus.SUCCEEDED
                self._condition.notify_all()
            return self._status

    @property
    def done(self) -> bool:
        return self.status in _TERMINAL

    @property
    def exception(self) -> BaseException | None:
        with self._condition:
            return self._exception

    @property
    def started_ns(self) -> int | None:
        with self._condition:
            if self._started_ns is None and self._start is not None and self._start.query():
                self._started_ns = self._queue._device_ns(self._start)
            return self._started_ns

    @property
    def finished_ns(self) -> int | None:
        with self._condition:
            if self._finished_ns is None and self._finish is not None and self._finish.query():
                started = self.started_ns
                self._finished_ns = max(self._queue._device_ns(self._finish), started or self._submitted_ns)
            return self._finished_ns

    def hip_event(self) -> torch.cuda.Event | None:
        """The HIP event the queue's stream records after this submission's work (GPU work only)."""
        with self._condition:
            return self._finish

    # ------------------------------------------------------------- lifecycle

    def cancel(self) -> bool:
        """Cancel the submission if it is still held on the host (PENDING); True if cancelled."""
        with self._condition:
            if self._status is not EventStatus.PENDING:
                return False
            self._status = EventStatus.CANCELLED
            self._finished_ns = time.monotonic_ns()
            self._condition.notify_all()
            return True

    def wait(self, timeout: float | None = None) -> None:
        """Block until the submission finished; re-raise its failure or cancellation."""
        if timeout is not None and timeout < 0:
            raise ValueError("timeout must be non-negative or None")
        deadline = None if timeout is None else time.monotonic() + timeout
        with self._condition:
            held = lambda: self._status is EventStatus.PENDING or (  # noqa: E731
                self._status is EventStatus.RUNNING and self._finish is None)
            if held() and not self._condition.wait_for(lambda: not held(), timeout=timeout):
                raise EventTimeoutError(f"event {self._name!r} did not complete within {timeout} s")
            finish = self._finish if self._status is EventStatus.RUNNING else None
        if finish is not None:
            if deadline is None:
                finish.synchronize()
            else:
                while not finish.query():
                    if time.monotonic() > deadline:
                        raise EventTimeoutError(f"event {self._name!r} did not complete within {timeout} s")
                    time.sleep(20e-6)
        status = self.status
        if status is EventStatus.CANCELLED:
            raise EventCancelledError(f"event {self._name!r} was cancelled")
        if status is EventStatus.FAILED:
            assert self._exception is not None
            raise self._exception

    # ------------------------------------------------- transitions (queue only)

    def _begin(self, on_host: bool) -> bool:
        """PENDING -> RUNNING; False when the event was cancelled first."""
        with self._condition:
            if self._status is EventStatus.CANCELLED:
                return False
            if self._status is not EventStatus.PENDING:
                raise RuntimeError("event cannot be started more than once")
            self._status = EventStatus.RUNNING
            if on_host:
                self._started_ns = time.monotonic_ns()
            return True

    def _issued(self, start: torch.cuda.Event, finish: torch.cuda.Event) -> None:
        with self._condition:
            self._start, self._finish = start, finish
            self._condition.notify_all()

    def _end(self, exception: BaseException | None = None) -> None:
        """Host work finished (or any work failed before reaching the stream)."""
        with self._condition:
            if self._status is EventStatus.CANCELLED:
                return
            self._exception = exception
            self._status = EventStatus.FAILED if exception is not None else EventStatus.SUCCEEDED
            self._start = self._finish = None
            self._finished_ns = time.monotonic_ns()
            self._condition.notify_all()

    def _held(self) -> bool:
        """Still on the host: not issued to a stream and not finished."""
        with self._condition:
            return self._status is EventStatus.PENDING or (
                self._status is EventStatus.RUNNING and self._finish is None)


_anchors: dict[torch.device, tuple[torch.cuda.Event, int]] = {}
_anchors_lock = threading.Lock()


def _device_anchor(device: torch.device) -> tuple[torch.cuda.Event, int]:
    """The device's clock anchor: a completed timing event and its host time.

    Device times map to the host's monotonic clock as anchor time + elapsed
    time since the anchor.  The anchor's host time is read just after it
    completes, so mapped times are at or a few microseconds after the true
    ones; one anchor per device keeps times of all its queues comparable.
    """
    key = torch.device("cuda", device.index if device.index is not None else torch.cuda.current_device())
    with _anchors_lock:
        if key not in _anchors:
            with torch.cuda.device(key):
                anchor = torch.cuda.Event(enable_timing=True)
                anchor.record(torch.cuda.current_stream(key))
                anchor.synchronize()
            _anchors[key] = (anchor, time.monotonic_ns())
        return _anchors[key]


class Queue:
    """In-order queue bound to one device and one HIP stream (or, for ``"cpu"``, host tasks only)."""

    def __init__(self, device: torch.device | int | str | None = None, stream: torch.cuda.Stream | None = None):
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
        self._lock = threading.Lock()
        self._events: list[Event] = []
        self._next_sequence = 0
        self._closed = False
        self._backlog = 0  # submissions handed to the worker and not yet issued or run
        self._issuing = False  # a submitting thread is launching onto the stream right now
        self._idle = threading.Condition(self._lock)
        self._work: SimpleQueue | None = None
        self._worker: threading.Thread | None = None
        if self.device.type == "cpu":
            self.stream = None
            return
        self.stream = stream if stream is not None else torch.cuda.Stream(device=self.device)
        self._anchor, self._anchor_ns = _device_anchor(self.device)

    def __enter__(self) -> "Queue":
        if self.closed:
            raise DeviceClosedError("queue is closed")
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    @property
    def closed(self) -> bool:
        with self._lock:
            return self._closed

    def close(self) -> None:
        """Stop accepting work and wait until everything submitted has finished."""
        with self._lock:
            if self._closed:
                return
            self._closed = True
            worker, work = self._worker, self._work
        if worker is not None:
            work.put(None)
            worker.join()
        if self.stream is not None:
            self.stream.synchronize()

    @property
    def handle(self) -> int:
        """The raw ``hipStream_t`` of this queue."""
        self._require_stream()
        return int(self.stream.cuda_stream)

    def synchronize(self) -> None:
        """Wait for every submission so far (work held on the host included)."""
        with self._lock:
            self._idle.wait_for(lambda: self._backlog == 0 and not self._issuing)
        if self.stream is not None:
            call("qxt_stream_wait", self.handle)

    # ------------------------------------------------------------ submission

    def order_after_caller(self, tensors: Iterable[Any] = ()) -> None:
        """Order this queue after the caller's current stream; keep ``tensors`` alive for it.

        The queue's stream waits for the work already issued on the caller's
        current stream of this device, and each CUDA tensor in ``tensors`` is
        recorded as used by the queue's stream.
        """
        if self.stream is None:
            return
        current = torch.cuda.current_stream(self.device)
        if current.cuda_stream != self.stream.cuda_stream:
            self.stream.wait_stream(current)
        for tensor in tensors:
            if isinstance(tensor, torch.Tensor) and tensor.is_cuda:
                tensor.record_stream(self.stream)

    def submit(
        self,
        kernel: Kernel,
        args: tuple[Any, ...] = (),
        *,
        grid: tuple[int, int, int] = (1, 1, 1),
        wait_for: Iterable[Event] = (),
        buffers: Iterable[Any] = (),
    ) -> Event:
        """Queue ``kernel`` on this queue's stream and return its completion event.

        An executor failure does not raise here: the event is FAILED and
        ``wait`` raises it, as the reference's worker does.  ``buffers`` is
        accepted for signature compatibility; stream order already
        serialises hazards on one queue.
        """
        launch = LaunchConfig(tuple(int(g) for g in grid))  # type: ignore[arg-type]
        self._require_stream()
        return self.launch(kernel.name, lambda: kernel.execute(self.handle, args, launch), tensors=args,
                           wait_for=wait_for)

    def launch(self, name: str, issue: Callable[[], None], *, tensors: Iterable[Any] = (),
               wait_for: Iterable[Event] = ()) -> Event:
        """Run ``issue`` (which enqueues GPU work on ``self.stream``) as one in-order submission."""
        self._require_stream()
        dependencies = self._normalize(wait_for)
        self.order_after_caller(tensors)
        with self._lock:
            event = self._new_event(name, "gpu", dependencies)
            defer = self._backlog > 0 or self._issuing or any(d._held() for d in dependencies)
            if defer:
                self._hand_to_worker(lambda: self._issue(event, issue, wait=True))
                return event
            self._issuing = True
        try:
            self._issue(event, issue, wait=False)
        finally:
            with self._lock:
                self._issuing = False
                self._idle.notify_all()
        return event

    def host_task(
        self,
        fn: Callable[[], None],
        *,
        wait_for: Iterable[Event] = (),
        buffers: Iterable[Any] = (),
        name: str | None = None,
    ) -> Event:
        """Run ``fn`` on the queue's worker after the queue's earlier work and ``wait_for``."""
        dependencies = self._normalize(wait_for)
        task_name = name if name is not None else str(getattr(fn, "__qualname__", "host_task"))
        with self._lock:
            event = self._new_event(task_name, "host", dependencies)
            self._hand_to_worker(lambda: self._run_host(event, fn))
        return event

    # ------------------------------------------------------------ trace export

    def chrome_trace(self) -> dict[str, list[dict[str, object]]]:
        """Chrome Trace Event payload of this queue's retained events (the reference's shape).

        Per started event: a queue-delay slice (submission to start) and an
        execution slice (start to finish, with the final status); per
        dependency of a started event, a flow arrow from the dependency's
        finish to the event's start.  Times are monotonic-clock microseconds.
        """
        with self._lock:
            events = tuple(self._events)
        trace: list[dict[str, object]] = []
        for event in events:
            started_ns = event.started_ns
            if started_ns is None:
                continue
            finished_ns = event.finished_ns
            submitted_us, started_us = event.submitted_ns / 1_000, started_ns / 1_000
            if started_ns > event.submitted_ns:
                trace.append({"name": f"queue delay: {event.name}", "cat": "queue", "ph": "X", "pid": TRACE_PROCESS,
                              "tid": "submission", "ts": submitted_us, "dur": started_us - submitted_us,
                              "args": {"event": event._sequence}})
            if finished_ns is not None:
                trace.append({"name": event.name, "cat": event.category, "ph": "X", "pid": TRACE_PROCESS,
                              "tid": event.category, "ts": started_us,
                              "dur": max(0, finished_ns - started_ns) / 1_000,
                              "args": {"event": event._sequence, "status": event.status.value}})
            for dependency in event._dependencies:
                dependency_finished_ns = dependency.finished_ns
                if dependency_finished_ns is None:
                    continue
                flow = f"{dependency._sequence}->{event._sequence}"
                trace.append({"name": "dependency", "cat": "sync", "ph": "s", "pid": TRACE_PROCESS,
                              "tid": dependency.category, "ts": dependency_finished_ns / 1_000, "id": flow})
                trace.append({"name": "dependency", "cat": "sync", "ph": "f", "pid": TRACE_PROCESS,
                              "tid": event.category, "ts": started_us, "id": flow})
        return {"traceEvents": trace}

    def write_chrome_trace(self, path: str | PathLike[str]) -> None:
        """Serialise ``chrome_trace`` to a Chrome Trace Event JSON file."""
        with open(path, "w", encoding="utf-8") as trace_file:
            json.dump(self.chrome_trace(), trace_file, separators=(",", ":"))

    def consume_completed_event_counts(self) -> dict[str, int]:
        """Count completed events by category and stop retaining them (bounded profiling memory)."""
        with self._lock:
            events = list(self._events)
        completed = [event for event in events if event.done]
        finished = set(map(id, completed))
        with self._lock:
            self._events = [event for event in self._events if id(event) not in finished]
        counts: dict[str, int] = {}
        for event in completed:
            counts[event.category] = counts.get(event.category, 0) + 1
        return counts

    # -------------------------------------------------------------- internals

    def _require_stream(self) -> None:
        if self.stream is None:
            raise DependencyError("this queue runs host tasks only; GPU work needs a queue on a HIP device")

    def _device_ns(self, hip_event: torch.cuda.Event) -> int:
        return self._anchor_ns + int(round(self._anchor.elapsed_time(hip_event) * 1e6))

    def _normalize(self, wait_for: Iterable[Event]) -> tuple[Event, ...]:
        dependencies: list[Event] = []
        for event in wait_for:
            if not isinstance(event, Event):
                raise DependencyError("wait_for accepts Events of this library only")
            if event.queue.device != self.device and "cpu" not in (event.queue.device.type, self.device.type):
                raise DependencyError("event dependency belongs to a different device")
            if event not in dependencies:
                dependencies.append(event)
        return tuple(dependencies)

    def _new_event(self, name: str, category: str, dependencies: tuple[Event, ...]) -> Event:
        """Called with the lock held."""
        if self._closed:
            raise DeviceClosedError("queue is closed")
        event = Event(self, sequence=self._next_sequence, name=name, category=category, dependencies=dependencies)
        self._next_sequence += 1
        self._events.append(event)
        return event

    def _hand_to_worker(self, action: Callable[[], None]) -> None:
        """Called with the lock held."""
        if self._worker is None:
            self._work = SimpleQueue()
            self._worker = threading.Thread(target=self._run_worker, name="qxt-queue", daemon=True)
            self._worker.start()
        self._backlog += 1
        self._work.put(action)

    def _run_worker(self) -> None:
        while True:
            action = self._work.get()
            if action is None:
                return
            with self._lock:
                # A launch decided before this item was handed over may still be issuing.
                self._idle.wait_for(lambda: not self._issuing)
            try:
                action()
            finally:
                with self._lock:
                    self._backlog -= 1
                    self._idle.notify_all()

    @staticmethod
    def _check_dependencies(dependencies: tuple[Event, ...], wait: bool) -> None:
        """Raise the failure of a failed or cancelled dependency (waiting first when ``wait``)."""
        for dependency in dependencies:
            if wait:
                with dependency._condition:
                    dependency._condition.wait_for(lambda: not dependency._held())
            status = dependency.status
            if status is EventStatus.FAILED:
                raise dependency.exception
            if status is EventStatus.CANCELLED:
                raise EventCancelledError(f"dependency {dependency.name!r} was cancelled")

    def _issue(self, event: Event, issue: Callable[[], None], wait: bool) -> None:
        if not event._begin(on_host=False):
            return
        try:
            self._check_dependencies(event._dependencies, wait)
            with torch.cuda.device(self.device):
                for dependency in event._dependencies:
                    finish = dependency.hip_event()
                    if finish is not None and dependency.queue is not self:
                        self.stream.wait_event(finish)
                start = torch.cuda.Event(enable_timing=True)
                start.record(self.stream)
                issue()
                finish = torch.cuda.Event(enable_timing=True)
                finish.record(self.stream)
        except BaseException as exc:  # noqa: BLE001 -- the failure belongs to the event
            event._end(exc)
            return
        event._issued(start, finish)

    def _run_host(self, event: Event, fn: Callable[[], None]) -> None:
        if not event._begin(on_host=True):
            return
        try:
            if self.stream is not None:
                self.stream.synchronize()  # the GPU work submitted before this task
            self._check_dependencies(event._dependencies, wait=True)
            for dependency in event._dependencies:
                finish = dependency.hip_event()
                if finish is not None:
                    finish.synchronize()
            fn()
        except BaseException as exc:  # noqa: BLE001
            event._end(exc)
            return
        event._end()
