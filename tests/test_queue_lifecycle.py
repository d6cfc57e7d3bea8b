"""The queue's event lifecycle and trace export on a host-only queue (no GPU).

Mirrors the reference's runtime tests (``tests/test_qpu_xla_runtime.py:99-170``):
in-order host tasks with timestamps, explicit dependencies, failure and
cancellation, the Chrome trace payload and the completed-event counts.
"""

from __future__ import annotations

import json
import threading

import pytest

from qpu_xla_amd import (DependencyError, DeviceClosedError, EventCancelledError, EventStatus, EventTimeoutError,
                         Kernel, KernelError, LaunchConfig, Queue)


def test_host_tasks_run_in_order_with_timestamps() -> None:
    with Queue("cpu") as queue:
        order: list[int] = []
        first = queue.host_task(lambda: order.append(1))
        second = queue.host_task(lambda: order.append(2))
        second.wait()
        assert order == [1, 2]
        assert first.status is EventStatus.SUCCEEDED and first.done
        assert second.started_ns is not None and second.finished_ns is not None
        assert second.submitted_ns <= second.started_ns <= second.finished_ns
        assert first.finished_ns <= second.started_ns


def test_explicit_dependencies_and_wait_timeout() -> None:
    with Queue("cpu") as queue, Queue("cpu") as other:
        gate = threading.Event()
        observed: list[str] = []
        first = queue.host_task(lambda: (gate.wait(), observed.append("first")))
        try:
            second = other.host_task(lambda: observed.append("second"), wait_for=(first,))
            assert first.status in (EventStatus.PENDING, EventStatus.RUNNING)
            with pytest.raises(EventTimeoutError):
                second.wait(timeout=0.01)
        finally:
            gate.set()
        second.wait()
        assert observed == ["first", "second"]


def test_failures_propagate_and_pending_work_can_be_cancelled() -> None:
    with Queue("cpu") as queue:
        failed = queue.host_task(lambda: (_ for _ in ()).throw(ValueError("boom")))
        with pytest.raises(ValueError, match="boom"):
            failed.wait()
        assert failed.status is EventStatus.FAILED and isinstance(failed.exception, ValueError)
        # A dependent of a failed event fails with the same exception.
        dependent = queue.host_task(lambda: None, wait_for=(failed,))
        with pytest.raises(ValueError, match="boom"):
            dependent.wait()

        gate = threading.Event()
        blocking = queue.host_task(gate.wait)
        try:
            cancelled = queue.host_task(lambda: pytest.fail("a cancelled task ran"))
            assert cancelled.status is EventStatus.PENDING
            assert cancelled.cancel()
            assert not cancelled.cancel()
        finally:
            gate.set()
        blocking.wait()
        with pytest.raises(EventCancelledError):
            cancelled.wait()
        assert cancelled.status is EventStatus.CANCELLED
        assert not blocking.cancel()  # already finished
        after = queue.host_task(lambda: None, wait_for=(cancelled,))
        with pytest.raises(EventCancelledError):
            after.wait()


def test_chrome_trace_payload_has_delay_execution_and_flow_entries(tmp_path) -> None:
    with Queue("cpu") as queue:
        gate = threading.Event()
        first = queue.host_task(gate.wait, name="prepare")
        try:
            second = queue.host_task(lambda: None, wait_for=(first,), name="finish")
        finally:
            gate.set()
        second.wait()
        trace = queue.chrome_trace()
        assert set(trace) == {"traceEvents"}
        execution = [e for e in trace["traceEvents"] if e["ph"] == "X" and e["cat"] != "queue"]
        assert {e["name"] for e in execution} == {"prepare", "finish"}
        for entry in execution:
            assert entry["pid"] == "qpu-xla" and entry["tid"] == "host" and entry["cat"] == "host"
            assert entry["dur"] >= 0 and entry["args"]["status"] == "succeeded"
            assert set(entry) == {"name", "cat", "ph", "pid", "tid", "ts", "dur", "args"}
        delays = [e for e in trace["traceEvents"] if e["cat"] == "queue"]
        assert all(e["name"].startswith("queue delay: ") and e["tid"] == "submission" for e in delays)
        assert any(e["name"] == "queue delay: finish" for e in delays)  # it waited behind "prepare"
        flows = [e for e in trace["traceEvents"] if e["cat"] == "sync"]
        assert [e["ph"] for e in flows] == ["s", "f"]
        assert flows[0]["id"] == flows[1]["id"] == f"{first._sequence}->{second._sequence}"
        assert flows[0]["ts"] <= flows[1]["ts"]
        path = tmp_path / "queue-trace.json"
        queue.write_chrome_trace(path)
        assert json.loads(path.read_text(encoding="utf-8")) == json.loads(json.dumps(queue.chrome_trace()))


def test_completed_event_counts_release_events() -> None:
    with Queue("cpu") as queue:
        queue.host_task(lambda: None)
        queue.host_task(lambda: None).wait()
        assert queue.consume_completed_event_counts() == {"host": 2}
        assert queue.consume_completed_event_counts() == {}
        assert queue.chrome_trace() == {"traceEvents": []}


def test_closed_queue_rejects_work_and_host_queue_rejects_kernels() -> None:
    queue = Queue("cpu")
    with pytest.raises(DependencyError, match="host tasks only"):
        queue.submit(Kernel("k", lambda backend, args, grid: None))
    done = queue.host_task(lambda: None)
    queue.close()
    assert done.status is EventStatus.SUCCEEDED  # close drains submitted work
    with pytest.raises(DeviceClosedError):
        queue.host_task(lambda: None)
    with pytest.raises(DeviceClosedError):
        with queue:
            pass


def test_executor_errors_are_wrapped_as_kernel_errors() -> None:
    # The Kernel contract (reference kernel.py:31-38): any executor failure becomes a KernelError.
    kernel = Kernel("bad", lambda backend, args, grid: (_ for _ in ()).throw(RuntimeError("bad")))
    with pytest.raises(KernelError, match="bad"):
        kernel.execute(None, (), LaunchConfig((1, 1, 1)))
