"""The queue's event lifecycle for GPU work: status, failures, cancellation, device timestamps, trace."""

from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

import oracle
from qpu_xla_amd import EventCancelledError, EventStatus, KernelError, Queue, _lib
from qpu_xla_amd.kernels import ggml_q4_0 as q4

pytestmark = pytest.mark.gpu


def _case(seed: int, rows: int = 1, blocks: int = 64, n: int = 2048):
    rng = np.random.default_rng(seed)
    act = oracle.pack_q8_0_blocks(rng.uniform(0.001, 0.2, (rows, blocks)).astype(np.float16),
                                  rng.integers(-128, 128, (rows, blocks, 32)))
    wt = oracle.pack_q4_0_blocks(rng.uniform(-0.2, 0.2, (n, blocks)).astype(np.float16),
                                 rng.integers(0, 16, (n, blocks, 32)))
    return (torch.from_numpy(act).cuda(), torch.from_numpy(wt).cuda(), oracle.q4_0_q8_0_reference(act, wt))


def _submit(queue: Queue, act, wt, destination, **kw):
    rows, n = destination.shape
    return queue.submit(q4.GGML_Q4_0_Q8_0_LINEAR_KERNEL, (act, wt, destination, 0, 0, n),
                        grid=q4.expected_grid(rows, n), **kw)


def test_gpu_event_succeeds_with_device_timestamps_and_traces() -> None:
    act, wt, expected = _case(71)
    destination = torch.full((1, 2048), float("nan"), device="cuda")
    with Queue() as queue:
        event = _submit(queue, act, wt, destination)
        assert event.status in (EventStatus.RUNNING, EventStatus.SUCCEEDED)
        event.wait()
        assert event.status is EventStatus.SUCCEEDED and event.done and event.exception is None
        assert event.submitted_ns <= event.started_ns <= event.finished_ns
        np.testing.assert_array_equal(destination.cpu().numpy(), expected)
        trace = queue.chrome_trace()["traceEvents"]
        slices = [e for e in trace if e["name"] == q4.GGML_Q4_0_Q8_0_LINEAR_KERNEL.name]
        assert len(slices) == 1 and slices[0]["cat"] == "gpu" and slices[0]["args"]["status"] == "succeeded"
        assert queue.consume_completed_event_counts() == {"gpu": 1}


def test_failed_submissions_surface_as_failed_events_and_write_nothing() -> None:
    act, wt, _ = _case(72, rows=4, n=32, blocks=8)
    destination = torch.full((4, 32), 7.0, device="cuda")
    with Queue() as queue:
        bad_grid = queue.submit(q4.GGML_Q4_0_Q8_0_LINEAR_KERNEL, (act, wt, destination, 0, 0, 32), grid=(1, 1, 1))
        _lib.set_failure_mask(_lib.FAIL_SUBMISSION)
        try:
            injected = _submit(queue, act, wt, destination)
        finally:
            _lib.set_failure_mask(_lib.FAIL_NONE)
        for event in (bad_grid, injected):
            assert event.status is EventStatus.FAILED and isinstance(event.exception, KernelError)
            with pytest.raises(KernelError):
                event.wait()
        # A dependent submission fails with its dependency's exception.
        dependent = _submit(queue, act, wt, destination, wait_for=(injected,))
        with pytest.raises(KernelError):
            dependent.wait()
        queue.synchronize()
        statuses = [e["args"]["status"] for e in queue.chrome_trace()["traceEvents"] if e.get("cat") == "gpu"]
        assert statuses == []  # failed launches never started on the device
    np.testing.assert_array_equal(destination.cpu().numpy(), 7.0)


def test_work_behind_a_pending_host_task_is_held_in_order_and_cancellable() -> None:
    act, wt, expected = _case(73)
    first_out = torch.full((1, 2048), float("nan"), device="cuda")
    cancelled_out = torch.full((1, 2048), -1.0, device="cuda")
    last_out = torch.full((1, 2048), float("nan"), device="cuda")
    seen: list[np.ndarray] = []
    gate = threading.Event()
    with Queue() as queue:
        first = _submit(queue, act, wt, first_out)
        # The host task runs after the GPU work submitted before it and sees its result.
        host = queue.host_task(lambda: (gate.wait(), seen.append(first_out.cpu().numpy())), name="inspect")
        try:
            held = _submit(queue, act, wt, cancelled_out)
            last = _submit(queue, act, wt, last_out)
            assert held.status is EventStatus.PENDING and last.status is EventStatus.PENDING
            assert held.cancel()
        finally:
            gate.set()  # the queue's worker always gets past the host task
        last.wait()
        host.wait()
        assert first.status is EventStatus.SUCCEEDED and last.status is EventStatus.SUCCEEDED
        with pytest.raises(EventCancelledError):
            held.wait()
        assert host.finished_ns <= last.started_ns
        names = [e["name"] for e in queue.chrome_trace()["traceEvents"] if e["ph"] == "X" and e["cat"] != "queue"]
        assert names.count("inspect") == 1 and held.started_ns is None
    np.testing.assert_array_equal(seen[0], expected)
    np.testing.assert_array_equal(last_out.cpu().numpy(), expected)
    np.testing.assert_array_equal(cancelled_out.cpu().numpy(), -1.0)


def test_cross_queue_dependency_on_held_work() -> None:
    act, wt, expected = _case(74)
    out = torch.full((1, 2048), float("nan"), device="cuda")
    copy = torch.full((1, 2048), float("nan"), device="cuda")
    gate = threading.Event()
    def issue_copy() -> None:
        with torch.cuda.stream(consumer.stream):
            copy.copy_(out)

    with Queue() as producer, Queue() as consumer:
        producer.host_task(gate.wait)
        try:
            made = _submit(producer, act, wt, out)
            assert made.status is EventStatus.PENDING
            copied = consumer.launch("copy", issue_copy, tensors=(out, copy), wait_for=(made,))
            assert copied.status is EventStatus.PENDING  # held behind the producer's held launch
        finally:
            gate.set()  # the producer's worker always gets past the host task
        copied.wait()
        assert copied.started_ns >= made.finished_ns
        flows = [e for e in consumer.chrome_trace()["traceEvents"] if e["cat"] == "sync"]
        assert [e["ph"] for e in flows] == ["s", "f"]
    np.testing.assert_array_equal(copy.cpu().numpy(), expected)
