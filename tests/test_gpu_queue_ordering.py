"""Queues and plans order their work after the caller's stream and keep freed arguments alive.

The caller produces an argument with asynchronous work on its current stream
(a slow chain of matrix products, then a non-blocking copy), submits, drops
its reference at once and allocates a same-sized tensor that the caching
allocator could hand the freed block to.  The queue's result must still be
bit-exact against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from qpu_xla_amd import Queue
from qpu_xla_amd.kernels import ggml_q4_0 as q4
from qpu_xla_amd.quantization import PreparedW8A8Linear, quantize_per_output_channel_int8

pytestmark = pytest.mark.gpu


def _slow_work_on_current_stream(products: int = 24) -> torch.Tensor:
    # About 3 TFLOP of fp32 products: several milliseconds of queued work.
    a = torch.full((4096, 4096), 1.0 / 4096, device="cuda")
    b = torch.empty_like(a)
    for _ in range(products):
        torch.mm(a, a, out=b)
        a, b = b, a
    return a


def test_queue_submit_waits_for_the_callers_stream_and_keeps_the_argument() -> None:
    rng = np.random.default_rng(61)
    rows, blocks, n = 1, 64, 2048
    act = oracle.pack_q8_0_blocks(rng.uniform(0.001, 0.2, (rows, blocks)).astype(np.float16),
                                  rng.integers(-128, 128, (rows, blocks, 32)))
    wt = oracle.pack_q4_0_blocks(rng.uniform(-0.2, 0.2, (n, blocks)).astype(np.float16),
                                 rng.integers(0, 16, (n, blocks, 32)))
    expected = oracle.q4_0_q8_0_reference(act, wt)
    weight = torch.from_numpy(wt).cuda()
    pinned = torch.from_numpy(act).pin_memory()
    torch.cuda.synchronize()
    with Queue() as queue:
        for _ in range(3):
            _slow_work_on_current_stream()
            activation = torch.empty(act.shape, dtype=torch.uint8, device="cuda")
            activation.copy_(pinned, non_blocking=True)  # lands after the products, in stream order
            destination = torch.full((rows, n), float("nan"), device="cuda")
            event = queue.submit(q4.GGML_Q4_0_Q8_0_LINEAR_KERNEL, (activation, weight, destination, 0, 0, n),
                                 grid=q4.expected_grid(rows, n))
            del activation
            junk = torch.empty(act.shape, dtype=torch.uint8, device="cuda")
            junk.fill_(0x7F)
            event.wait()
            np.testing.assert_array_equal(destination.cpu().numpy(), expected)
            del junk


def test_prepared_plan_waits_for_the_callers_stream_and_keeps_the_source() -> None:
    rng = np.random.default_rng(62)
    m, k, n = 8, 512, 256
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    x = rng.standard_normal((m, k), dtype=np.float32)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    qw, sw = oracle.quantize_per_output_channel_int8(w)
    expected = oracle.w8a8_linear_reference(x, qw, sw, bias)
    weight = quantize_per_output_channel_int8(torch.from_numpy(w).cuda())
    pinned = torch.from_numpy(x).pin_memory()
    with Queue() as queue, PreparedW8A8Linear(weight, max_batch=m, bias=torch.from_numpy(bias).cuda()) as plan:
        torch.cuda.synchronize()
        for _ in range(3):
            _slow_work_on_current_stream()
            source = torch.empty((m, k), device="cuda")
            source.copy_(pinned, non_blocking=True)
            destination = torch.full((m, n), float("nan"), device="cuda")
            event = plan.execute(destination, source, queue=queue)
            del source
            junk = torch.empty((m, k), device="cuda")
            junk.fill_(float("inf"))
            event.wait()
            np.testing.assert_array_equal(destination.cpu().numpy(), expected)
            del junk
