"""GPU parity of the Q8_0 x Q8_0 linear against the NumPy oracle (bit-exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from qpu_xla_amd import KernelError, Queue
from qpu_xla_amd.kernels import ggml_q8_0 as q8

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(123456.0)


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def operands(seed: int, rows: int, outputs: int, blocks: int):
    rng = np.random.default_rng(seed)
    act = oracle.pack_q8_0_blocks(rng.uniform(-0.1, 0.1, (rows, blocks)).astype(np.float16),
                                  rng.integers(-128, 128, (rows, blocks, 32)))
    wt = oracle.pack_q8_0_blocks(rng.uniform(-0.1, 0.1, (outputs, blocks)).astype(np.float16),
                                 rng.integers(-128, 128, (outputs, blocks, 32)))
    return act, wt


def test_m4_kernel_contract_with_resident_partition() -> None:
    # tests/test_qpu_xla_ggml_q8_0.py:34-69 of the reference: 4 rows, 32 outputs, 3 blocks,
    # weight columns [16, 32) resident, destination columns [0, 16) keep the sentinel.
    act, wt = operands(4854, 4, 32, 3)
    expected = oracle.q8_0_q8_0_reference(act, wt)
    destination = torch.full((4, 32), float(SENTINEL), device="cuda")
    with Queue() as queue:
        queue.submit(q8.GGML_Q8_0_Q8_0_LINEAR_M4_KERNEL, (dev(act), dev(wt[16:]), destination, 0, 16, 16),
                     grid=(1, 1, 1)).wait()
        out = destination.cpu().numpy()
        np.testing.assert_array_equal(out[:, :16], SENTINEL)
        np.testing.assert_array_equal(out[:, 16:], expected[:, 16:])
        with pytest.raises(KernelError, match="grid"):
            queue.submit(q8.GGML_Q8_0_Q8_0_LINEAR_M4_KERNEL, (dev(act), dev(wt), destination, 0, 0, 32),
                         grid=(1, 1, 1)).wait()
        with pytest.raises(KernelError, match="M=4"):
            queue.submit(q8.GGML_Q8_0_Q8_0_LINEAR_M4_KERNEL, (dev(act[:3]), dev(wt), destination[:3], 0, 0, 32),
                         grid=(2, 1, 1)).wait()


@pytest.mark.parametrize("rows,blocks,n,wcol0,ncols", [
    (4, 128, 4096, 0, 4096),   # a Llama-7B-class M=4 shape (K=4096)
    (1, 64, 5632, 0, 5632),    # M=1, K=2048
    (3, 3, 40, 5, 30),         # blocks % 8 != 0: one block per thread, any column range
    (7, 16, 64, 0, 64),        # two row groups
    (2, 344, 33, 1, 31),       # K = 11008 (down projection), ragged columns
])
def test_random_shapes_bit_exact(rows: int, blocks: int, n: int, wcol0: int, ncols: int) -> None:
    act, wt = operands(4900 + rows + blocks, rows, n, blocks)
    out = torch.full((rows, ncols + 16), float(SENTINEL), device="cuda")
    q8.ggml_q8_0_q8_0_linear(dev(act), dev(wt), out, weight_column_start=wcol0, output_column_start=16,
                             column_count=ncols)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got[:, :16], SENTINEL)
    np.testing.assert_array_equal(got[:, 16:], oracle.q8_0_q8_0_reference(act, wt[wcol0:wcol0 + ncols]))
