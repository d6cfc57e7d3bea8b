"""GPU parity of the fused GEGLU -> Q8_0 producer against the NumPy oracle (bit-exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from qpu_xla_amd import KernelError, Queue
from qpu_xla_amd.kernels import ggml_geglu_q8 as geglu
from qpu_xla_amd.kernels import ggml_q4_0 as q4

pytestmark = pytest.mark.gpu


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host_u8(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint8)


def gate_up(seed: int, rows: int, columns: int, sigma: float = 0.8) -> tuple[np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    gate = rng.normal(0.0, sigma, size=(rows, columns)).astype(np.float32)
    up = rng.normal(0.0, sigma, size=(rows, columns)).astype(np.float32)
    return gate, up


def q4_weight(rng: np.random.Generator, outputs: int, columns: int) -> np.ndarray:
    return oracle.pack_q4_0_blocks(
        rng.uniform(-0.15, 0.15, size=(outputs, columns // 32)).astype(np.float16),
        rng.integers(0, 16, size=(outputs, columns // 32, 32), dtype=np.uint8),
    )


def test_fused_geglu_q8_matches_reference_and_chains_into_q4_down() -> None:
    # tests/test_qpu_xla_ggml_geglu_q8.py:33-78 of the reference (seed 4964).
    rng = np.random.default_rng(4964)
    rows, columns, outputs = 16, 64, 32
    gate_host = rng.normal(0.0, 0.8, size=(rows, columns)).astype(np.float32)
    up_host = rng.normal(0.0, 0.8, size=(rows, columns)).astype(np.float32)
    expected_q8 = oracle.geglu_q8_0_reference(gate_host, up_host)
    weight_host = q4_weight(rng, outputs, columns)
    expected_down = oracle.q4_0_q8_0_reference(expected_q8, weight_host)
    table = geglu.ggml_gelu_fp16_table("cuda")
    q8 = torch.full(expected_q8.shape, 0xCD, dtype=torch.uint8, device="cuda")
    destination = torch.full(expected_down.shape, float("nan"), device="cuda")
    with Queue() as queue:
        queue.submit(geglu.GGML_GEGLU_Q8_0_KERNEL, (dev(gate_host), dev(up_host), q8, table),
                     grid=(columns // 32, rows, 1)).wait()
        actual_q8 = host_u8(q8)
        queue.submit(q4.GGML_Q4_0_Q8_0_LINEAR_KERNEL, (q8, dev(weight_host), destination, 0, 0, outputs),
                     grid=(outputs // 16, rows // 4, 1)).wait()
        actual_down = destination.cpu().numpy()
    np.testing.assert_array_equal(actual_q8, expected_q8)
    np.testing.assert_array_equal(actual_down, expected_down)


def test_split_geglu_q8_chains_into_tiled_q4_down() -> None:
    # tests/test_qpu_xla_ggml_geglu_q8.py:81-134 of the reference (seed 4965).
    rng = np.random.default_rng(4965)
    rows, columns, outputs = 16, 64, 32
    gate_host = rng.normal(0.0, 0.8, size=(rows, columns)).astype(np.float32)
    up_host = rng.normal(0.0, 0.8, size=(rows, columns)).astype(np.float32)
    expected_q8 = oracle.geglu_q8_0_reference(gate_host, up_host)
    weight_host = q4_weight(rng, outputs, columns)
    weight_scales, weight_q = q4.pack_ggml_q4_0_tiled_weights(dev(weight_host))
    expected_down = oracle.q4_0_q8_0_reference(expected_q8, weight_host)
    blocks = columns // 32
    table = geglu.ggml_gelu_fp16_table("cuda")
    scales = torch.full((rows, blocks), -1, dtype=torch.int32, device="cuda")
    values = torch.full((rows, columns), 0x55, dtype=torch.uint8, device="cuda")
    destination = torch.full(expected_down.shape, float("nan"), device="cuda")
    with Queue() as queue:
        queue.submit(geglu.GGML_GEGLU_Q8_0_SPLIT_KERNEL, (dev(gate_host), dev(up_host), scales, values, table),
                     grid=(blocks, rows, 1)).wait()
        queue.submit(q4.GGML_Q4_0_Q8_0_TILED_LINEAR_KERNEL, (values, scales, weight_q, weight_scales, destination),
                     grid=(outputs // 16, rows // 16, 1)).wait()
        actual_scales = scales.cpu().numpy().view(np.uint32)
        actual_q = values.cpu().numpy()
        actual_down = destination.cpu().numpy()
    np.testing.assert_array_equal(actual_scales, expected_q8[..., :2].copy().view(np.uint16).reshape(rows, blocks))
    np.testing.assert_array_equal(actual_q.reshape(rows, blocks, 32), expected_q8[..., 2:])
    np.testing.assert_array_equal(actual_down, expected_down)


@pytest.mark.parametrize("rows,columns,sigma", [
    (1, 5632, 0.8),      # one decode row of a 5632-wide FFN
    (7, 2080, 2.0),      # odd rows, 65 blocks
    (257, 2048, 0.5),    # the reference README's M=257 chain
    (512, 5632, 1.0),    # a prefill batch
    (3, 32, 8.0),        # one block per row, large magnitudes
])
def test_random_shapes_bit_exact(rows: int, columns: int, sigma: float) -> None:
    gate, up = gate_up(5100 + rows, rows, columns, sigma)
    expected = oracle.geglu_q8_0_reference(gate, up)
    actual = geglu.ggml_geglu_q8_0(dev(gate), dev(up))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host_u8(actual), expected)
    words, planes = oracle.geglu_q8_0_split_reference(gate, up)
    for dtype in (torch.int32, torch.int16):
        scales = torch.empty((rows, columns // 32), dtype=dtype, device="cuda")
        scales, values = geglu.ggml_geglu_q8_0_split(dev(gate), dev(up), scales=scales)
        torch.cuda.synchronize()
        got = scales.cpu().numpy().view(np.uint32 if dtype == torch.int32 else np.uint16)
        np.testing.assert_array_equal(got.astype(np.uint32), words)
        np.testing.assert_array_equal(values.cpu().numpy(), planes)


BAND_MIN_BLOCKS = 1 << 16  # jobs of at least this many blocks take the LDS-band kernel


@pytest.mark.parametrize("copies", [1, 34])  # 1: global-table kernel; 34 copies: >= 65536 blocks, LDS band
def test_every_fp16_gate_value(copies: int) -> None:
    # Every finite fp16 value as a gate (the whole table through the kernel's
    # lookup path), with up = 1 and with random up, in rows of 1024 gates.
    bits = np.arange(1 << 16, dtype=np.uint16)
    finite = np.isfinite(bits.view(np.float16))
    values = np.tile(bits[finite].view(np.float16).astype(np.float32), copies)
    values = values[: values.size // 1024 * 1024].reshape(-1, 1024)
    assert (values.size // 32 >= BAND_MIN_BLOCKS) == (copies > 1)
    rng = np.random.default_rng(5200 + copies)
    table = geglu.ggml_gelu_fp16_table("cuda")
    for up in (np.ones_like(values), rng.normal(0.0, 1.0, size=values.shape).astype(np.float32)):
        expected = oracle.geglu_q8_0_reference(values, up)
        actual = geglu.ggml_geglu_q8_0(dev(values), dev(up), table)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host_u8(actual), expected)
    scales, planes = geglu.ggml_geglu_q8_0_split(dev(values), dev(up), table)
    torch.cuda.synchronize()
    words, expected_planes = oracle.geglu_q8_0_split_reference(values, up)
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), words)
    np.testing.assert_array_equal(planes.cpu().numpy(), expected_planes)


def test_fp16_ties_subnormals_and_zero_blocks() -> None:
    rng = np.random.default_rng(5201)
    lows = rng.integers(0x0001, 0x7BFF, size=2048).astype(np.uint16)
    mid = ((lows.view(np.float16).astype(np.float64) + (lows + 1).view(np.float16).astype(np.float64)) / 2)
    ties = (mid * np.where(rng.random(2048) < 0.5, -1.0, 1.0)).astype(np.float32).reshape(-1, 32)
    subnormal = (rng.integers(1, 1024, size=(8, 32)) * 2.0 ** -24 * rng.choice([-1.0, 1.0], size=(8, 32)))
    zeros = np.zeros((2, 32), np.float32)
    tiny_negative = np.full((2, 32), -20.0, np.float32)  # gelu underflows to -0: d = 0 blocks
    gate = np.concatenate([ties, subnormal.astype(np.float32), zeros, tiny_negative]).reshape(-1, 64)
    up = rng.normal(0.0, 1.0, size=gate.shape).astype(np.float32)
    up[-1] = 0.0
    expected = oracle.geglu_q8_0_reference(gate, up)
    actual = geglu.ggml_geglu_q8_0(dev(gate), dev(up))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host_u8(actual), expected)


def test_strided_unaligned_rows_and_destination() -> None:
    # Rows inside wider buffers at a 4-byte (not 16-byte) offset take the
    # scalar-load path; the destination rows are strided too.
    gate_full, up_full = gate_up(5202, 9, 1 + 96 + 3)
    gate, up = gate_full[:, 1:97], up_full[:, 1:97]
    expected = oracle.geglu_q8_0_reference(gate, up)
    out_full = torch.full((9, 4, 34), 0xEE, dtype=torch.uint8, device="cuda")
    geglu.ggml_geglu_q8_0(dev(gate_full)[:, 1:97], dev(up_full)[:, 1:97], destination=out_full[:, 1:4])
    torch.cuda.synchronize()
    got = host_u8(out_full)
    np.testing.assert_array_equal(got[:, 1:4], expected)
    assert np.all(got[:, 0] == 0xEE)


def test_band_kernel_strided_rows_and_misaligned_table() -> None:
    # A job above the band threshold with rows at a 4-byte offset (scalar
    # loads) and strided destination rows; then the same job with a table
    # that is only 2-byte aligned, which the band kernel cannot copy with
    # 16-byte loads and leaves to the global-table kernel.
    rows, columns = 520, 4096
    assert rows * columns // 32 >= BAND_MIN_BLOCKS
    gate_full, up_full = gate_up(5204, rows, columns + 4, 1.2)
    gate, up = gate_full[:, 1:columns + 1], up_full[:, 1:columns + 1]
    expected = oracle.geglu_q8_0_reference(gate, up)
    out_full = torch.full((rows, columns // 32 + 1, 34), 0xEE, dtype=torch.uint8, device="cuda")
    geglu.ggml_geglu_q8_0(dev(gate_full)[:, 1:columns + 1], dev(up_full)[:, 1:columns + 1],
                          destination=out_full[:, 1:])
    torch.cuda.synchronize()
    got = host_u8(out_full)
    np.testing.assert_array_equal(got[:, 1:], expected)
    assert np.all(got[:, 0] == 0xEE)
    padded = torch.zeros(TABLE_PAD + (1 << 16), dtype=torch.int16, device="cuda")
    padded[TABLE_PAD:] = geglu.ggml_gelu_fp16_table("cuda").view(torch.int16)
    table = padded[TABLE_PAD:].view(torch.uint16)
    assert table.data_ptr() % 16 == 2
    actual = geglu.ggml_geglu_q8_0(dev(gate), dev(up), table)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host_u8(actual), expected)


TABLE_PAD = 1  # one int16 in front of the table: its data pointer is 2 mod 16


def test_kernel_contract_checks() -> None:
    gate, up = gate_up(5203, 4, 64)
    table = geglu.ggml_gelu_fp16_table("cuda")
    q8 = torch.empty((4, 2, 34), dtype=torch.uint8, device="cuda")
    with Queue() as queue:
        with pytest.raises(KernelError, match="grid"):
            queue.submit(geglu.GGML_GEGLU_Q8_0_KERNEL, (dev(gate), dev(up), q8, table), grid=(4, 2, 1)).wait()
        with pytest.raises(KernelError, match="contiguous"):
            queue.submit(geglu.GGML_GEGLU_Q8_0_KERNEL, (dev(gate), dev(up), q8[:, :1], table), grid=(1, 4, 1)).wait()
        with pytest.raises(KernelError, match="split"):
            queue.submit(geglu.GGML_GEGLU_Q8_0_SPLIT_KERNEL,
                         (dev(gate), dev(up), torch.empty((4, 2), dtype=torch.float32, device="cuda"),
                          torch.empty((4, 64), dtype=torch.uint8, device="cuda"), table), grid=(2, 4, 1)).wait()
    with pytest.raises(ValueError, match="gelu_table"):
        geglu.ggml_geglu_q8_0(dev(gate), dev(up), table[:100])
    with pytest.raises(ValueError):
        geglu.ggml_geglu_q8_0(dev(gate[:, :48]), dev(up[:, :48]))
