"""GPU parity of the bridge's approximate weight modes (COLUMN_W8, ROWCOL_W8A8), through the C ABI.

The prepared linear re-quantises its resident Q4_0 columns to int8 with one
fp32 scale per column on the GPU; each submission then runs the column-scale
matrix-core kernel (COLUMN_W8) or re-quantises the Q8_0 rows and runs the
W8A8 GEMM (ROWCOL_W8A8).  Outputs are bit-exact against
``oracle/llama_approx.py`` over row counts around the kernels' 64-row tiles,
resident partitions with sentinels, CPU_REPACK weights, interleaved Q8_0x4
activations, zero columns and rows, and a TinyLlama FFN shape.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle.llama_approx import (
    column_w8_reference,
    requantize_q4_0_columns_w8,
    requantize_q8_0_rows_w8,
    rowcol_w8a8_reference,
)
from qpu_xla_amd.llama_bridge import (
    FORMAT_REPACK_4X4,
    WEIGHT_COLUMN_W8,
    WEIGHT_ROWCOL_W8A8,
    Execution,
    LlamaContext,
    LlamaQ4_0Linear,
)

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(-98765.0)
MODES = {"column_w8": WEIGHT_COLUMN_W8, "rowcol_w8a8": WEIGHT_ROWCOL_W8A8}


def _operands(rng: np.random.Generator, rows: int, blocks: int, n: int) -> tuple[np.ndarray, np.ndarray]:
    act = oracle.pack_q8_0_blocks(rng.uniform(0.0005, 0.05, (rows, blocks)).astype(np.float16),
                                  rng.integers(-128, 128, (rows, blocks, 32)))
    weight = oracle.pack_q4_0_blocks(rng.uniform(0.0005, 0.05, (n, blocks)).astype(np.float16),
                                     rng.integers(0, 16, (n, blocks, 32)))
    return act, weight


def _expected(mode: str, act: np.ndarray, weight: np.ndarray) -> np.ndarray:
    wq, cs = requantize_q4_0_columns_w8(weight)
    if mode == "column_w8":
        return column_w8_reference(act, wq, cs)
    aq, rs = requantize_q8_0_rows_w8(act)
    return rowcol_w8a8_reference(aq, rs, wq, cs)


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("rows,blocks", [(5, 2), (16, 8), (63, 4), (65, 3), (130, 16)])
def test_approximate_modes_bit_exact_with_partitions(mode: str, rows: int, blocks: int) -> None:
    rng = np.random.default_rng(100 * rows + blocks)
    n, start, count = 96, 16, 64
    act, weight = _operands(rng, rows, blocks, n)
    expected = _expected(mode, act, weight)
    k = blocks * 32
    with LlamaContext() as ctx, LlamaQ4_0Linear(ctx, weight, input_columns=k, output_columns=n, rows=rows,
                                                 resident_column_start=start, resident_column_count=count,
                                                 weight_mode=MODES[mode]) as linear:
        # The whole resident range, then a sub-range and fewer rows than prepared.
        destination = np.full((rows, n), SENTINEL, dtype=np.float32)
        linear.execute(Execution(act, destination, start, count))
        np.testing.assert_array_equal(destination[:, start:start + count], expected[:, start:start + count])
        np.testing.assert_array_equal(destination[:, :start], SENTINEL)
        np.testing.assert_array_equal(destination[:, start + count:], SENTINEL)

        sub_rows = max(1, rows - 3)
        destination = np.full((sub_rows, n), SENTINEL, dtype=np.float32)
        linear.execute(Execution(np.ascontiguousarray(act[:sub_rows]), destination, start + 32, 16, rows=sub_rows))
        # ROWCOL re-quantises each row on its own, so fewer rows give the same rows.
        np.testing.assert_array_equal(destination[:, start + 32:start + 48], expected[:sub_rows, start + 32:start + 48])
        np.testing.assert_array_equal(destination[:, :start + 32], SENTINEL)
        np.testing.assert_array_equal(destination[:, start + 48:], SENTINEL)


@pytest.mark.parametrize("mode", list(MODES))
def test_approximate_modes_repacked_weights_and_interleaved_activations(mode: str) -> None:
    rng = np.random.default_rng(7)
    rows, blocks, n = 12, 4, 64
    act, weight = _operands(rng, rows, blocks, n)
    expected = _expected(mode, act, weight)
    k = blocks * 32
    with LlamaContext() as ctx, LlamaQ4_0Linear(ctx, oracle.pack_q4_0x4(weight), input_columns=k, output_columns=n,
                                                 rows=rows, weight_mode=MODES[mode],
                                                 weight_format=FORMAT_REPACK_4X4) as linear:
        for interleave in (0, 4, 8):
            source = act if interleave == 0 else oracle.interleave_q8_0x4(act, interleave)
            destination = np.full((rows, n), SENTINEL, dtype=np.float32)
            linear.execute(Execution(source, destination, 0, n, activation_interleave=interleave))
            np.testing.assert_array_equal(destination, expected, err_msg=f"interleave {interleave}")


@pytest.mark.parametrize("mode", list(MODES))
def test_approximate_modes_zero_columns_and_rows(mode: str) -> None:
    rng = np.random.default_rng(8)
    rows, blocks, n = 8, 2, 32
    act, weight = _operands(rng, rows, blocks, n)
    weight[5, :, :2] = 0  # all block scales of column 5 are +0: its column scale is 0
    act[3, :, :2] = 0     # row 3's block scales are +0: its row scale is 0 (ROWCOL)
    expected = _expected(mode, act, weight)
    assert not expected[:, 5].any() and np.isfinite(expected).all()
    with LlamaContext() as ctx, LlamaQ4_0Linear(ctx, weight, input_columns=blocks * 32, output_columns=n, rows=rows,
                                                 weight_mode=MODES[mode]) as linear:
        destination = np.full((rows, n), SENTINEL, dtype=np.float32)
        linear.execute(Execution(act, destination, 0, n))
        np.testing.assert_array_equal(destination, expected)


@pytest.mark.parametrize("mode", list(MODES))
def test_approximate_modes_tinyllama_gate_shape(mode: str) -> None:
    # M = 64 prompt rows through TinyLlama's gate projection (K = 2048, N = 5632).
    rng = np.random.default_rng(9)
    rows, blocks, n = 64, 64, 5632
    act, weight = _operands(rng, rows, blocks, n)
    expected = _expected(mode, act, weight)
    with LlamaContext() as ctx, LlamaQ4_0Linear(ctx, weight, input_columns=blocks * 32, output_columns=n, rows=rows,
                                                 weight_mode=MODES[mode]) as linear:
        destination = np.full((rows, n), SENTINEL, dtype=np.float32)
        linear.execute(Execution(act, destination, 0, n))
        np.testing.assert_array_equal(destination, expected)
