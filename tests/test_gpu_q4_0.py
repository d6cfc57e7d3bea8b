"""GPU parity of the Q4_0 x Q8_0 linear against the NumPy oracle (bit-exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import load_golden
from qpu_xla_amd import EventStatus, KernelError, Queue, _lib
from qpu_xla_amd.kernels import ggml_q4_0 as q4

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(123456.0)


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def random_blocks(rng, rows, blocks, outputs):
    act = oracle.pack_q8_0_blocks(
        rng.uniform(0.0001, 0.2, (rows, blocks)).astype(np.float16), rng.integers(-128, 128, (rows, blocks, 32))
    )
    wt = oracle.pack_q4_0_blocks(
        rng.uniform(-0.2, 0.2, (outputs, blocks)).astype(np.float16), rng.integers(0, 16, (outputs, blocks, 32))
    )
    return act, wt


@pytest.mark.parametrize("name", ["kat_q4_0_m1", "kat_q4_0_m4", "kat_q4_0_mx"])
def test_native_smoke_kats_through_the_queue_contract(name: str) -> None:
    # Resident partition [16, 32) as in qpu_llama_q4_0_smoke.c; columns 0..15 keep the sentinel.
    g = load_golden(name)
    rows = g["activation"].shape[0]
    start = int(g["resident_start"])
    resident = dev(g["weight"][start:])
    destination = torch.full((rows, g["weight"].shape[0]), float(SENTINEL), device="cuda")
    with Queue() as queue:
        queue.submit(
            q4.GGML_Q4_0_Q8_0_LINEAR_KERNEL,
            (dev(g["activation"]), resident, destination, 0, start, int(g["resident_count"])),
            grid=q4.expected_grid(rows, int(g["resident_count"])),
        ).wait()
    out = destination.cpu().numpy()
    np.testing.assert_array_equal(out[:, :start], SENTINEL)
    np.testing.assert_array_equal(out[:, start:], g["expected"][:, start:])


def test_reference_seed_fixture_bit_exact_and_block_dots() -> None:
    # Inputs of tests/test_qpu_xla_ggml_q4_0.py:47-80 (seed 4404).
    g = load_golden("oracle_q4_0_linear_seed4404")
    act, wt = dev(g["activation"]), dev(g["weight"])
    out = q4.ggml_q4_0_q8_0_linear(act, wt)
    np.testing.assert_array_equal(out.cpu().numpy(), g["expected"])
    dots = q4.ggml_q4_0_q8_0_block_dots(act, wt)
    np.testing.assert_array_equal(dots.cpu().numpy(), g["dots"])


@pytest.mark.parametrize(
    "rows,blocks,outputs",
    [
        (1, 1, 16),      # generic path, single block
        (1, 3, 50),      # generic path, ragged N
        (2, 8, 33),      # fast path, ragged N
        (3, 16, 64),
        (4, 64, 5632),   # cfg0-like K=2048 at M=4
        (1, 176, 100),   # K=5632 (22 units of 8 blocks)
        (5, 24, 40),     # row group 4 + 1
        (16, 8, 48),
        (1, 1024, 16),   # K=32768: 128 units per column, two columns per workgroup
        (4, 128, 11000),  # four rows, wide tiles: 43 columns per workgroup in three rounds, ragged last tile
        (8, 128, 4100),   # two row groups of wide tiles, three rounds per workgroup
        (6, 16, 130),     # four-row matrix-core tiles over native rows, two block ranges per unit
        (4, 32, 77),      # four block ranges per unit
        (4, 64, 9000),    # eight block ranges per unit, tiles of several rounds
        (1, 448, 300),    # K=14336 at one row: split units over 512 threads, 448 Q8_0 blocks fetched
        (1, 512, 200),    # K=16384: the largest row the split single linear fetches into registers
    ],
)
def test_random_shapes_bit_exact(rows: int, blocks: int, outputs: int) -> None:
    rng = np.random.default_rng(rows * 1000 + blocks * 10 + outputs)
    act, wt = random_blocks(rng, rows, blocks, outputs)
    out = q4.ggml_q4_0_q8_0_linear(dev(act), dev(wt))
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.q4_0_q8_0_reference(act, wt))
    dots = q4.ggml_q4_0_q8_0_block_dots(dev(act), dev(wt))
    np.testing.assert_array_equal(dots.cpu().numpy(), oracle.q4_0_q8_0_block_dots(act, wt))


def test_every_aligned_subrange_of_48_columns_leaves_the_rest_untouched() -> None:
    # qpu_llama_native_safety_smoke.c: every aligned 16-column subrange of 48 columns.
    rng = np.random.default_rng(48)
    act, wt = random_blocks(rng, 4, 8, 48)
    expected = oracle.q4_0_q8_0_reference(act, wt)
    a, w = dev(act), dev(wt)
    for start in range(0, 48, 16):
        for count in range(16, 48 - start + 1, 16):
            destination = torch.full((4, 48), float(SENTINEL), device="cuda")
            q4.ggml_q4_0_q8_0_linear(a, w, destination, weight_column_start=start,
                                     output_column_start=start, column_count=count)
            out = destination.cpu().numpy()
            np.testing.assert_array_equal(out[:, start:start + count], expected[:, start:start + count])
            mask = np.ones(48, bool)
            mask[start:start + count] = False
            np.testing.assert_array_equal(out[:, mask], SENTINEL)


def test_sequential_block_order_is_reproduced() -> None:
    # ((0 + 1) + 2**-24) - 1 == 0 only when blocks are summed in order.
    codes = np.full((1, 3, 32), 8, np.uint8)
    codes[0, :, 0] = 9
    a_vals = np.zeros((1, 3, 32), np.int16)
    a_vals[0, :, 0] = [1, 1, -1]
    act = oracle.pack_q8_0_blocks(np.array([[1.0, 2.0**-12, 1.0]], np.float16), a_vals)
    wt = oracle.pack_q4_0_blocks(np.array([[1.0, 2.0**-12, 1.0]], np.float16), codes)
    wt16 = np.repeat(wt, 16, axis=0)
    out = q4.ggml_q4_0_q8_0_linear(dev(act), dev(wt16)).cpu().numpy()
    np.testing.assert_array_equal(out, np.zeros((1, 16), np.float32))


def test_contract_errors_leave_destination_untouched() -> None:
    rng = np.random.default_rng(5)
    act, wt = random_blocks(rng, 4, 8, 32)
    a, w = dev(act), dev(wt)
    destination = torch.full((4, 32), float(SENTINEL), device="cuda")
    with Queue() as queue:
        # As the reference's worker does, a failed executor fails the event;
        # wait() raises the KernelError and nothing reaches the stream.
        failed = queue.submit(q4.GGML_Q4_0_Q8_0_LINEAR_KERNEL, (a, w, destination, 0, 0, 32), grid=(1, 1, 1))
        with pytest.raises(KernelError, match="grid"):
            failed.wait()
        assert failed.status is EventStatus.FAILED and isinstance(failed.exception, KernelError)
        with pytest.raises(KernelError, match="aligned"):
            queue.submit(q4.GGML_Q4_0_Q8_0_LINEAR_KERNEL, (a, w, destination, 8, 0, 16), grid=(1, 1, 1)).wait()
        _lib.set_failure_mask(_lib.FAIL_SUBMISSION)
        try:
            injected = queue.submit(q4.GGML_Q4_0_Q8_0_LINEAR_KERNEL, (a, w, destination, 0, 0, 32), grid=(2, 1, 1))
        finally:
            _lib.set_failure_mask(_lib.FAIL_NONE)
        with pytest.raises(KernelError):
            injected.wait()
        assert injected.status is EventStatus.FAILED
        queue.synchronize()
    np.testing.assert_array_equal(destination.cpu().numpy(), SENTINEL)


def _cfg_case(seed: int, rows: int, k: int, n: int):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((rows, k), dtype=np.float32)
    return w, x


@pytest.mark.parametrize(
    "seed,rows,k,n",
    [
        (0, 1, 2048, 5632),   # BASELINE cfg0: TinyLlama FFN-up, M=1
        (2, 4, 4096, 4096),   # cfg2 (second shape), M=4
        (2, 4, 4096, 11008),  # cfg2 (first shape), M=4
        (3, 1, 5632, 2048),   # cfg3 down projection
        (3, 1, 2048, 256),    # cfg3 k/v projection
    ],
)
def test_baseline_configs_end_to_end_bit_exact(seed: int, rows: int, k: int, n: int) -> None:
    from qpu_xla_amd.kernels.quantize import quantize_q4_0, quantize_q8_0

    w, x = _cfg_case(seed, rows, k, n)
    wq = quantize_q4_0(dev(w))
    xq = quantize_q8_0(dev(x))
    wq_ref = oracle.quantize_q4_0_blocks(w)
    xq_ref = oracle.quantize_q8_0_blocks(x)
    np.testing.assert_array_equal(wq.cpu().numpy(), wq_ref)
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)
    out = q4.ggml_q4_0_q8_0_linear(xq, wq).cpu().numpy()
    expected = oracle.q4_0_q8_0_reference(xq_ref, wq_ref)
    np.testing.assert_array_equal(out, expected)
    # The north-star tolerance (rel 1e-5 of max|ref|) holds a fortiori.
    assert np.abs(out - expected).max() <= 1e-5 * np.abs(expected).max()


def _batch_case(seed: int, shapes, fused_every: int = 2):
    """Tasks over (rows, k, n, wcol0, ncols) with alternating fp32 (fused) / native Q8_0 inputs."""
    rng = np.random.default_rng(seed)
    tasks, expected = [], []
    for i, (rows, k, n, wcol0, ncols) in enumerate(shapes):
        w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        x = rng.standard_normal((rows, k), dtype=np.float32)
        x[0, :32] = 0.0  # an all-zero activation block
        wq = oracle.quantize_q4_0_blocks(w)
        xq = oracle.quantize_q8_0_blocks(x)
        dest = torch.full((rows, ncols + 16), float(SENTINEL), device="cuda")
        task = {"weight": dev(wq), "destination": dest, "weight_column_start": wcol0,
                "output_column_start": 16, "column_count": ncols}
        if i % fused_every == 0:
            task["x"] = dev(x)
        else:
            task["activation"] = dev(xq)
        tasks.append(task)
        expected.append(oracle.q4_0_q8_0_reference(xq, wq[wcol0:wcol0 + ncols]))
    return tasks, expected


def _check_batch(tasks, expected) -> None:
    for task, want in zip(tasks, expected):
        out = task["destination"].cpu().numpy()
        np.testing.assert_array_equal(out[:, :16], SENTINEL)
        np.testing.assert_array_equal(out[:, 16:], want)


def test_batch_m1_mixed_shapes_bit_exact() -> None:
    shapes = [(1, 2048, 2048, 0, 2048), (1, 2048, 256, 0, 256), (1, 5632, 2048, 0, 2048),
              (1, 2048, 5632, 0, 5632), (1, 256, 48, 16, 17), (1, 4096, 100, 3, 90)]
    tasks, expected = _batch_case(31, shapes)
    with q4.Q4_0LinearBatch(tasks) as batch:
        assert batch.task_count == len(shapes) and batch.work_items > len(shapes)
        batch.launch()
        torch.cuda.synchronize()
        _check_batch(tasks, expected)
        for t in tasks:
            t["destination"][:, 16:] = -1.0
        batch.launch()  # a second launch of the same prepared batch
        torch.cuda.synchronize()
        _check_batch(tasks, expected)


def test_batch_many_work_items_eager_and_graph_replays() -> None:
    # More column tiles than the device holds workgroups at once (several
    # dispatch rounds), launched repeatedly, eagerly and from a captured graph.
    shapes = [(1, 2048, 5632, 0, 5632)] * 6 + [(1, 5632, 2048, 0, 2048)] * 6 + [(1, 2048, 256, 16, 240)] * 4
    tasks, expected = _batch_case(35, shapes)
    with q4.Q4_0LinearBatch(tasks) as batch:
        assert batch.work_items > 1024
        stream = torch.cuda.Stream()
        for _ in range(3):
            for t in tasks:
                t["destination"][:, 16:] = -1.0
            batch.launch(stream)
            stream.synchronize()
            _check_batch(tasks, expected)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            batch.launch(stream)
        for _ in range(3):
            for t in tasks:
                t["destination"][:, 16:] = -1.0
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            _check_batch(tasks, expected)
        del graph


@pytest.mark.parametrize("count", [1, 4, 5])
def test_batch_in_kernel_arguments_and_in_device_tables_bit_exact(count: int) -> None:
    # Up to four tasks travel in the kernel arguments (each workgroup finds its
    # task and column tile from its index), more in device tables.  Either
    # form, launched eagerly and replayed from a captured graph, matches the
    # oracle; ragged tiles end every task.
    shapes = [(1, 2048, 700, 0, 700), (1, 5632, 300, 4, 290), (1, 256, 64, 0, 64), (1, 4096, 96, 16, 77),
              (1, 2048, 130, 0, 130)][:count]
    tasks, expected = _batch_case(60 + count, shapes, fused_every=1)
    stream = torch.cuda.Stream()
    with q4.Q4_0LinearBatch(tasks) as batch:
        assert batch.task_count == count and batch.work_items >= count
        batch.launch(stream)
        stream.synchronize()
        _check_batch(tasks, expected)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            batch.launch(stream)
        for _ in range(2):
            for t in tasks:
                t["destination"][:, 16:] = -1.0
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            _check_batch(tasks, expected)
        del graph


@pytest.mark.parametrize("shapes", [
    [(1, 2048, 2048, 0, 2048), (1, 2048, 256, 0, 256), (1, 2048, 256, 0, 256)],  # q/k/v-like items
    [(1, 2048, 300, 4, 290), (1, 256, 40, 0, 40)],                                  # narrow items
    [(1, 5632, 2048, 0, 2048)],                                                       # down-like items
])
def test_stage_batch_mixing_lane_and_native_weights_bit_exact(shapes) -> None:
    # One prefetching stage batch whose tasks alternate lane-layout and native
    # weights (the kernel then chooses the load form per task), for item widths
    # whose units are split over four, two or one waves.
    tasks, expected = _batch_case(90 + len(shapes), shapes, fused_every=1)
    for i, t in enumerate(tasks):
        if i % 2 == 0:
            t["weight"] = q4.pack_ggml_q4_0_lane_weights(t["weight"])
    with q4.Q4_0LinearBatch(tasks) as batch:
        batch.launch()
        torch.cuda.synchronize()
    _check_batch(tasks, expected)


@pytest.mark.parametrize("k", [2048, 5632])
def test_stage_batch_activation_blocks_outside_the_fast_scale_range_bit_exact(k: int) -> None:
    # The prefetching stage kernels quantise their fp32 row with the
    # division-free Q8_0 scale and quantise a thread's chunks again with
    # divisions when one of its blocks has absmax outside [2^-96, 2^120]:
    # zero blocks, tiny blocks, blocks on the range's edges, next to ordinary
    # ones, through both weight layouts.
    rng = np.random.default_rng(k)
    x = rng.standard_normal((1, k), dtype=np.float32)
    blocks = x.reshape(1, k // 32, 32)
    for b, scale in [(0, 0.0), (3, 2.0**-100), (5, 2.0**-96), (8, 2.0**-97), (13, 2.0**-95), (21, 2.0**-110),
                     (34, 2.0**-120), (55, 0.0)]:
        blocks[0, b] *= np.float32(scale)
    n = 300
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    wq = oracle.quantize_q4_0_blocks(w)
    want = oracle.q4_0_q8_0_reference(oracle.quantize_q8_0_blocks(x), wq)
    for weight in (dev(wq), q4.pack_ggml_q4_0_lane_weights(dev(wq))):
        dest = torch.full((1, n + 16), float(SENTINEL), device="cuda")
        tasks = [{"x": dev(x), "weight": weight, "destination": dest, "weight_column_start": 0,
                  "output_column_start": 16, "column_count": n}]
        with q4.Q4_0LinearBatch(tasks) as batch:
            batch.launch()
            torch.cuda.synchronize()
        _check_batch(tasks, [want])


def test_batch_small_m_bit_exact() -> None:
    shapes = [(4, 4096, 64, 0, 64), (2, 2048, 40, 8, 32), (3, 256, 16, 0, 16), (1, 512, 33, 0, 33)]
    tasks, expected = _batch_case(32, shapes, fused_every=3)
    with q4.Q4_0LinearBatch(tasks) as batch:
        batch.launch()
        torch.cuda.synchronize()
    _check_batch(tasks, expected)


def test_batch_rejects_unsupported_tasks_and_injected_allocation_failure() -> None:
    tasks, _ = _batch_case(33, [(1, 96, 16, 0, 16)])  # K % 256 != 0
    with pytest.raises(_lib.QxtError) as info:
        q4.Q4_0LinearBatch(tasks)
    assert info.value.status == _lib.INVALID_ARGUMENT
    tasks, _ = _batch_case(34, [(1, 256, 16, 0, 16)])
    _lib.set_failure_mask(_lib.FAIL_ALLOCATION)
    try:
        with pytest.raises(_lib.QxtError) as info:
            q4.Q4_0LinearBatch(tasks)
        assert info.value.status == _lib.ALLOCATION_FAILED
    finally:
        _lib.set_failure_mask(_lib.FAIL_NONE)


# ------------------------------------------------------------ tiled / prefill


def _split_case(seed: int, rows: int, blocks: int, outputs: int):
    rng = np.random.default_rng(seed)
    act = oracle.pack_q8_0_blocks(
        rng.uniform(0.001, 0.2, (rows, blocks)).astype(np.float16), rng.integers(-127, 128, (rows, blocks, 32))
    )
    wt = oracle.pack_q4_0_blocks(
        rng.uniform(-0.2, 0.2, (outputs, blocks)).astype(np.float16), rng.integers(0, 16, (outputs, blocks, 32))
    )
    return act, wt


@pytest.mark.parametrize("blocks", [1, 2])
@pytest.mark.parametrize("scale_mode", ["fp16", "word"])
def test_tiled_linear_reference_case_bit_exact(blocks: int, scale_mode: str) -> None:
    # Inputs of tests/test_qpu_xla_ggml_q4_0.py:164-229 (seed 4480 + blocks, 16 x 16);
    # the reference checks its QPU program within rtol 2e-6, this kernel is bit-exact.
    rng = np.random.default_rng(4480 + blocks)
    rows = outputs = 16
    act = oracle.pack_q8_0_blocks(
        rng.uniform(0.001, 0.2, (rows, blocks)).astype(np.float16), rng.integers(-127, 128, (rows, blocks, 32))
    )
    wt = oracle.pack_q4_0_blocks(
        rng.uniform(-0.2, 0.2, (outputs, blocks)).astype(np.float16), rng.integers(0, 16, (outputs, blocks, 32))
    )
    expected = oracle.q4_0_q8_0_reference(act, wt)
    scales, quants = oracle.split_q8_0_blocks(act)
    if scale_mode == "word":
        scales = scales.astype(np.uint32).view(np.int32)
    else:
        scales = scales.view(np.int16)
    wscales, wquants = oracle.pack_q4_0_tiled_weights(wt)
    destination = torch.full((rows, outputs), float("nan"), device="cuda")
    args = (dev(quants), dev(scales), dev(wquants.view(np.int32)), dev(wscales.view(np.int16)), destination)
    with Queue() as queue:
        queue.submit(q4.GGML_Q4_0_Q8_0_TILED_LINEAR_KERNEL, args, grid=q4.tiled_grid(rows, outputs)).wait()
    np.testing.assert_array_equal(destination.cpu().numpy(), expected)


@pytest.mark.parametrize("rows,blocks,outputs", [(16, 2, 768), (17, 3, 40), (64, 5, 64), (130, 32, 300), (128, 64, 512)])
def test_tiled_linear_shapes_bit_exact_and_device_packing(rows: int, blocks: int, outputs: int) -> None:
    act, wt = _split_case(4488 + rows, rows, blocks, outputs)
    expected = oracle.q4_0_q8_0_reference(act, wt)
    wscales, wquants = q4.pack_ggml_q4_0_tiled_weights(dev(wt))
    ref_scales, ref_quants = oracle.pack_q4_0_tiled_weights(wt)
    np.testing.assert_array_equal(wscales.cpu().numpy().view(np.uint16), ref_scales)
    np.testing.assert_array_equal(wquants.cpu().numpy().view(np.uint32), ref_quants)
    ascales, aquants = q4.split_ggml_q8_0_blocks(dev(act))
    out = q4.ggml_q4_0_q8_0_tiled_linear(aquants, ascales, wquants, wscales).cpu().numpy()
    np.testing.assert_array_equal(out, expected)


@pytest.mark.parametrize("rows,blocks,wcol0,ncols", [
    (16, 8, 0, 48), (33, 5, 3, 61), (100, 12, 0, 128), (64, 1, 16, 16),
    (33, 5, 3, 60),  # the last activation block and the last weight block both end 2 bytes into a dword
    (530, 176, 0, 200),  # several staged groups, a ragged last row tile
])
def test_native_linear_prefill_rows_run_on_matrix_cores_bit_exact(rows: int, blocks: int, wcol0: int, ncols: int) -> None:
    # rows >= 16 through the native-layout entry point: odd block counts give
    # activation rows that are not 4-byte aligned; a column partition with a
    # sentinel prefix checks that only the requested columns are written.  A
    # block whose 32 values (or 16 nibble bytes) start 2 bytes into a dword
    # needs 2 bytes of the dword after them; when that block ends the tensor,
    # the rest of that dword lies past the operand's range.
    act, wt = _split_case(5000 + rows + blocks, rows, blocks, wcol0 + ncols + 5)
    destination = torch.full((rows, ncols + 16), float(SENTINEL), device="cuda")
    q4.ggml_q4_0_q8_0_linear(dev(act), dev(wt), destination, weight_column_start=wcol0,
                             output_column_start=16, column_count=ncols)
    out = destination.cpu().numpy()
    np.testing.assert_array_equal(out[:, :16], SENTINEL)
    np.testing.assert_array_equal(out[:, 16:], oracle.q4_0_q8_0_reference(act, wt[wcol0:wcol0 + ncols]))


def _extreme_scale_case(rows: int, blocks: int, outputs: int):
    """Scales at and past the ends of fp16 and dots of zero, placed in the first
    two 64-column tiles only: the other tiles keep finite scales throughout."""
    rng = np.random.default_rng(77)
    da = rng.uniform(0.001, 0.2, (rows, blocks)).astype(np.float16)
    av = rng.integers(-127, 128, (rows, blocks, 32))
    dw = rng.uniform(-0.2, 0.2, (outputs, blocks)).astype(np.float16)
    codes = rng.integers(0, 16, (outputs, blocks, 32))
    dw[3, 1] = np.inf       # dot * inf: +-inf, or NaN where the dot is 0
    dw[70, 0] = -np.inf
    dw[5, 2] = np.nan
    dw[7, :] = 65504.0
    dw[8, :] = -65504.0
    dw[9, :] = np.float16(2.0**-24)  # smallest fp16 subnormal
    dw[10, :] = 0.0
    dw[11, :] = -0.0
    dw[12, :] = -0.125
    codes[12] = 8                    # weight values 0: every dot of column 12 is 0
    av[2, 1] = 0                     # row 2, block 1: every dot is 0 (0 * inf in column 3)
    da[4, 0] = np.inf                # an infinite activation scale against finite dw
    da[6, 2] = 65504.0
    av[6, 2] = 127
    act = oracle.pack_q8_0_blocks(da, av)
    wt = oracle.pack_q4_0_blocks(dw, codes)
    with np.errstate(invalid="ignore", over="ignore"):
        expected = oracle.q4_0_q8_0_reference(act, wt)
    assert np.isnan(expected[2, 3]) and np.isinf(expected[:, 3]).any() and np.isnan(expected[:, 5]).all()
    assert np.isfinite(expected[np.ix_([0, 1, 3, 5], range(128, outputs))]).all()
    return act, wt, expected


@pytest.mark.parametrize("layout", ["native", "split"])
def test_prefill_non_finite_and_extreme_block_scales_bit_exact(layout: str) -> None:
    # The prefill kernels read block dots biased by 1.5 * 2^23 through one fma
    # per output when every weight scale of the workgroup's tile is finite,
    # and compute a tile again in the exact conversion form when one is not:
    # both forms against the oracle, NaN where the oracle gives NaN.
    rows, blocks, outputs = 40, 3, 200
    act, wt, expected = _extreme_scale_case(rows, blocks, outputs)
    if layout == "native":
        out = torch.full((rows, outputs), float(SENTINEL), device="cuda")
        q4.ggml_q4_0_q8_0_linear(dev(act), dev(wt), out)
    else:
        wscales, wquants = q4.pack_ggml_q4_0_tiled_weights(dev(wt))
        ascales, aquants = q4.split_ggml_q8_0_blocks(dev(act))
        out = q4.ggml_q4_0_q8_0_tiled_linear(aquants, ascales, wquants, wscales)
    np.testing.assert_array_equal(out.cpu().numpy(), expected)


# ------------------------------------------------------------- lane layout


@pytest.mark.parametrize("n,blocks", [(5632, 64), (37, 176), (2048, 176), (3, 8)])
def test_lane_pack_kernel_matches_the_layout_definition(n: int, blocks: int) -> None:
    rng = np.random.default_rng(n + blocks)
    native = rng.integers(0, 256, size=(n, blocks, 18), dtype=np.uint8)
    lanes = q4.pack_ggml_q4_0_lane_weights(dev(native))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(lanes.packed.cpu().numpy(), oracle.pack_q4_0_lanes(native))
    assert lanes.packed.numel() == _lib.load().qxt_q4_0_lanes_bytes(n, blocks)


@pytest.mark.parametrize("rows,k,n,wcol0,ncols", [
    (1, 2048, 5632, 0, 5632),   # cfg0
    (4, 4096, 4096, 0, 4096),   # cfg2 (K=4096, N=4096)
    (4, 4096, 11000, 8, 10984),  # wide four-row tiles over lane weights, several rounds, ragged
    (1, 5632, 2048, 16, 2032),  # a column range starting inside a lane group
    (2, 256, 37, 5, 31),        # a partial last group, any column range
    (17, 512, 64, 0, 64),       # rows beyond one MFMA-free row group
    (4, 14336, 1024, 0, 1024),  # K = 14336 at four rows: one-column tiles above 64 KB of LDS
    (8, 14336, 512, 16, 496),   # two row groups at K = 14336
    # four-row matrix-core tiles at every block range per unit that divides 16
    (4, 256, 37, 5, 31),        # one block range per unit, ragged
    (6, 512, 130, 2, 128),      # two, a partial second row group
    (5, 1024, 200, 3, 190),     # four, one row in the second row group
    (4, 2048, 300, 0, 300),     # eight
    (4, 2048, 9000, 3, 8990),   # eight, tiles of several rounds (units over two waves each)
])
def test_lane_linear_bit_exact_against_oracle(rows: int, k: int, n: int, wcol0: int, ncols: int) -> None:
    rng = np.random.default_rng(5000 + rows + n)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((rows, k), dtype=np.float32)
    wq, xq = oracle.quantize_q4_0_blocks(w), oracle.quantize_q8_0_blocks(x)
    lanes = q4.pack_ggml_q4_0_lane_weights(dev(wq))
    out = torch.full((rows, ncols + 16), float(SENTINEL), device="cuda")
    q4.ggml_q4_0_q8_0_lane_linear(dev(xq), lanes, out, weight_column_start=wcol0, output_column_start=16,
                                  column_count=ncols)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got[:, :16], SENTINEL)
    np.testing.assert_array_equal(got[:, 16:], oracle.q4_0_q8_0_reference(xq, wq[wcol0:wcol0 + ncols]))


def test_lane_batch_matches_native_batch_and_oracle() -> None:
    shapes = [(1, 2048, 2048, 0, 2048), (1, 2048, 256, 0, 256), (1, 5632, 2048, 0, 2048),
              (1, 2048, 5632, 0, 5632), (1, 256, 48, 16, 17), (4, 4096, 100, 3, 90)]
    tasks, expected = _batch_case(36, shapes)
    lane_tasks = []
    for t in tasks:
        lt = dict(t)
        lt["weight"] = q4.pack_ggml_q4_0_lane_weights(t["weight"])
        lt["destination"] = torch.full_like(t["destination"], float(SENTINEL))
        lane_tasks.append(lt)
    with q4.Q4_0LinearBatch(tasks) as native, q4.Q4_0LinearBatch(lane_tasks) as lanes:
        assert lanes.work_items == native.work_items
        native.launch()
        lanes.launch()
        torch.cuda.synchronize()
    _check_batch(tasks, expected)
    _check_batch(lane_tasks, expected)


def test_lane_entry_points_validate_before_launching() -> None:
    lib = _lib.load()
    assert lib.qxt_q4_0_lanes_bytes(10, 12) == 0 and lib.qxt_q4_0_lanes_bytes(0, 8) == 0
    assert lib.qxt_q4_0_lanes_bytes(65, 8) == 2 * 9216
    w = torch.zeros((8, 8, 18), dtype=torch.uint8, device="cuda")
    small = torch.zeros(9216 - 16, dtype=torch.uint8, device="cuda")
    status = lib.qxt_q4_0_pack_lanes(w.data_ptr(), 144, small.data_ptr(), small.numel(), 8, 8, None)
    assert status == _lib.INVALID_ARGUMENT
    lanes = q4.pack_ggml_q4_0_lane_weights(w)
    act = torch.zeros((1, 8, 34), dtype=torch.uint8, device="cuda")
    out = torch.zeros((1, 16), device="cuda")
    status = lib.qxt_ggml_q4_0_q8_0_linear_lanes(act.data_ptr(), 272, lanes.packed.data_ptr(), 8, out.data_ptr(), 64,
                                                  1, 8, 4, 0, 8, None)
    assert status == _lib.INVALID_ARGUMENT and "past the packed matrix" in _lib.last_error()


def test_cfg3_headline_step_lane_batch_through_the_prepass_bit_exact() -> None:
    # The exact launch bench.py times for cfg3: all 154 TinyLlama decode
    # linears (22 layers x q, k, v, o, gate, up, down) as one batch over
    # lane-layout weights with fp32 activations, so the batch runs the Q8_0
    # pre-pass launch (> 1024 work items) before the linear grid.  Every
    # linear's output is checked against the oracle, on two launches.
    from qpu_xla_amd.kernels.quantize import quantize_q4_0

    layer = (("q", 2048, 2048), ("k", 2048, 256), ("v", 2048, 256), ("o", 2048, 2048),
             ("gate", 2048, 5632), ("up", 2048, 5632), ("down", 5632, 2048))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    tasks, weights, inputs = [], [], []
    for _ in range(22):
        for _name, k, n in layer:
            w = torch.randn((n, k), generator=gen, device="cuda", dtype=torch.float32) * 0.02
            wq = quantize_q4_0(w)
            del w
            x = torch.randn((1, k), generator=gen, device="cuda", dtype=torch.float32)
            y = torch.full((1, n), float("nan"), device="cuda")
            tasks.append({"x": x, "weight": q4.pack_ggml_q4_0_lane_weights(wq), "destination": y})
            weights.append(wq)
            inputs.append(x)
    with q4.Q4_0LinearBatch(tasks) as batch:
        assert batch.task_count == 154 and batch.work_items > 1024
        for launch in range(2):
            for t in tasks:
                t["destination"].fill_(float("nan"))
            torch.cuda.synchronize()
            with _lib.launch_timing() as timing:
                batch.launch()
                torch.cuda.synchronize()
            assert [name for name, _ in timing.records] == ["q8_0_prepass_kernel", "q4_0_batch_kernel"]
            if launch == 0:
                expected = [oracle.q4_0_q8_0_reference(oracle.quantize_q8_0_blocks(x.cpu().numpy()), wq.cpu().numpy())
                            for x, wq in zip(inputs, weights)]
            for i, (t, want) in enumerate(zip(tasks, expected)):
                np.testing.assert_array_equal(t["destination"].cpu().numpy(), want, err_msg=f"linear {i}")


@pytest.mark.parametrize("rows", [3, 4, 8])
def test_native_linear_at_k14336_small_rows_bit_exact(rows: int) -> None:
    # The v_dot4 kernel over native rows at a K whose activation rows need more
    # than 64 KB of LDS at three or more rows (Llama-3-8B down projection).
    rng = np.random.default_rng(7100 + rows)
    k, n = 14336, 768
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((rows, k), dtype=np.float32)
    wq, xq = oracle.quantize_q4_0_blocks(w), oracle.quantize_q8_0_blocks(x)
    out = q4.ggml_q4_0_q8_0_linear(dev(xq), dev(wq))
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.q4_0_q8_0_reference(xq, wq))


@pytest.mark.parametrize("shapes", [
    # a decode step's dependency stages: q/k/v, o, gate/up, down (fp32 rows, K <= 6144)
    [(1, 2048, 2048, 0, 2048), (1, 2048, 256, 0, 256), (1, 2048, 256, 0, 256)],
    [(1, 2048, 5632, 0, 5632), (1, 2048, 5632, 0, 5632)],
    [(1, 5632, 2048, 0, 2048)],
    # K = 256 / 4096 / 6144 (two, four and six prefetched chunks per thread), ragged column ranges
    [(1, 256, 48, 16, 17), (1, 256, 300, 5, 290)],
    [(1, 4096, 1000, 8, 984), (1, 4096, 37, 0, 37)],
    [(1, 6144, 700, 3, 650), (1, 2048, 64, 0, 64)],
])
def test_one_row_fp32_stage_batches_with_activation_prefetch_bit_exact(shapes) -> None:
    # Small one-row batches whose activations are all fp32 rows: one launch,
    # the row quantised in every workgroup after being requested before the
    # weights; lane weights and native rows.
    tasks, expected = _batch_case(41 + len(shapes), shapes, fused_every=1)
    lane_tasks = [dict(t, weight=q4.pack_ggml_q4_0_lane_weights(t["weight"]),
                       destination=torch.full_like(t["destination"], float(SENTINEL))) for t in tasks]
    for batch_tasks in (tasks, lane_tasks):
        with q4.Q4_0LinearBatch(batch_tasks) as batch:
            assert batch.work_items <= 1024
            for _ in range(2):
                for t in batch_tasks:
                    t["destination"][:, 16:] = -1.0
                with _lib.launch_timing() as timing:
                    batch.launch()
                    torch.cuda.synchronize()
                assert [name for name, _ in timing.records] == ["q4_0_batch_kernel"]
                _check_batch(batch_tasks, expected)


@pytest.mark.parametrize("k_last", [8192, 8448])
def test_prepass_batch_native_row_prefetch_bit_exact(k_last: int) -> None:
    # A batch of more than 1024 work items runs the Q8_0 pre-pass; when every
    # resulting row has at most 256 blocks (K <= 8192) each workgroup requests
    # its row's blocks before its weights, otherwise (one task at K = 8448)
    # the whole batch stages rows after the weights.  Both bit-exact, with a
    # caller-given native Q8_0 row among the pre-pass rows.
    rng = np.random.default_rng(4096 + k_last)
    shared = {}
    tasks, expected = [], []
    shapes = [(8192, 2048)] * 7 + [(k_last, 2048), (2048, 256)]
    for i, (k, n) in enumerate(shapes):
        if k not in shared:
            w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
            shared[k] = oracle.quantize_q4_0_blocks(w)
        wq = shared[k][:n]
        x = rng.standard_normal((1, k), dtype=np.float32)
        x[0, 32:64] = 0.0
        xq = oracle.quantize_q8_0_blocks(x)
        task = {"weight": dev(wq), "destination": torch.full((1, n + 16), float(SENTINEL), device="cuda"),
                "weight_column_start": 0, "output_column_start": 16, "column_count": n}
        if i == 3:
            task["activation"] = dev(xq)
        else:
            task["x"] = dev(x)
        tasks.append(task)
        expected.append(oracle.q4_0_q8_0_reference(xq, wq))
    with q4.Q4_0LinearBatch(tasks) as batch:
        assert batch.work_items > 1024
        for _ in range(2):
            for t in tasks:
                t["destination"][:, 16:] = -1.0
            batch.launch()
            torch.cuda.synchronize()
            _check_batch(tasks, expected)


@pytest.mark.parametrize("count", [1, 4, 5])
@pytest.mark.parametrize("k_big", [8192, 8448])
def test_native_row_batches_in_arguments_and_tables_bit_exact(count: int, k_big: int) -> None:
    # Every task hands over a native Q8_0 row: batches of at most 256 blocks
    # per row request each row before the weights (up to four tasks in the
    # kernel arguments, more in device tables); a task of 264 blocks (K =
    # 8448) makes the whole batch stage rows after the weights.  Ragged
    # tiles end every task; a second launch repeats the result.
    shapes = [(1, k_big, 300, 0, 300), (1, 2048, 700, 4, 690), (1, 256, 64, 0, 64), (1, 4096, 96, 16, 77),
              (1, 5632, 130, 0, 130)][:count]
    tasks, expected = _batch_case(700 + count + k_big, shapes, fused_every=len(shapes) + 1)
    assert all("activation" in t for t in tasks[1:]) and "x" in tasks[0]
    # Task 0 too: give it its Q8_0 row instead of the fp32 row.
    x0 = tasks[0].pop("x").cpu().numpy()
    tasks[0]["activation"] = dev(oracle.quantize_q8_0_blocks(x0))
    stream = torch.cuda.Stream()
    with q4.Q4_0LinearBatch(tasks) as batch:
        assert batch.task_count == count
        for _ in range(2):
            for t in tasks:
                t["destination"][:, 16:] = -1.0
            batch.launch(stream)
            stream.synchronize()
            _check_batch(tasks, expected)


def test_batch_prepare_allocations_are_counted() -> None:
    # The library counts its own device allocations (qxt_allocation_count):
    # preparing a batch allocates its device tables, launching it does not.
    from qpu_xla_amd import _lib

    tasks, expected = _batch_case(41, [(1, 2048, 256, 0, 256)])
    before = _lib.allocation_count()
    with q4.Q4_0LinearBatch(tasks) as batch:
        prepared = _lib.allocation_count()
        assert prepared > before
        batch.launch()
        torch.cuda.synchronize()
        assert _lib.allocation_count() == prepared
    _check_batch(tasks, expected)
