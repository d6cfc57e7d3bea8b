"""GPU parity for kernel forms the shape-driven dispatch reaches only at larger or less usual shapes.

Each case names the kernel form it reaches (qxt_w8a8.hip / qxt_quantize.hip /
qxt_q4_0_tiled.hip dispatch rules) and is compared bit for bit with the
oracle, on sampled rows where a full NumPy product would take minutes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from qpu_xla_amd import Queue
from qpu_xla_amd.kernels import gemm_int8
from qpu_xla_amd.kernels.ggml_q4_0 import ggml_q4_0_q8_0_linear
from qpu_xla_amd.kernels.quantize import quantize_rows_int8
from qpu_xla_amd.quantization import quantize_per_output_channel_int8, w8a8_linear

pytestmark = pytest.mark.gpu


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def words(a: np.ndarray) -> torch.Tensor:
    return dev(np.ascontiguousarray(a).view(np.int32))


def _gemm_operands(seed: int, m: int, n: int, k: int):
    rng = np.random.default_rng(seed)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    return a, w, sa, sw, bias


@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("m,n,k", [
    (4096, 4096, 512),   # >= 256 tiles of 256 x 256, K % 128 == 0: the eight-wave large-tile kernel
    (4096, 4100, 4160),  # K % 128 == 64: the generic 256 x 256 kernel (ragged last tile column)
])
def test_large_tiles_epilogue_with_and_without_bias_sampled_rows(m: int, n: int, k: int, with_bias: bool) -> None:
    a, w, sa, sw, bias = _gemm_operands(m + n + k + with_bias, m, n, k)
    out = gemm_int8.w8a8_gemm_dequantize(dev(a), dev(w), dev(sa), dev(sw), dev(bias) if with_bias else None)
    rows = np.array([0, 1, 255, 256, 2047, 3840, m - 1])
    expected = oracle.dequantize_epilogue(oracle.int8_gemm_i32(a[rows], w), sa[rows], sw,
                                          bias if with_bias else None)
    np.testing.assert_array_equal(out.cpu().numpy()[rows], expected)


def test_mid_size_tiles_epilogue_without_bias_exact() -> None:
    # Fewer 256 x 256 tiles than CUs, at least as many 128 x 128 ones.
    a, w, sa, sw, _ = _gemm_operands(1281, 520, 8200, 208)
    out = gemm_int8.w8a8_gemm_dequantize(dev(a), dev(w), dev(sa), dev(sw))
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.dequantize_epilogue(oracle.int8_gemm_i32(a, w), sa, sw))


@pytest.mark.parametrize("p,q,r", [(512, 208, 8192), (4096, 256, 4096)])
def test_packed_k4_operands_fused_epilogue_at_larger_tiles(p: int, q: int, r: int) -> None:
    # The reference's tiled contract (packed K4 words) at the 128 x 128 and
    # generic 256 x 256 tile sizes, with the fused dequantising epilogue.
    rng = np.random.default_rng(p + q + r)
    left_v = rng.integers(-127, 128, size=(p, q), dtype=np.int8)
    right_v = rng.integers(-127, 128, size=(q, r), dtype=np.int8)
    sa = rng.uniform(0.001, 0.1, p).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, r).astype(np.float32)
    left, right = oracle.pack_int8_gemm_operands(left_v, right_v)
    destination = torch.empty((p, r), dtype=torch.float32, device="cuda")
    with Queue() as queue:
        queue.submit(gemm_int8.TILED_W8A8_GEMM_DEQUANTIZE_KERNEL,
                     (words(left), words(right), dev(sa), dev(sw), destination), grid=(r // 16, p // 16, 1)).wait()
    rows = np.array([0, 1, 127, 128, p // 2, p - 1])
    acc = (left_v[rows].astype(np.int64) @ right_v.astype(np.int64)).astype(np.int32)
    np.testing.assert_array_equal(destination.cpu().numpy()[rows], oracle.dequantize_epilogue(acc, sa[rows], sw))


@pytest.mark.parametrize("k", [4100, 5632, 8192])
def test_row_quantiser_eight_chunks_per_thread(k: int) -> None:
    # 4096 < K <= 8192 holds each row as eight 16-byte chunks per thread.
    rng = np.random.default_rng(k)
    x = rng.standard_normal((9, k), dtype=np.float32)
    x[1] *= np.float32(1e-4)  # the 1/127 floor active
    x[2, k // 3] = np.float32(40.0)  # one outlier sets the scale
    q, s = quantize_rows_int8(dev(x))
    want_q, want_s = oracle.quantize_rows_int8(x)
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 9])
def test_linear_without_bias_bit_exact(m: int) -> None:
    # qxt_w8a8_linear with no bias: the fused GEMV (M <= 4) and the
    # quantiser + GEMM (M = 9), epilogue without the bias add.
    rng = np.random.default_rng(70 + m)
    k, n = 2048, 300
    x = rng.standard_normal((m, k), dtype=np.float32)
    wf = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    weight = quantize_per_output_channel_int8(dev(wf))
    y = w8a8_linear(dev(x), weight, None).cpu().numpy()
    qw, sw = oracle.quantize_per_output_channel_int8(wf)
    np.testing.assert_array_equal(y, oracle.w8a8_linear_reference(x, qw, sw, None))


def test_native_prefill_on_a_large_grid_sampled_rows() -> None:
    # A native-layout prefill grid of at least two workgroups per CU runs the
    # staged kernel's branch-free form (plain dots): M = 512, K = 2048,
    # N = 5632 is 8 x 88 = 704 workgroups.
    rng = np.random.default_rng(512)
    m, k, n = 512, 2048, 5632
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((m, k), dtype=np.float32)
    wq = oracle.quantize_q4_0_blocks(w)
    xq = oracle.quantize_q8_0_blocks(x)
    y = ggml_q4_0_q8_0_linear(dev(xq), dev(wq)).cpu().numpy()
    rows = np.array([0, 1, 63, 64, 255, 448, m - 1])
    np.testing.assert_array_equal(y[rows], oracle.q4_0_q8_0_reference(xq[rows], wq))


@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("m,k", [(1, 16), (2, 1040), (4, 4096)])
def test_packed_k4_fused_linear_short_rows(m: int, k: int, with_bias: bool) -> None:
    # qxt_w8a8_linear over packed-K4 [K/4, N] weights at K <= 4096: the
    # 256-thread K4N GEMV holding each fp32 row as four 16-byte chunks per
    # thread, quantising it inside every workgroup.
    from qpu_xla_amd import _lib
    from qpu_xla_amd._tensors import ptr, row_stride

    rng = np.random.default_rng(900 + m + k + with_bias)
    n = 132
    x = rng.standard_normal((m, k), dtype=np.float32)
    wf = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    qw, sw = oracle.quantize_per_output_channel_int8(wf)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    w_d = words(np.ascontiguousarray(oracle.pack_int8_quads(qw).T))
    xd, sw_d, b_d = dev(x), dev(sw), dev(bias)
    qa = torch.empty((m, k), dtype=torch.int8, device="cuda")
    sa = torch.empty((m,), dtype=torch.float32, device="cuda")
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    _lib.call("qxt_w8a8_linear", ptr(xd), row_stride(xd), ptr(qa), row_stride(qa), ptr(sa), ptr(w_d), row_stride(w_d),
              ptr(sw_d), ptr(b_d) if with_bias else None, ptr(y), row_stride(y), m, n, k, _lib.WEIGHT_K4N, 0, None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), oracle.w8a8_linear_reference(x, qw, sw, bias if with_bias else None))


@pytest.mark.parametrize("m", [1, 2, 4])
def test_gemv_epilogue_without_bias_both_layouts(m: int) -> None:
    # Stored int8 rows (M <= 4): the GEMV kernels' dequantising epilogue
    # without the bias add, over [N, K] and packed-K4 weights.
    from qpu_xla_amd import _lib
    from qpu_xla_amd._tensors import ptr, row_stride

    rng = np.random.default_rng(40 + m)
    n, k = 4096, 2048
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    expected = oracle.dequantize_epilogue(oracle.int8_gemm_i32(a, w), sa, sw)
    y = gemm_int8.w8a8_gemm_dequantize(dev(a), dev(w), dev(sa), dev(sw)).cpu().numpy()
    np.testing.assert_array_equal(y, expected)
    left, right = oracle.pack_int8_gemm_operands(a, np.ascontiguousarray(w.T))
    lw, rw, sa_d, sw_d = words(left), words(right), dev(sa), dev(sw)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    _lib.call("qxt_w8a8_gemm_dequantize", ptr(lw), row_stride(lw), ptr(rw), row_stride(rw), ptr(sa_d), ptr(sw_d),
              None, ptr(out), row_stride(out), m, n, k, _lib.WEIGHT_K4N, None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), expected)


SENTINEL = np.float32(123456.0)


@pytest.mark.parametrize("rows,k,n,layout", [
    (1, 4096, 8192, "native"),   # 16 columns x 16 units = 256 units per tile: split units over two waves
    (1, 4096, 8192, "lanes"),
    (1, 2048, 16384, "lanes"),   # 32 columns x 8 units, the same split form
    (1, 4096, 16384, "lanes"),   # 512 units per tile: the two-units-per-thread lane kernel
    (3, 2048, 700, "lanes"),     # three rows over lane weights
    (2, 288, 100, "native"),     # 9 blocks per row (not a multiple of 8): the general kernel
    (3, 288, 70, "native"),
])
def test_q4_0_single_linear_forms_bit_exact(rows: int, k: int, n: int, layout: str) -> None:
    from qpu_xla_amd.kernels import ggml_q4_0 as q4

    rng = np.random.default_rng(rows * 100000 + k + n)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((rows, k), dtype=np.float32)
    wq, xq = oracle.quantize_q4_0_blocks(w), oracle.quantize_q8_0_blocks(x)
    ncols = n - 4
    out = torch.full((rows, ncols + 16), float(SENTINEL), device="cuda")
    if layout == "lanes":
        q4.ggml_q4_0_q8_0_lane_linear(dev(xq), q4.pack_ggml_q4_0_lane_weights(dev(wq)), out, weight_column_start=4,
                                      output_column_start=16, column_count=ncols)
    else:
        q4.ggml_q4_0_q8_0_linear(dev(xq), dev(wq), out, weight_column_start=4, output_column_start=16,
                                 column_count=ncols)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got[:, :16], SENTINEL)
    np.testing.assert_array_equal(got[:, 16:], oracle.q4_0_q8_0_reference(xq, wq[4:]))


@pytest.mark.parametrize("rows", [2, 3])
def test_q4_0_block_dots_general_kernel(rows: int) -> None:
    # The debug block-dot path on rows whose blocks are not a multiple of 8.
    from qpu_xla_amd.kernels import ggml_q4_0 as q4

    rng = np.random.default_rng(77 + rows)
    k, n = 288, 48
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((rows, k), dtype=np.float32)
    wq, xq = oracle.quantize_q4_0_blocks(w), oracle.quantize_q8_0_blocks(x)
    dots = q4.ggml_q4_0_q8_0_block_dots(dev(xq), dev(wq)).cpu().numpy()
    np.testing.assert_array_equal(dots, oracle.q4_0_q8_0_block_dots(xq, wq))


_STAGE_WEIGHTS: dict = {}


def _stage_weight(k: int):
    """One quantised [6144, K] weight per K, shared by the stage-batch cases (oracle quantisation is slow)."""
    if k not in _STAGE_WEIGHTS:
        rng = np.random.default_rng(8000 + k)
        w = (rng.standard_normal((6144, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        _STAGE_WEIGHTS[k] = oracle.quantize_q4_0_blocks(w)
    return _STAGE_WEIGHTS[k]


@pytest.mark.parametrize("layout", ["native", "lanes", "mixed"])
@pytest.mark.parametrize("count", [1, 5])
@pytest.mark.parametrize("n", [1024, 6144])
@pytest.mark.parametrize("k", [2048, 4096, 6144])
def test_fp32_row_stage_batches_every_prefetch_form(k: int, n: int, count: int, layout: str) -> None:
    # One-row batches of fp32 activations (quantised inside each workgroup,
    # the row requested before the weights as 2, 4 or 6 chunks per thread of
    # 256, i.e. 1, 2 or 3 of 512), tiles narrowed until they fill the chip and
    # each unit split over four or two waves, tasks in the kernel arguments
    # (one) or in device tables (five), over native, lane or mixed weights.
    from qpu_xla_amd.kernels import ggml_q4_0 as q4

    wq_all = _stage_weight(k)
    rng = np.random.default_rng(k + n + count)
    tasks, expected = [], []
    for i in range(count):
        ncols = n // count - 4 * i
        wcol0 = 8 * i
        wq = wq_all[wcol0:wcol0 + ncols]
        x = rng.standard_normal((1, k), dtype=np.float32)
        weight = dev(wq_all)
        if layout == "lanes" or (layout == "mixed" and i % 2 == 0):
            weight = q4.pack_ggml_q4_0_lane_weights(weight)
        tasks.append({"weight": weight, "x": dev(x), "weight_column_start": wcol0, "output_column_start": 16,
                      "column_count": ncols,
                      "destination": torch.full((1, ncols + 16), float(SENTINEL), device="cuda")})
        expected.append(oracle.q4_0_q8_0_reference(oracle.quantize_q8_0_blocks(x), wq))
    with q4.Q4_0LinearBatch(tasks) as batch:
        batch.launch()
        torch.cuda.synchronize()
    for t, want in zip(tasks, expected):
        got = t["destination"].cpu().numpy()
        np.testing.assert_array_equal(got[:, :16], SENTINEL)
        np.testing.assert_array_equal(got[:, 16:], want)


@pytest.mark.parametrize("layout", ["native", "lanes"])
@pytest.mark.parametrize("k,n", [(2048, 20480), (4096, 9216), (6144, 6144)])
def test_fp32_row_batch_of_full_width_tiles(k: int, n: int, layout: str) -> None:
    # Enough columns for one full-width tile per CU (256 to 1024 work items):
    # two units per thread, the fp32 row still requested before the weights.
    from qpu_xla_amd.kernels import ggml_q4_0 as q4

    rng = np.random.default_rng(k * 3 + n)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    wq = oracle.quantize_q4_0_blocks(w)
    x = rng.standard_normal((1, k), dtype=np.float32)
    weight = dev(wq)
    if layout == "lanes":
        weight = q4.pack_ggml_q4_0_lane_weights(weight)
    task = {"weight": weight, "x": dev(x), "weight_column_start": 0, "output_column_start": 0, "column_count": n,
            "destination": torch.full((1, n), float(SENTINEL), device="cuda")}
    with q4.Q4_0LinearBatch([task]) as batch:
        assert 256 <= batch.work_items <= 1024
        batch.launch()
        torch.cuda.synchronize()
    np.testing.assert_array_equal(task["destination"].cpu().numpy(),
                                  oracle.q4_0_q8_0_reference(oracle.quantize_q8_0_blocks(x), wq))


def _q8_operands(seed: int, rows: int, outputs: int, blocks: int):
    rng = np.random.default_rng(seed)
    act = oracle.pack_q8_0_blocks(rng.uniform(-0.1, 0.1, (rows, blocks)).astype(np.float16),
                                  rng.integers(-128, 128, (rows, blocks, 32)))
    wt = oracle.pack_q8_0_blocks(rng.uniform(-0.1, 0.1, (outputs, blocks)).astype(np.float16),
                                 rng.integers(-128, 128, (outputs, blocks, 32)))
    return act, wt


@pytest.mark.parametrize("rows,blocks,weight_offset", [
    (1, 3, 0),    # one row, blocks % 8 != 0: one block per thread
    (2, 5, 0),    # two rows, one block per thread
    (3, 16, 0),   # three rows, eight blocks per thread (16-byte aligned weight rows)
    (2, 8, 2),    # weights 2 bytes past a 16-byte boundary: one block per thread
])
def test_q8_0_linear_row_counts_and_weight_alignment(rows: int, blocks: int, weight_offset: int) -> None:
    # The Q8_0 x Q8_0 linear at one, two and three rows per workgroup, with
    # and without the eight-blocks-per-thread weight reads (those need
    # blocks % 8 == 0 and 16-byte aligned weight rows).
    from qpu_xla_amd.kernels import ggml_q8_0 as q8

    act, wt = _q8_operands(5300 + rows * 10 + blocks, rows, 96, blocks)
    storage = torch.zeros(wt.size + weight_offset, dtype=torch.uint8, device="cuda")
    weight = storage[weight_offset:].view(wt.shape)
    weight.copy_(torch.from_numpy(wt))
    assert weight.is_contiguous() and (weight.data_ptr() % 16 != 0) == (weight_offset != 0)
    out = torch.full((rows, 80 + 16), float(SENTINEL), device="cuda")
    q8.ggml_q8_0_q8_0_linear(dev(act), weight, out, weight_column_start=7, output_column_start=16, column_count=80)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got[:, :16], SENTINEL)
    np.testing.assert_array_equal(got[:, 16:], oracle.q8_0_q8_0_reference(act, wt[7:87]))


def _offset_rows(values: np.ndarray) -> torch.Tensor:
    # A view whose rows start 4 bytes into an allocation with one spare
    # column: neither the base pointer nor the row stride is 16-byte aligned.
    rows, columns = values.shape
    base = torch.zeros((rows, columns + 1), dtype=torch.float32, device="cuda")
    view = base[:, 1:]
    view.copy_(torch.from_numpy(values))
    assert view.data_ptr() % 16 != 0 and (view.stride(0) * 4) % 16 != 0
    return view


@pytest.mark.parametrize("rows,columns", [(3, 96), (17, 2048)])
def test_quantisers_on_unaligned_rows_bit_exact(rows: int, columns: int) -> None:
    # The scalar-load forms of the Q8_0 and Q4_0 quantisers.
    from qpu_xla_amd.kernels.quantize import quantize_q4_0, quantize_q8_0

    rng = np.random.default_rng(rows + columns)
    x = rng.standard_normal((rows, columns), dtype=np.float32)
    x[0, :32] = 0.0  # an all-zero block
    np.testing.assert_array_equal(quantize_q8_0(_offset_rows(x)).cpu().numpy(), oracle.quantize_q8_0_blocks(x))
    np.testing.assert_array_equal(quantize_q4_0(_offset_rows(x)).cpu().numpy(), oracle.quantize_q4_0_blocks(x))


@pytest.mark.parametrize("rows,columns", [(5, 160), (64, 33 * 1024)])  # gather kernel; >= 65536 blocks: LDS band
def test_geglu_on_unaligned_rows_every_output_layout(rows: int, columns: int) -> None:
    # The scalar-load forms of both GEGLU kernels, writing native blocks and
    # split planes with four- and two-byte scales.
    from qpu_xla_amd.kernels import ggml_geglu_q8 as geglu

    rng = np.random.default_rng(rows * 7 + columns)
    gate = rng.normal(0.0, 1.5, (rows, columns)).astype(np.float32)
    up = rng.normal(0.0, 1.0, (rows, columns)).astype(np.float32)
    gate_d, up_d = _offset_rows(gate), _offset_rows(up)
    np.testing.assert_array_equal(geglu.ggml_geglu_q8_0(gate_d, up_d).cpu().numpy(),
                                  oracle.geglu_q8_0_reference(gate, up))
    words, planes = oracle.geglu_q8_0_split_reference(gate, up)
    for dtype, view in ((torch.int32, np.uint32), (torch.int16, np.uint16)):
        scales = torch.empty((rows, columns // 32), dtype=dtype, device="cuda")
        scales, values = geglu.ggml_geglu_q8_0_split(gate_d, up_d, scales=scales)
        np.testing.assert_array_equal(scales.cpu().numpy().view(view).astype(np.uint32), words)
        np.testing.assert_array_equal(values.cpu().numpy(), planes)


@pytest.mark.parametrize("rows,blocks,n,wcol0,ncols", [
    (4, 8, 96, 0, 96),        # 8 blocks: one wave along K, lanes 8..63 idle
    (4, 32, 200, 5, 190),     # ragged last tile, weight column offset
    (5, 64, 300, 3, 290),     # 64 blocks (one wave along K); the second row group has one row
    (8, 128, 520, 0, 520),    # 128 blocks: two waves along K, two full row groups
    (4, 176, 70, 0, 70),      # 176 blocks: four waves along K, the last one idle
    (3, 256, 40, 0, 40),      # 256 blocks (K = 8192): the largest with one block per lane
    (4, 264, 40, 0, 40),      # 264 blocks: two per lane, the second only for lanes 0..7 of wave 0
    (2, 344, 120, 7, 100),    # K = 11008 (a down projection), two blocks per lane
    (1, 512, 64, 0, 64),      # 512 blocks (K = 16384): the largest block-per-lane K
    (1, 520, 40, 0, 40),      # 520 blocks: past it, the unit form (one row: its LDS holds 4 rows only to K = 12288)
])
def test_q8_0_linear_block_per_lane_forms(rows: int, blocks: int, n: int, wcol0: int, ncols: int) -> None:
    # Up to 512 blocks the Q8_0 x Q8_0 linear takes one block per lane (one,
    # two or four waves along K, two blocks per lane past 256, the activation
    # blocks in registers); beyond, units of eight blocks per thread.  Both
    # sum the same block terms in block order.
    from qpu_xla_amd.kernels import ggml_q8_0 as q8

    act, wt = _q8_operands(5400 + rows + blocks, rows, n, blocks)
    out = torch.full((rows, ncols + 16), float(SENTINEL), device="cuda")
    q8.ggml_q8_0_q8_0_linear(dev(act), dev(wt), out, weight_column_start=wcol0, output_column_start=16,
                             column_count=ncols)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got[:, :16], SENTINEL)
    np.testing.assert_array_equal(got[:, 16:], oracle.q8_0_q8_0_reference(act, wt[wcol0:wcol0 + ncols]))


def test_geglu_band_two_blocks_per_pass_every_output_layout() -> None:
    # At least 2^18 blocks: the band kernel takes two blocks per 8-lane group
    # and pass (fewer take one, as every smaller GEGLU case here).
    from qpu_xla_amd.kernels import ggml_geglu_q8 as geglu

    rows, columns = 1600, 5632
    assert rows * columns // 32 >= 1 << 18
    rng = np.random.default_rng(5501)
    gate = rng.normal(0.0, 1.0, (rows, columns)).astype(np.float32)
    up = rng.normal(0.0, 1.0, (rows, columns)).astype(np.float32)
    np.testing.assert_array_equal(geglu.ggml_geglu_q8_0(dev(gate), dev(up)).cpu().numpy(),
                                  oracle.geglu_q8_0_reference(gate, up))
    words, planes = oracle.geglu_q8_0_split_reference(gate, up)
    for dtype, view in ((torch.int32, np.uint32), (torch.int16, np.uint16)):
        scales = torch.empty((rows, columns // 32), dtype=dtype, device="cuda")
        scales, values = geglu.ggml_geglu_q8_0_split(dev(gate), dev(up), scales=scales)
        np.testing.assert_array_equal(scales.cpu().numpy().view(view).astype(np.uint32), words)
        np.testing.assert_array_equal(values.cpu().numpy(), planes)


@pytest.mark.parametrize("rows,blocks,n,wcol0,ncols,weight_offset", [
    (2, 65, 40, 0, 40, 0),      # two rows spread past 64 blocks
    (3, 64, 40, 0, 40, 0),      # three rows of 64 blocks: still the unit kernels
    (4, 65, 8192, 0, 8192, 0),  # four rows over 8192 columns spread past 64 blocks
    (4, 65, 8191, 0, 8191, 0),  # one column fewer: the unit kernels
    (5, 65, 40, 0, 40, 0),      # five rows spread past 64 blocks
    (12, 100, 50, 3, 40, 0),    # twelve rows: row groups of four
    (15, 130, 30, 0, 30, 2),    # fifteen rows, the most: a last row group of three; weights 2 bytes off
    (2, 65, 1, 0, 1, 0),        # one column
    (1, 129, 64, 0, 64, 0),     # one row of 129 blocks: still the split kernel (one row spreads past 256)
    (1, 300, 64, 0, 64, 0),     # one row, two blocks per lane
    (2, 176, 2048, 0, 2048, 0),  # K = 5632 (TinyLlama down), two rows: one block per lane
    (3, 200, 50, 0, 50, 0),     # three rows, one block per lane
    (2, 300, 60, 1, 50, 0),     # two rows, two blocks per lane
    (2, 600, 30, 0, 30, 0),     # two rows, three blocks per lane
    (3, 700, 30, 0, 30, 2),     # three rows, three blocks per lane, weights 2 bytes off
    (4, 256, 100, 3, 90, 0),    # K = 8192, the last count with one block per lane
    (3, 257, 40, 0, 40, 2),     # two blocks per lane; weights 2 bytes past a 16-byte boundary
    (4, 344, 300, 10, 280, 0),  # K = 11008 (Llama-7B down), four rows
    (5, 448, 70, 0, 70, 0),     # K = 14336, a second row group of one row
    (1, 513, 40, 0, 40, 0),     # three blocks per lane
    (4, 768, 33, 0, 33, 0),     # K = 24576: the largest spread over lanes
    (1, 776, 40, 0, 40, 0),     # past it: the unit kernels
])
def test_q4_0_native_linear_long_rows_blocks_spread_over_lanes(rows: int, blocks: int, n: int, wcol0: int, ncols: int,
                                                               weight_offset: int) -> None:
    # Native Q4_0 rows longer than 64 blocks (128 for four activation rows
    # over fewer than 8192 columns, 256 for one row) and up to 15 activation
    # rows: each lane takes
    # blocks kw * 64 + l (+ 256, + 512), the activation blocks and -8 * sum(a)
    # in registers; the block terms are summed in block order.
    rng = np.random.default_rng(5600 + rows * 7 + blocks)
    w = (rng.standard_normal((n, blocks * 32), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    wq = oracle.quantize_q4_0_blocks(w)
    act = oracle.quantize_q8_0_blocks(rng.standard_normal((rows, blocks * 32), dtype=np.float32))
    storage = torch.zeros(wq.size + weight_offset, dtype=torch.uint8, device="cuda")
    weight = storage[weight_offset:].view(wq.shape)
    weight.copy_(torch.from_numpy(wq))
    out = torch.full((rows, ncols + 16), float(SENTINEL), device="cuda")
    ggml_q4_0_q8_0_linear(dev(act), weight, out, weight_column_start=wcol0, output_column_start=16,
                          column_count=ncols)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got[:, :16], SENTINEL)
    np.testing.assert_array_equal(got[:, 16:], oracle.q4_0_q8_0_reference(act, wq[wcol0:wcol0 + ncols]))
