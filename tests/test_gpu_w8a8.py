"""GPU parity of the W8A8 int8 MFMA GEMM, its epilogue and the whole linear (bit-exact)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import load_golden
from qpu_xla_amd import DependencyError, Queue
from qpu_xla_amd.kernels import gemm_int8, gemv_int8, w8a8_epilogue
from qpu_xla_amd.quantization import PreparedW8A8Linear, QuantizedMatrixInt8, quantize_per_output_channel_int8, w8a8_linear

pytestmark = pytest.mark.gpu


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def words(a: np.ndarray) -> torch.Tensor:
    return dev(np.ascontiguousarray(a).view(np.int32))


def test_native_w8a8_smoke_kat_through_gemv_kernel() -> None:
    g = load_golden("kat_w8a8")
    left, right = oracle.pack_int8_gemm_operands(g["activation"], g["weight_kn"])
    destination = torch.full((1, 16), -1, dtype=torch.int32, device="cuda")
    with Queue() as queue:
        queue.submit(gemv_int8.W8A8_GEMV_KERNEL, (words(left), words(right), destination), grid=(1, 1, 1)).wait()
    np.testing.assert_array_equal(destination.cpu().numpy(), g["expected"])


@pytest.mark.parametrize("shape", [(16, 16, 16), (32, 64, 32)])
def test_tiled_gemm_packed_operands_exact(shape) -> None:
    # tests/test_qpu_xla_gemm_int8.py:28-54 (seed 91 + q).
    p, q, r = shape
    rng = np.random.default_rng(91 + q)
    left_v = rng.integers(-127, 128, size=(p, q), dtype=np.int8)
    right_v = rng.integers(-127, 128, size=(q, r), dtype=np.int8)
    left, right = oracle.pack_int8_gemm_operands(left_v, right_v)
    destination = torch.empty((p, r), dtype=torch.int32, device="cuda")
    with Queue() as queue:
        queue.submit(gemm_int8.TILED_W8A8_GEMM_KERNEL, (words(left), words(right), destination),
                     grid=(r // 16, p // 16, 1)).wait()
    expected = (left_v.astype(np.int64) @ right_v.astype(np.int64)).astype(np.int32)
    np.testing.assert_array_equal(destination.cpu().numpy(), expected)


def test_fused_dequantize_fixture_bit_exact() -> None:
    # tests/test_qpu_xla_gemm_int8.py:57-92 (seed 1765), assert_array_equal as the reference does.
    g = load_golden("oracle_w8a8_fused_seed1765")
    left, right = oracle.pack_int8_gemm_operands(g["left"], g["right"])
    p, r = g["expected"].shape
    destination = torch.empty((p, r), dtype=torch.float32, device="cuda")
    with Queue() as queue:
        queue.submit(
            gemm_int8.TILED_W8A8_GEMM_DEQUANTIZE_KERNEL,
            (words(left), words(right), dev(g["row_scales"]), dev(g["column_scales"]), destination),
            grid=(r // 16, p // 16, 1),
        ).wait()
    np.testing.assert_array_equal(destination.cpu().numpy(), g["expected"])
    # Same through the natural [N, K] weight layout.
    out = gemm_int8.w8a8_gemm_dequantize(dev(g["left"]), dev(np.ascontiguousarray(g["right"].T)),
                                         dev(g["row_scales"]), dev(g["column_scales"]))
    np.testing.assert_array_equal(out.cpu().numpy(), g["expected"])


@pytest.mark.parametrize(
    "m,n,k",
    [(1, 16, 16), (7, 33, 48), (129, 257, 64), (128, 128, 4096), (300, 1000, 1040), (1, 4096, 14336), (64, 14336, 4096),
     # >= 256 tiles of 256 x 256 with K % 64 == 0: the large-tile kernel, with
     # partial edge tiles (N % 4 != 0 among them) and one to three K stages.
     (4000, 4100, 1024), (4096, 4096, 256), (4352, 4096, 128), (4096, 4098, 64), (4100, 4096, 192)],
)
def test_gemm_i32_random_shapes_exact(m: int, n: int, k: int) -> None:
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    out = gemm_int8.w8a8_gemm_i32(dev(a), dev(w))
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.int8_gemm_i32(a, w))


def test_mid_size_tiles_both_layouts_and_epilogue_exact() -> None:
    # Fewer 256 x 256 tiles than CUs but at least as many 128 x 128 ones: the
    # 128 x 128 kernel, over [N, K] weights with ragged M, N and a K that is
    # not a multiple of its 64-byte stage (int32 and fused epilogue), and over
    # the packed-K4 [K/4, N] words of the reference's tiled contract.
    rng = np.random.default_rng(1280)
    m, n, k = 520, 8200, 208
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    want = oracle.int8_gemm_i32(a, w)
    np.testing.assert_array_equal(gemm_int8.w8a8_gemm_i32(dev(a), dev(w)).cpu().numpy(), want)
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    out = gemm_int8.w8a8_gemm_dequantize(dev(a), dev(w), dev(sa), dev(sw), dev(bias)).cpu().numpy()
    np.testing.assert_array_equal(out, oracle.dequantize_epilogue(want, sa, sw, bias))
    p_, q_, r_ = 512, 208, 8192
    left_v = rng.integers(-127, 128, size=(p_, q_), dtype=np.int8)
    right_v = rng.integers(-127, 128, size=(q_, r_), dtype=np.int8)
    left, right = oracle.pack_int8_gemm_operands(left_v, right_v)
    destination = torch.empty((p_, r_), dtype=torch.int32, device="cuda")
    with Queue() as queue:
        queue.submit(gemm_int8.TILED_W8A8_GEMM_KERNEL, (words(left), words(right), destination),
                     grid=(r_ // 16, p_ // 16, 1)).wait()
    np.testing.assert_array_equal(destination.cpu().numpy(), (left_v.astype(np.int64) @ right_v.astype(np.int64)).astype(np.int32))


def test_streaming_kernel_fused_epilogue_on_edge_tiles_bit_exact() -> None:
    rng = np.random.default_rng(2718)
    m, n, k = 4000, 4100, 512
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    out = gemm_int8.w8a8_gemm_dequantize(dev(a), dev(w), dev(sa), dev(sw), dev(bias)).cpu().numpy()
    rows = np.array([0, 1, 255, 256, 3839, 3840, 3999])
    expected = oracle.dequantize_epilogue(oracle.int8_gemm_i32(a[rows], w), sa[rows], sw, bias)
    np.testing.assert_array_equal(out[rows], expected)


@pytest.mark.parametrize("m,n,k", [(1, 16, 16), (1, 33, 48), (2, 100, 4096), (3, 4096, 2048), (4, 17, 1040),
                                   (1, 14336, 4096), (1, 4096, 14336), (4, 64, 14336)])
def test_gemv_rows_exact_both_layouts_and_epilogue(m: int, n: int, k: int) -> None:
    # M <= 4 runs the dot4 GEMV kernels (weight [N, K] or packed K4 [K/4, N]).
    rng = np.random.default_rng(m * 1000 + n + k)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    expected = oracle.int8_gemm_i32(a, w)
    np.testing.assert_array_equal(gemm_int8.w8a8_gemm_i32(dev(a), dev(w)).cpu().numpy(), expected)
    if n % 4 == 0:
        left, right = oracle.pack_int8_gemm_operands(a, np.ascontiguousarray(w.T))
        out = torch.empty((m, n), dtype=torch.int32, device="cuda")
        from qpu_xla_amd import _lib
        from qpu_xla_amd._tensors import ptr, row_stride

        lw, rw = words(left), words(right)
        _lib.call("qxt_w8a8_gemm_i32", ptr(lw), row_stride(lw), ptr(rw), row_stride(rw), ptr(out), row_stride(out),
                  m, n, k, _lib.WEIGHT_K4N, None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), expected)
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    y = gemm_int8.w8a8_gemm_dequantize(dev(a), dev(w), dev(sa), dev(sw), dev(bias)).cpu().numpy()
    np.testing.assert_array_equal(y, oracle.dequantize_epilogue(expected, sa, sw, bias))


@pytest.mark.parametrize("m,n,k", [(1, 16, 16), (1, 4096, 14336), (2, 100, 4096), (3, 33, 2048), (4, 14336, 4096),
                                   (3, 70, 4112), (4, 300, 14336), (3, 4096, 14336)])
@pytest.mark.parametrize("floor", [True, False])
def test_small_m_linear_quantises_in_the_gemv_kernel_bit_exact(m: int, n: int, k: int, floor: bool) -> None:
    # M <= 2, or K > 4096 over at most 48 MiB of weights: one launch
    # quantises the rows inside every GEMV workgroup; other three- or four-row
    # problems take the row pre-pass and the unfused GEMV.  Either way the
    # workspaces receive the int8 rows and scales.
    from qpu_xla_amd import _lib
    from qpu_xla_amd._tensors import ptr, row_stride

    rng = np.random.default_rng(7000 + m * 10 + k)
    x = rng.standard_normal((m, k), dtype=np.float32)
    if k >= 64:
        x[:, rng.choice(k, max(1, k // 1000), replace=False)] *= 20.0
    x[0, :4] = [0.5, -0.5, 1.5, 2.5]
    wf = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    qw, sw = oracle.quantize_per_output_channel_int8(wf)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    xd = dev(x)
    qa = torch.full((m, k), 99, dtype=torch.int8, device="cuda")
    sa = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    w_d, sw_d, b_d = dev(qw), dev(sw), dev(bias)
    flags = 0 if floor else _lib.QUANT_NO_SCALE_FLOOR
    _lib.call("qxt_w8a8_linear", ptr(xd), row_stride(xd), ptr(qa), row_stride(qa), ptr(sa), ptr(w_d), row_stride(w_d),
              ptr(sw_d), ptr(b_d), ptr(y), row_stride(y), m, n, k, _lib.WEIGHT_NK, flags, None)
    torch.cuda.synchronize()
    qa_ref, sa_ref = oracle.quantize_rows_int8(x, floor=floor)
    np.testing.assert_array_equal(qa.cpu().numpy(), qa_ref)
    np.testing.assert_array_equal(sa.cpu().numpy(), sa_ref)
    expected = oracle.dequantize_epilogue(oracle.int8_gemm_i32(qa_ref, qw), sa_ref, sw, bias)
    np.testing.assert_array_equal(y.cpu().numpy(), expected)


def test_large_tile_gemm_over_several_rounds_with_edge_tile_exact() -> None:
    # 16 x 56 tiles of 256 x 256 (several rounds on a 256-CU device), the last
    # column of tiles partial; int32 accumulators and the fused epilogue.
    rng = np.random.default_rng(2720)
    m, n, k = 4096, 14336 - 64, 128
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    out = gemm_int8.w8a8_gemm_i32(dev(a), dev(w)).cpu().numpy()
    np.testing.assert_array_equal(out, oracle.int8_gemm_i32(a, w))
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    y = gemm_int8.w8a8_gemm_dequantize(dev(a), dev(w), dev(sa), dev(sw), dev(bias)).cpu().numpy()
    np.testing.assert_array_equal(y, oracle.dequantize_epilogue(out, sa, sw, bias))


def test_large_tile_epilogue_with_unaligned_output_rows_bit_exact() -> None:
    # Output rows 4 * 4099 bytes apart: not 16-byte aligned, so the row-store
    # epilogue writes element by element; the padding column stays untouched.
    rng = np.random.default_rng(2719)
    m, n, k = 4096, 4096, 128
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    storage = torch.full((m, n + 3), -7.0, dtype=torch.float32, device="cuda")
    out = storage[:, :n]
    gemm_int8.w8a8_gemm_dequantize(dev(a), dev(w), dev(sa), dev(sw), dev(bias), out=out)
    got = storage.cpu().numpy()
    rows = np.array([0, 3, 127, 128, 255, 2048, 4095])
    expected = oracle.dequantize_epilogue(oracle.int8_gemm_i32(a[rows], w), sa[rows], sw, bias)
    np.testing.assert_array_equal(got[rows, :n], expected)
    np.testing.assert_array_equal(got[:, n:], -7.0)


def test_gemm_i32_extreme_accumulators_exact() -> None:
    k = 4096
    a = np.full((32, k), 127, np.int8)
    a[1::2] = -127
    w = np.full((32, k), 127, np.int8)
    out = gemm_int8.w8a8_gemm_i32(dev(a), dev(w)).cpu().numpy()
    assert out[0, 0] == k * 127 * 127 and out[1, 0] == -k * 127 * 127
    np.testing.assert_array_equal(out, oracle.int8_gemm_i32(a, w))


def test_epilogue_rounds_each_step_and_adds_bias_separately() -> None:
    s = np.full(16, 1 + 2.0**-12, np.float32)
    a = np.zeros((16, 16), np.int8)
    a[:, 0] = 1
    w = np.zeros((16, 16), np.int8)
    w[:, 0] = 1
    bias = np.full(16, -1.0, np.float32)
    out = gemm_int8.w8a8_gemm_dequantize(dev(a), dev(w), dev(s), dev(s), dev(bias)).cpu().numpy()
    np.testing.assert_array_equal(out, np.full((16, 16), 2.0**-11, np.float32))
    acc = torch.ones((16, 16), dtype=torch.int32, device="cuda")
    out2 = w8a8_epilogue.w8a8_dequantize(acc, dev(s), dev(s), dev(bias)).cpu().numpy()
    np.testing.assert_array_equal(out2, out)


def test_standalone_dequantize_kernel_contract() -> None:
    rng = np.random.default_rng(9)
    acc = rng.integers(-2**24, 2**24, size=(32, 48), dtype=np.int32)
    sa = rng.uniform(0.001, 0.1, 32).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, 48).astype(np.float32)
    destination = torch.empty((32, 48), dtype=torch.float32, device="cuda")
    with Queue() as queue:
        queue.submit(w8a8_epilogue.W8A8_DEQUANTIZE_KERNEL, (dev(acc), dev(sa), dev(sw), destination),
                     grid=(3, 2, 1)).wait()
    np.testing.assert_array_equal(destination.cpu().numpy(), oracle.dequantize_epilogue(acc, sa, sw))


@pytest.mark.parametrize("m,k,n,seed", [(512, 512, 512, 1), (1, 512, 512, 1731), (37, 2048, 5632, 5)])
def test_whole_linear_bit_exact(m: int, k: int, n: int, seed: int) -> None:
    # cfg1 (M=K=N=512; x ~ N(0,1), W ~ N(0,0.05): weight floor active, bias ~ N(0,0.1)).
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    x = rng.standard_normal((m, k), dtype=np.float32)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    weight = quantize_per_output_channel_int8(dev(w))
    qw, sw = oracle.quantize_per_output_channel_int8(w)
    np.testing.assert_array_equal(weight.values.cpu().numpy(), qw)
    np.testing.assert_array_equal(weight.scales.cpu().numpy(), sw)
    y = w8a8_linear(dev(x), weight, dev(bias)).cpu().numpy()
    np.testing.assert_array_equal(y, oracle.w8a8_linear_reference(x, qw, sw, bias))


@pytest.mark.parametrize("k,n,kernel", [(4096, 14336, "w8a8_gemm_stream_kernel"),
                                        (14336, 4096, "w8a8_gemm_stream_kernel")], ids=["gate_up", "down"])
def test_cfg4_shape_sampled_rows_bit_exact(k: int, n: int, kernel: str) -> None:
    # cfg4 (M=4096; gate_up K=4096, N=14336 and down K=14336, N=4096; seed 4;
    # 0.1% outlier channels x20): all rows on the GPU through the 256 x 256
    # tiles (gate_up's 896 tiles in three and a half rounds, down's 256 with
    # 112 K stages one per workgroup), the oracle on 48 sampled rows (the oracle's
    # cost, not the kernel's, sets the sample).  Mirrors the reference's
    # assert_array_equal at tests/test_qpu_xla_gemm_int8.py:57-92.
    from qpu_xla_amd import _lib

    rng = np.random.default_rng(4)
    m = 4096
    x = rng.standard_normal((m, k), dtype=np.float32)
    x[:, rng.choice(k, round(0.001 * k), replace=False)] *= np.float32(20.0)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    weight = quantize_per_output_channel_int8(dev(w))
    xd, bd = dev(x), dev(bias)
    torch.cuda.synchronize()
    with _lib.launch_timing() as timing:
        y = w8a8_linear(xd, weight, bd)
    assert kernel in [name for name, _ in timing.records]
    rows = np.sort(rng.choice(m, 48, replace=False))
    rows[0], rows[-1] = 0, m - 1
    qw, sw = oracle.quantize_per_output_channel_int8(w)
    np.testing.assert_array_equal(weight.values.cpu().numpy(), qw)
    np.testing.assert_array_equal(weight.scales.cpu().numpy(), sw)
    expected = oracle.w8a8_linear_reference(x[rows], qw, sw, bias)
    np.testing.assert_array_equal(y[torch.from_numpy(rows).cuda()].cpu().numpy(), expected)


def test_prepared_plan_binds_queue_pads_k_and_matches_oracle() -> None:
    rng = np.random.default_rng(77)
    k, n = 100, 48  # K not a multiple of 16: the plan pads with zero columns
    w = rng.standard_normal((n, k), dtype=np.float32)
    x = rng.standard_normal((5, k), dtype=np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    qw, sw = oracle.quantize_per_output_channel_int8(w)
    weight = QuantizedMatrixInt8(dev(qw), dev(sw))
    destination = torch.empty((5, n), dtype=torch.float32, device="cuda")
    with Queue() as queue, Queue() as other, PreparedW8A8Linear(weight, max_batch=8, bias=dev(bias)) as plan:
        plan.execute(destination, dev(x), queue=queue).wait()
        np.testing.assert_array_equal(destination.cpu().numpy(), oracle.w8a8_linear_reference(x, qw, sw, bias))
        with pytest.raises(DependencyError):
            plan.execute(destination, dev(x), queue=other)
        with pytest.raises(ValueError):
            plan.execute(torch.empty((9, n), device="cuda"), dev(np.zeros((9, k), np.float32)), queue=queue)


def _plan_case(seed: int, m: int, k: int, n: int):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k), dtype=np.float32)
    x = rng.standard_normal((m, k), dtype=np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    qw, sw = oracle.quantize_per_output_channel_int8(w)
    return x, QuantizedMatrixInt8(dev(qw), dev(sw)), bias, oracle.w8a8_linear_reference(x, qw, sw, bias)


@pytest.mark.parametrize("batch", [1, 17])
def test_prepared_hybrid_output_split_on_two_streams_bit_exact(batch: int) -> None:
    # Reference: test_prepared_w8a8_hybrid_output_split_matches_dynamic_reference_on_qpu (K=32, N=48, split 16).
    x, weight, bias, expected = _plan_case(801 + batch, batch, 32, 48)
    destination = torch.full((batch, 48), float("nan"), device="cuda")
    with Queue() as first, Queue() as second, PreparedW8A8Linear(weight, max_batch=max(16, batch),
                                                                 bias=dev(bias)) as plan:
        event = plan.execute_hybrid(destination, dev(x), qpu_queue=first, cpu_queue=second, qpu_outputs=16)
        event.wait()
        assert event.name == "gfx950.w8a8_linear.hybrid_join"
        np.testing.assert_array_equal(destination.cpu().numpy(), expected)
        with pytest.raises(ValueError, match="aligned"):
            plan.execute_hybrid(destination, dev(x), qpu_queue=first, cpu_queue=second, qpu_outputs=48)
        with pytest.raises(DependencyError):
            plan.execute_hybrid(destination, dev(x), qpu_queue=first, cpu_queue=first, qpu_outputs=16)


def test_prepared_hybrid_row_split_pads_k_bit_exact() -> None:
    # Reference: test_prepared_w8a8_hybrid_row_split_matches_dynamic_reference_on_qpu (31 x 20 -> 19, split 16).
    x, weight, bias, expected = _plan_case(1907, 31, 20, 19)
    destination = torch.full((31, 19), float("nan"), device="cuda")
    with Queue() as first, Queue() as second, PreparedW8A8Linear(weight, max_batch=32, bias=dev(bias)) as plan:
        plan.execute_hybrid_rows(destination, dev(x), qpu_queue=first, cpu_queue=second, qpu_rows=16).wait()
        np.testing.assert_array_equal(destination.cpu().numpy(), expected)
        # A strided source view goes through the plan's staging buffer.
        wide = dev(np.concatenate([x, x], axis=1))[:, :20]
        destination.fill_(float("nan"))
        plan.execute_hybrid_rows(destination, wide, qpu_queue=first, cpu_queue=second, qpu_rows=16).wait()
        np.testing.assert_array_equal(destination.cpu().numpy(), expected)


def test_prepared_execute_prepared_reads_the_activation_workspace() -> None:
    from qpu_xla_amd.kernels.quantize import quantize_rows_int8

    x, weight, bias, expected = _plan_case(1731, 3, 64, 32)
    destination = torch.empty((3, 32), device="cuda")
    with Queue() as queue, PreparedW8A8Linear(weight, max_batch=4, bias=dev(bias)) as plan:
        qa, sa = plan.activation_workspace
        with torch.cuda.stream(queue.stream):
            quantize_rows_int8(dev(x), out=qa, scales=sa, stream=queue)
        plan.execute_prepared(destination, batch=3, queue=queue).wait()
        np.testing.assert_array_equal(destination.cpu().numpy(), expected)


def test_calibrated_auto_selects_the_fastest_exact_partition_axis() -> None:
    # Reference: test_calibrated_w8a8_auto_selects_the_fastest_exact_partition_axis, with "gpu"
    # records in place of the VideoCore "qpu" ones.
    from qpu_xla_amd import Placement
    from qpu_xla_amd.candidates import (CandidateRecord, CandidateRegistry, CandidateStatus, CorrectnessEvidence,
                                        PartitionEvidence, PerformanceEvidence)
    from qpu_xla_amd.quantization import CalibratedW8A8Linear

    x, weight, _, _ = _plan_case(2921, 32, 16, 32)
    qw, sw = weight.values.cpu().numpy(), weight.scales.cpu().numpy()
    expected = oracle.w8a8_linear_reference(x, qw, sw, None)
    exact = CorrectnessEvidence("oracle", 1, True, 0.0, 0.0, 0.0, 0.0)

    def record(name, seconds, placement="gpu", partition=None):
        return CandidateRecord(name, "linear", "w8a8-i32-fp32", "row-major-packed-k4", "32x16x32", "hash",
                               CandidateStatus.SUPPORTED_WIN, exact, PerformanceEvidence("numpy", (0.010,), (seconds,)),
                               placement=placement, partition=partition)

    registry = CandidateRegistry((
        record("gpu", 0.004),
        record("hybrid-rows", 0.001, "hybrid", PartitionEvidence("rows", 16, 32, 16)),
        record("hybrid-outputs", 0.002, "hybrid", PartitionEvidence("outputs", 16, 32, 16)),
    ))
    destination = torch.empty((32, 32), device="cuda")
    with Queue() as first, Queue() as second, CalibratedW8A8Linear(weight, max_batch=32,
                                                                   candidates=registry) as plan:
        plan.execute(destination, dev(x), queue=first, cpu_queue=second).wait()
        assert plan.last_dispatch.record.name == "hybrid-rows"
        np.testing.assert_array_equal(destination.cpu().numpy(), expected)
        destination.fill_(float("nan"))
        plan.execute(destination, dev(x), queue=first, cpu_queue=second, qpu_outputs=16).wait()
        assert plan.last_dispatch.record.name == "hybrid-outputs"
        np.testing.assert_array_equal(destination.cpu().numpy(), expected)
        destination.fill_(float("nan"))
        event = plan.execute(destination, dev(x), queue=first)
        event.wait()
        assert plan.last_dispatch.record.name == "gpu" and event.name == "gfx950.w8a8_linear"
        np.testing.assert_array_equal(destination.cpu().numpy(), expected)
        with pytest.raises(ValueError, match="no CPU reference fallback"):
            plan.execute(destination[:31], dev(x[:31]), queue=first)
        with pytest.raises(ValueError, match="no CPU placement"):
            plan.execute(destination, dev(x), queue=first, placement=Placement.CPU)
    with CalibratedW8A8Linear(weight, max_batch=32, candidates=CandidateRegistry()) as empty:
        assert empty._gpu is None
        with pytest.raises(ValueError, match="no CPU reference fallback"):
            empty.execute(destination, dev(x), queue=Queue())


@pytest.mark.parametrize("layout", ["nk", "k4n"])
@pytest.mark.parametrize("m", [1, 2, 4])
@pytest.mark.parametrize("k", [8192, 8208, 16384])
def test_fused_rows_at_register_chunk_boundaries_bit_exact(layout: str, m: int, k: int) -> None:
    # The fused row quantiser holds K / (4 NT) 16-byte chunks per thread: K =
    # 8192 is the last K of 4 chunks on the 512-thread [N, K] kernel (and of 8
    # on the 256-thread K4N kernel), 8208 the first of the next size, 16384
    # fills 8 (16) chunks exactly.  (M = 4 at K = 16384 needs 64 KiB of rows
    # and runs the two-kernel path.)  Each row starts with the known-answer
    # row of tests/q8_0_kats.py, whose absmax is the row's absmax, so its
    # codes and scale are checked against literals as well as the oracle.
    import q8_0_kats
    from qpu_xla_amd import _lib
    from qpu_xla_amd._tensors import ptr, row_stride

    name, kat, _, scale_bits, codes = q8_0_kats.row_kats()[0]
    rng = np.random.default_rng(k + m)
    n = 96
    x = np.clip(rng.standard_normal((m, k), dtype=np.float32), -4.0, 4.0).astype(np.float32)
    x[:, : kat.size] = kat
    wf = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    qw, sw = oracle.quantize_per_output_channel_int8(wf)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    if layout == "nk":
        w_d, kind = dev(qw), _lib.WEIGHT_NK
    else:
        w_d, kind = words(np.ascontiguousarray(oracle.pack_int8_quads(qw).T)), _lib.WEIGHT_K4N
    xd, sw_d, b_d = dev(x), dev(sw), dev(bias)
    qa = torch.full((m, k), 99, dtype=torch.int8, device="cuda")
    sa = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    _lib.call("qxt_w8a8_linear", ptr(xd), row_stride(xd), ptr(qa), row_stride(qa), ptr(sa), ptr(w_d), row_stride(w_d),
              ptr(sw_d), ptr(b_d), ptr(y), row_stride(y), m, n, k, kind, 0, None)
    torch.cuda.synchronize()
    qa_ref, sa_ref = oracle.quantize_rows_int8(x)
    got_q, got_s = qa.cpu().numpy(), sa.cpu().numpy()
    np.testing.assert_array_equal(got_q, qa_ref)
    np.testing.assert_array_equal(got_s, sa_ref)
    for r in range(m):
        np.testing.assert_array_equal(got_q[r, : kat.size].astype(np.int64),
                                      q8_0_kats.expected_codes(codes, kat.size), err_msg=name)
        assert int(got_s[r : r + 1].view(np.uint32)[0]) == scale_bits
    expected = oracle.dequantize_epilogue(oracle.int8_gemm_i32(qa_ref, qw), sa_ref, sw, bias)
    np.testing.assert_array_equal(y.cpu().numpy(), expected)


def _fused_case(m: int, n: int, k: int, bias: bool, seed: int) -> None:
    from qpu_xla_amd import _lib
    from qpu_xla_amd._tensors import ptr, row_stride

    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=np.float32)
    x[:, rng.choice(k, max(1, k // 1000), replace=False)] *= 20.0
    qw = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sw = rng.uniform(0.0005, 0.002, n).astype(np.float32)
    b = rng.standard_normal(n, dtype=np.float32) if bias else None
    xd, w_d, sw_d = dev(x), dev(qw), dev(sw)
    b_d = dev(b) if bias else None
    qa = torch.full((m, k), 99, dtype=torch.int8, device="cuda")
    sa = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    _lib.call("qxt_w8a8_linear", ptr(xd), row_stride(xd), ptr(qa), row_stride(qa), ptr(sa), ptr(w_d), row_stride(w_d),
              ptr(sw_d), ptr(b_d) if bias else None, ptr(y), row_stride(y), m, n, k, _lib.WEIGHT_NK, 0, None)
    torch.cuda.synchronize()
    qa_ref, sa_ref = oracle.quantize_rows_int8(x)
    np.testing.assert_array_equal(qa.cpu().numpy(), qa_ref)
    np.testing.assert_array_equal(sa.cpu().numpy(), sa_ref)
    expected = oracle.dequantize_epilogue(oracle.int8_gemm_i32(qa_ref, qw), sa_ref, sw, b)
    np.testing.assert_array_equal(y.cpu().numpy(), expected)


# Column counts in units of the persistent form's waves: two 512-thread
# workgroups per CU, eight waves each.
def _waves() -> int:
    return 16 * torch.cuda.get_device_properties(0).multi_processor_count


@pytest.mark.parametrize("m,cols,k", [
    (1, (2, 0), 16),      # one row: exactly two columns per wave, one 16-byte chunk per column
    (1, (2, 3), 4112),    # ragged: a partial last kilobyte, three waves with a third column
    (1, (2, -1), 2048),   # one column short of two per wave: the one-column-per-wave kernel
    (1, (3, 1000), 4096),  # three or four columns per wave
    (1, (2, 5), 8208),    # rows of more than 8192 columns: eight row chunks per thread
    (1, (64, 0), 16),     # 64 columns per wave, the most the persistent form holds
    (1, (64, 1), 16),     # one more: the one-column-per-wave kernel
    (2, (0, 100), 4096),  # two rows: a grid of 13 workgroups, most waves without a column
    (2, (0, 3000), 4112),
    (2, (0, 520), 16384),  # the longest fused row
    (2, (0, 4096), 14336),
    (2, (64, 0), 16),
    (2, (64, 1), 16),
])
@pytest.mark.parametrize("bias", [True, False])
def test_fused_gemv_persistent_form_bit_exact(m: int, cols: tuple, k: int, bias: bool) -> None:
    # One or two fused rows over [N, K] weights: each workgroup quantises the
    # rows once, then every wave streams its columns gw, gw + W, ... with four
    # kilobyte loads in flight across column boundaries and stores them after
    # the last load.  N = per_wave * W + extra.
    per_wave, extra = cols
    n = per_wave * _waves() + extra
    _fused_case(m, n, k, bias, seed=8100 + m * 7 + k + per_wave)


@pytest.mark.parametrize("m,cols,k", [
    (1, (0, 7), 16),        # fewer columns than waves: a grid of one workgroup
    (1, (2, 3), 4112),      # ragged K: a partial last kilobyte
    (3, (0, 5000), 4096),
    (4, (0, 4096), 14336),  # four rows of 14 KB: two workgroups per CU fit the LDS
    (2, (1, 0), 8208),
    (4, (64, 0), 16),       # 64 columns per wave, the most the persistent form holds
    (4, (64, 1), 16),       # one more: the one-row-chunk kernel
])
@pytest.mark.parametrize("epilogue", ["i32", "dequantize", "dequantize_bias"])
def test_unfused_gemv_persistent_form_bit_exact(m: int, cols: tuple, k: int, epilogue: str) -> None:
    # Int8 rows given (qxt_w8a8_gemm_i32 / _dequantize at M <= 4): three
    # workgroups per CU load the rows once each, then every wave streams its
    # columns with three kilobyte loads in flight.  N = per_wave * W + extra,
    # W = 24 waves per CU.
    from qpu_xla_amd import _lib
    from qpu_xla_amd._tensors import ptr, row_stride

    per_wave, extra = cols
    n = per_wave * 24 * torch.cuda.get_device_properties(0).multi_processor_count + extra
    rng = np.random.default_rng(9100 + m * 13 + k + per_wave)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    expected = oracle.int8_gemm_i32(a, w)
    a_d, w_d = dev(a), dev(w)
    if epilogue == "i32":
        out = torch.full((m, n), -7, dtype=torch.int32, device="cuda")
        _lib.call("qxt_w8a8_gemm_i32", ptr(a_d), row_stride(a_d), ptr(w_d), row_stride(w_d), ptr(out),
                  row_stride(out), m, n, k, _lib.WEIGHT_NK, None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), expected)
        return
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32) if epilogue == "dequantize_bias" else None
    sa_d, sw_d = dev(sa), dev(sw)
    b_d = dev(bias) if bias is not None else None
    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    _lib.call("qxt_w8a8_gemm_dequantize", ptr(a_d), row_stride(a_d), ptr(w_d), row_stride(w_d), ptr(sa_d), ptr(sw_d),
              ptr(b_d) if b_d is not None else None, ptr(y), row_stride(y), m, n, k, _lib.WEIGHT_NK, None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), oracle.dequantize_epilogue(expected, sa, sw, bias))


@pytest.mark.parametrize("m,n,k", [(1, 9000, 4096), (2, 3000, 4112), (4, 9000, 4096), (3, 6000, 14336)])
def test_small_m_linear_padded_rows_bit_exact(m: int, n: int, k: int) -> None:
    # Row strides past the rows on every operand (fp32 input, int8 workspace,
    # weight, output): the persistent GEMV forms (fused for one and two rows,
    # over the pre-pass's int8 rows for three and four) address each row
    # through its stride.
    from qpu_xla_amd import _lib
    from qpu_xla_amd._tensors import ptr, row_stride

    rng = np.random.default_rng(9300 + m + k)
    x_full = rng.standard_normal((m, k + 20), dtype=np.float32)
    w_full = rng.integers(-127, 128, size=(n, k + 48), dtype=np.int8)
    x, qw = x_full[:, :k], w_full[:, :k]
    sw = rng.uniform(0.0005, 0.002, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    xd, wd = dev(x_full), dev(w_full)
    qa_full = torch.full((m, k + 32), 99, dtype=torch.int8, device="cuda")
    sa = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
    y_full = torch.full((m, n + 5), float("nan"), dtype=torch.float32, device="cuda")
    sw_d, b_d = dev(sw), dev(bias)
    _lib.call("qxt_w8a8_linear", ptr(xd), row_stride(xd), ptr(qa_full), row_stride(qa_full), ptr(sa), ptr(wd),
              row_stride(wd), ptr(sw_d), ptr(b_d), ptr(y_full), row_stride(y_full), m, n, k, _lib.WEIGHT_NK, 0, None)
    torch.cuda.synchronize()
    qa_ref, sa_ref = oracle.quantize_rows_int8(np.ascontiguousarray(x))
    got_q = qa_full.cpu().numpy()
    np.testing.assert_array_equal(got_q[:, :k], qa_ref)
    np.testing.assert_array_equal(got_q[:, k:], 99)
    np.testing.assert_array_equal(sa.cpu().numpy(), sa_ref)
    got_y = y_full.cpu().numpy()
    expected = oracle.dequantize_epilogue(oracle.int8_gemm_i32(qa_ref, np.ascontiguousarray(qw)), sa_ref, sw, bias)
    np.testing.assert_array_equal(got_y[:, :n], expected)
    assert np.isnan(got_y[:, n:]).all()


@pytest.mark.parametrize("m,n,k", [(1, 14336, 4096), (2, 4096, 14336), (4, 9000, 4096)])
def test_small_m_linear_graph_replays_bit_exact(m: int, n: int, k: int) -> None:
    # The persistent GEMV forms captured in a HIP graph (for four rows: the row
    # pre-pass and the GEMV over its int8 rows) and replayed three times, the
    # outputs and the int8 workspaces cleared by eager work between replays.
    from qpu_xla_amd import _lib
    from qpu_xla_amd._tensors import ptr, row_stride

    rng = np.random.default_rng(9400 + m)
    x = rng.standard_normal((m, k), dtype=np.float32)
    qw = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sw = rng.uniform(0.0005, 0.002, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    qa_ref, sa_ref = oracle.quantize_rows_int8(x)
    want = oracle.dequantize_epilogue(oracle.int8_gemm_i32(qa_ref, qw), sa_ref, sw, bias)
    xd, wd, sw_d, b_d = dev(x), dev(qw), dev(sw), dev(bias)
    qa = torch.empty((m, k), dtype=torch.int8, device="cuda")
    sa = torch.empty((m,), dtype=torch.float32, device="cuda")
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    capture = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=capture):
        _lib.call("qxt_w8a8_linear", ptr(xd), row_stride(xd), ptr(qa), row_stride(qa), ptr(sa), ptr(wd),
                  row_stride(wd), ptr(sw_d), ptr(b_d), ptr(y), row_stride(y), m, n, k, _lib.WEIGHT_NK, 0,
                  ctypes.c_void_p(capture.cuda_stream))
    for _ in range(3):
        y.fill_(float("nan"))
        qa.fill_(99)
        sa.fill_(-1.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(qa.cpu().numpy(), qa_ref)
        np.testing.assert_array_equal(sa.cpu().numpy(), sa_ref)
        np.testing.assert_array_equal(y.cpu().numpy(), want)


def _int8_case(seed: int, m: int, n: int, k: int):
    rng = np.random.default_rng(seed)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    return a, w, sa, sw, bias


def test_large_tile_graph_replays_and_two_streams_bit_exact() -> None:
    # The 256 x 256 stream kernel over 272 tiles (more than one round):
    # launches on two streams at once, then one launch captured in a graph and
    # replayed three times, every result checked in full.
    m, n, k = 4096, 4352, 256
    cases = [_int8_case(seed, m, n, k) for seed in (5, 6)]
    wants = [oracle.dequantize_epilogue(oracle.int8_gemm_i32(a, w), sa, sw, bias) for a, w, sa, sw, bias in cases]
    ops = [tuple(dev(t) for t in case) for case in cases]
    outs = [torch.full((m, n), float("nan"), device="cuda") for _ in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for _ in range(2):  # concurrent eager launches
        for (a, w, sa, sw, bias), out, stream in zip(ops, outs, streams):
            with torch.cuda.stream(stream):
                gemm_int8.w8a8_gemm_dequantize(a, w, sa, sw, bias, out=out, stream=stream)
        torch.cuda.synchronize()
        for out, want in zip(outs, wants):
            np.testing.assert_array_equal(out.cpu().numpy(), want)
            out.fill_(float("nan"))
        torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    a, w, sa, sw, bias = ops[0]
    capture = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=capture):
        gemm_int8.w8a8_gemm_dequantize(a, w, sa, sw, bias, out=outs[0], stream=capture)
    for _ in range(3):
        outs[0].fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(outs[0].cpu().numpy(), wants[0])
