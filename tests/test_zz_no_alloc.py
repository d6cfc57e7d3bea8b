"""The allocation-free W8A8 linear equals the workspace entry point bit for bit (through the C ABI)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from qpu_xla_amd import _lib
from qpu_xla_amd.quantization import quantize_per_output_channel_int8

pytestmark = pytest.mark.gpu


def _p(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(None if t is None else t.data_ptr())


def _operands(seed: int, m: int, k: int, n: int, bias: bool):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((m, k), generator=g, device="cuda")
    x[:, :: max(1, k // 7)] *= 20.0  # outlier channels
    weight = quantize_per_output_channel_int8(torch.randn((n, k), generator=g, device="cuda") * 0.02)
    b = torch.randn((n,), generator=g, device="cuda") * 0.1 if bias else None
    return x, weight, b


def _with_workspace(x, weight, bias, m, k, n, flags):
    qa = torch.empty((m, k), dtype=torch.int8, device="cuda")
    sa = torch.empty((m,), dtype=torch.float32, device="cuda")
    y = torch.full((m, n), float("nan"), device="cuda")
    _lib.call("qxt_w8a8_linear", _p(x), x.stride(0) * 4, _p(qa), k, _p(sa), _p(weight.values), k,
              _p(weight.scales), _p(bias), _p(y), n * 4, m, n, k, 0, flags, None)
    return y


def _without_allocation(x, weight, bias, m, k, n, flags, stream):
    y = torch.full((m, n), float("nan"), device="cuda")
    torch.cuda.synchronize()
    _lib.call("qxt_w8a8_linear_noalloc", _p(x), x.stride(0) * 4, _p(weight.values), k, _p(weight.scales), _p(bias),
              _p(y), n * 4, m, n, k, 0, flags, ctypes.c_void_p(stream.cuda_stream))
    stream.synchronize()
    return y


@pytest.mark.parametrize("first,second", [
    ((512, 4096, 4096, True, 0), (64, 1024, 2048, False, 0)),       # GEMM path, then a smaller GEMM
    ((4096, 4096, 14336, True, 0), (3, 2048, 512, True, 1)),        # cfg4 gate_up (stream kernel), then M = 3 GEMV
    ((4096, 14336, 4096, True, 0), (1, 4096, 4096, True, 0)),       # cfg4 down, then one decode row
])
def test_noalloc_linear_equals_the_workspace_entry_point_twice(first, second) -> None:
    stream = torch.cuda.Stream()
    for seed, (m, k, n, bias, flags) in enumerate((first, second)):
        x, weight, b = _operands(100 + seed, m, k, n, bias)
        want = _with_workspace(x, weight, b, m, k, n, flags)
        got = _without_allocation(x, weight, b, m, k, n, flags, stream)
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (m, k, n)
        assert not torch.isnan(got).any()


def test_noalloc_linear_allocates_no_device_memory() -> None:
    # After a first call on the device (which loads the library's code object,
    # workspace included), further calls leave the device's free memory and
    # the caching allocator's statistics unchanged, and give the same bits.
    m, k, n = 256, 2048, 1024
    x, weight, b = _operands(7, m, k, n, True)
    y = torch.empty((m, n), device="cuda")

    def call():
        _lib.call("qxt_w8a8_linear_noalloc", _p(x), k * 4, _p(weight.values), k, _p(weight.scales), _p(b), _p(y),
                  n * 4, m, n, k, 0, 0, None)

    call()
    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    allocated_before = torch.cuda.memory_stats()["allocation.all.allocated"]
    library_before = _lib.allocation_count()
    for _ in range(3):
        call()
    torch.cuda.synchronize()
    # Pass criteria: no allocation by the library's own code and none through
    # torch's caching allocator.  The device-wide free memory is reported, not
    # asserted: another process on the same GPU can move it.
    assert _lib.allocation_count() == library_before
    assert torch.cuda.memory_stats()["allocation.all.allocated"] == allocated_before
    print(f"device free memory before / after: {free_before} / {torch.cuda.mem_get_info()[0]} bytes")
    want = _with_workspace(x, weight, b, m, k, n, 0)
    assert torch.equal(y.view(torch.int32), want.view(torch.int32))
