"""The reference's real activation vector through the GPU path, bit-exact against the oracle.

``tests/golden/mtp_activation.f32`` is a copy of the reference's
``artifact/evidence/mtp/activation.f32``: 256 little-endian fp32 values
captured from the M=1, K=256 MTP node of its llama.cpp runs (its weight file
is not kept, so the weights here are seeded).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from qpu_xla_amd.kernels import ggml_geglu_q8 as geglu
from qpu_xla_amd.kernels import ggml_q4_0 as q4
from qpu_xla_amd.kernels.quantize import quantize_q8_0, quantize_rows_int8

pytestmark = pytest.mark.gpu

ACTIVATION = np.fromfile(Path(__file__).resolve().parent / "golden" / "mtp_activation.f32", dtype="<f4").reshape(1, 256)


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def test_real_activation_quantisers() -> None:
    q8 = quantize_q8_0(dev(ACTIVATION))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q8.cpu().numpy(), oracle.quantize_q8_0_blocks(ACTIVATION))
    q, s = quantize_rows_int8(dev(ACTIVATION))
    torch.cuda.synchronize()
    expected_q, expected_s = oracle.quantize_rows_int8(ACTIVATION)
    np.testing.assert_array_equal(q.cpu().numpy(), expected_q)
    np.testing.assert_array_equal(s.cpu().numpy(), expected_s)


@pytest.mark.parametrize("outputs", [32, 2048])
def test_real_activation_q4_0_linear(outputs: int) -> None:
    rng = np.random.default_rng(256 + outputs)
    weight = oracle.quantize_q4_0_blocks(
        (rng.standard_normal((outputs, 256), dtype=np.float32) * np.float32(0.02)).astype(np.float32))
    xq = oracle.quantize_q8_0_blocks(ACTIVATION)
    expected = oracle.q4_0_q8_0_reference(xq, weight)
    out = q4.ggml_q4_0_q8_0_linear(dev(xq), dev(weight))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), expected)
    lanes = q4.pack_ggml_q4_0_lane_weights(dev(weight))
    out = q4.ggml_q4_0_q8_0_lane_linear(dev(xq), lanes)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), expected)


def test_real_activation_as_geglu_gate() -> None:
    up = np.random.default_rng(257).standard_normal(ACTIVATION.shape, dtype=np.float32)
    out = geglu.ggml_geglu_q8_0(dev(ACTIVATION), dev(up))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.geglu_q8_0_reference(ACTIVATION, up))
