"""GPU parity of the Q8_0, per-row int8 and Q4_0 quantisers (bit-exact codes and scales)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import load_golden
from qpu_xla_amd.kernels.quantize import quantize_q4_0, quantize_q8_0, quantize_rows_int8

pytestmark = pytest.mark.gpu


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def test_fixture_vectors() -> None:
    g = load_golden("oracle_quantizers_seed2024")
    x = dev(g["x"])
    np.testing.assert_array_equal(quantize_q8_0(x).cpu().numpy(), g["q8_0_blocks"])
    q, s = quantize_rows_int8(x)
    np.testing.assert_array_equal(q.cpu().numpy(), g["rows_q"])
    np.testing.assert_array_equal(s.cpu().numpy(), g["rows_scale"])
    np.testing.assert_array_equal(quantize_q4_0(dev(g["w"])).cpu().numpy(), g["q4_0_blocks"])


def test_q8_0_scale_without_division_equals_ieee_division_for_every_absmax() -> None:
    # The Q8_0 quantisers compute d = fl32(absmax / 127) and inv = fl32(1 / d)
    # without division sequences; the device compares both with IEEE division
    # for all 2^31 non-negative fp32 bit patterns (zero, subnormals, the fast
    # range's edges, inf and NaN included).
    from qpu_xla_amd import _lib

    counter = torch.zeros(1, dtype=torch.int64, device="cuda")
    _lib.call("qxt_q8_0_scale_check", ctypes.c_void_p(counter.data_ptr()), None)
    torch.cuda.synchronize()
    assert int(counter.item()) == 0


def test_q8_0_blocks_at_the_edges_of_the_fast_scale_range_bit_exact() -> None:
    # Blocks whose absmax sits at, just inside and just outside [2^-96, 2^120]
    # (outside, the quantisers divide) and at all-ones significands: the codes
    # and fp16 scales equal the oracle's, which divides.  (Smaller maxima give
    # subnormal scales whose reciprocal overflows; the scale check above covers
    # them.)
    edges = [2.0**-96, 2.0**120, np.nextafter(np.float32(2.0**-96), np.float32(0)),
             np.nextafter(np.float32(2.0**120), np.float32(np.inf)), np.float32(2.0**-96) * np.float32(1.9999999),
             np.float32(2.0**119) * np.float32(1.9999999), np.float32(1.9999999), np.float32(127.0),
             np.float32(2.0**-90) * np.float32(1.5), np.float32(65504.0) * np.float32(127.0)]
    rng = np.random.default_rng(77)
    x = np.empty((len(edges), 64), dtype=np.float32)
    for i, e in enumerate(edges):
        block = (rng.uniform(-1.0, 1.0, 64) * np.float32(e)).astype(np.float32)
        block[rng.integers(0, 32)] = np.float32(e) * (1 if i % 2 else -1)
        block[32 + rng.integers(0, 32)] = np.float32(e)
        x[i] = block
    np.testing.assert_array_equal(quantize_q8_0(dev(x)).cpu().numpy(), oracle.quantize_q8_0_blocks(x))


@pytest.mark.parametrize("rows,cols", [(1, 32), (3, 96), (7, 2048), (64, 5632), (2, 14336)])
def test_q8_0_random_bit_exact(rows: int, cols: int) -> None:
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(rng.uniform(0.01, 10))
    x[0, :32] = 0.0
    np.testing.assert_array_equal(quantize_q8_0(dev(x)).cpu().numpy(), oracle.quantize_q8_0_blocks(x))


def test_q8_0_half_even_ties_and_tiny_scales() -> None:
    x = np.zeros((2, 64), np.float32)
    x[0, :6] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5]
    x[1, :32] = np.float32(1e-6) * np.arange(32, dtype=np.float32)  # subnormal fp16 scale
    x[1, 32:] = np.float32(7e4) * np.sin(np.arange(32, dtype=np.float32))  # scale near fp16 max
    np.testing.assert_array_equal(quantize_q8_0(dev(x)).cpu().numpy(), oracle.quantize_q8_0_blocks(x))


@pytest.mark.parametrize("rows,cols,pad", [(1, 16, 16), (5, 300, 304), (8, 4096, 4096), (3, 14336, 14336), (2, 20000, 20000), (4, 5, 16)])
def test_rows_int8_random_bit_exact(rows: int, cols: int, pad: int) -> None:
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    x[-1] *= np.float32(1e-3)  # floor active on the last row
    q, s = quantize_rows_int8(dev(x), padded_columns=pad)
    qr, sr = oracle.quantize_rows_int8(x)
    np.testing.assert_array_equal(s.cpu().numpy(), sr)
    qn = q.cpu().numpy()
    np.testing.assert_array_equal(qn[:, :cols], qr)
    np.testing.assert_array_equal(qn[:, cols:], 0)


def test_rows_int8_outlier_channels_like_cfg4() -> None:
    rng = np.random.default_rng(4)
    k = 4096
    x = rng.standard_normal((64, k), dtype=np.float32)
    outliers = rng.choice(k, round(0.001 * k), replace=False)
    x[:, outliers] *= np.float32(20.0)
    q, s = quantize_rows_int8(dev(x))
    qr, sr = oracle.quantize_rows_int8(x)
    np.testing.assert_array_equal(q.cpu().numpy(), qr)
    np.testing.assert_array_equal(s.cpu().numpy(), sr)


def _near_half_integer_rows(rng, scales: np.ndarray, cols: int) -> np.ndarray:
    """Rows whose scale is fl32(fl32(127 t) / 127) for each target t, filled with
    fl32((k + 1/2) s) moved by -3..3 ulps: quotients at and beside rounding ties."""
    rows = len(scales)
    x = np.empty((rows, cols), np.float32)
    for i, t in enumerate(scales.astype(np.float32)):
        amax = np.float32(np.float32(127.0) * t)
        s = np.float32(amax / np.float32(127.0))
        k = rng.integers(-127, 127, cols - 1)
        v = ((k.astype(np.float64) + 0.5) * np.float64(s)).astype(np.float32)
        steps = rng.integers(-3, 4, cols - 1)
        v = np.nextafter(v, np.where(steps > 0, np.inf, -np.inf).astype(np.float32))
        for _ in range(2):
            more = np.abs(steps) > 1
            v[more] = np.nextafter(v[more], np.where(steps[more] > 0, np.inf, -np.inf).astype(np.float32))
            steps = np.where(more, steps - np.sign(steps), steps)
        v[steps == 0] = ((k[steps == 0].astype(np.float64) + 0.5) * np.float64(s)).astype(np.float32)
        x[i, 0] = amax
        x[i, 1:] = np.clip(v, -amax, amax)
    return x


def test_rows_int8_quotients_at_rounding_ties_bit_exact() -> None:
    # The quantiser divides by the row scale through its reciprocal with one
    # fused correction step; every quotient must still round as IEEE x / s.
    rng = np.random.default_rng(77)
    sig = rng.integers(1 << 23, 1 << 24, 64)
    sig[:8] = (1 << 24) - 1  # all-ones significands
    sig[8:12] = 1 << 23
    scales = (sig.astype(np.float64) * np.exp2(rng.integers(-6, 10, 64) - 23)).astype(np.float32)
    x = _near_half_integer_rows(rng, scales, 4096)
    q, s = quantize_rows_int8(dev(x))
    qr, sr = oracle.quantize_rows_int8(x)
    np.testing.assert_array_equal(s.cpu().numpy(), sr)
    np.testing.assert_array_equal(q.cpu().numpy(), qr)
    # Without the 1/127 floor: scales above and below the reciprocal form's lower limit.
    tiny = np.array([1e-18, 3e-20, 1e-21, 1e-25, 2.0**-69, 2.0**-71], np.float64).astype(np.float32)
    x = _near_half_integer_rows(rng, tiny, 1024)
    q, s = quantize_rows_int8(dev(x), floor=False)
    qr, sr = oracle.quantize_rows_int8(x, floor=False)
    np.testing.assert_array_equal(s.cpu().numpy(), sr)
    np.testing.assert_array_equal(q.cpu().numpy(), qr)


def test_rows_int8_without_floor_is_labelled_non_reference() -> None:
    x = np.zeros((2, 32), np.float32)
    x[1] = np.float32(1e-4) * np.arange(32, dtype=np.float32)
    q, s = quantize_rows_int8(dev(x), floor=False)
    qr, sr = oracle.quantize_rows_int8(x, floor=False)
    np.testing.assert_array_equal(s.cpu().numpy(), sr)
    np.testing.assert_array_equal(q.cpu().numpy(), qr)


@pytest.mark.parametrize("rows,cols", [(4, 32), (9, 256), (256, 2048), (16, 5632)])
def test_q4_0_weights_bit_exact(rows: int, cols: int) -> None:
    rng = np.random.default_rng(rows * cols)
    w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    w[0, :32] = 0.0
    w[1, :32] = np.float32(0.5)  # ties in |max|: first element wins
    w[1, 5] = np.float32(-0.5)
    np.testing.assert_array_equal(quantize_q4_0(dev(w)).cpu().numpy(), oracle.quantize_q4_0_blocks(w))


def test_q4_0_weights_known_answer_blocks() -> None:
    # The hand-worked blocks of ggml's rule (ties round up, first max wins,
    # -0.0 scale of a zero block, fp16-subnormal scale, x * fl32(1/d) rather
    # than x / d, codes from the fp32 d): codes and scale bits as literals.
    import q4_0_kats

    w, expected = q4_0_kats.kat_matrix()
    blocks = quantize_q4_0(dev(w)).cpu().numpy()
    np.testing.assert_array_equal(blocks, oracle.quantize_q4_0_blocks(w))
    _, values = oracle.unpack_q4_0_blocks(blocks)
    for b, (name, scale_bits, codes) in enumerate(expected):
        np.testing.assert_array_equal(values[0, b].astype(np.int64) + 8, codes, err_msg=name)
        if scale_bits is not None:
            assert int(blocks[0, b, 0]) | (int(blocks[0, b, 1]) << 8) == scale_bits, name


# ------------------------------------------------ known answers of tests/q8_0_kats.py


def _q8_0_kat_row() -> tuple[np.ndarray, list[tuple[str, int, list[int]]]]:
    """The Q8_0 known-answer blocks as one fp32 row [1, 32 B] and (name, fp16 scale bits, 32 codes) per block."""
    import q8_0_kats

    kats = q8_0_kats.q8_0_kat_blocks()
    row = np.concatenate([values for _, values, _, _ in kats])[None, :].astype(np.float32)
    return row, [(name, bits, q8_0_kats.expected_codes(codes, 32)) for name, _, bits, codes in kats]


def _check_q8_0_blocks(blocks: np.ndarray, expected, scale_shift: int = 0) -> None:
    """Blocks u8 [B, 34] hold the literal codes; their scales the literal fp16 bits (times 2^scale_shift)."""
    for b, (name, bits, codes) in enumerate(expected):
        got_bits = int(blocks[b, 0]) | (int(blocks[b, 1]) << 8)
        want = float(np.array([bits], np.uint16).view(np.float16)[0]) * 2.0**scale_shift
        assert got_bits == int(np.float16(want).view(np.uint16)), f"{name}: scale bits {got_bits:#06x}"
        np.testing.assert_array_equal(blocks[b, 2:].view(np.int8).astype(np.int64), codes, err_msg=name)


def test_q8_0_known_answer_blocks_bit_exact() -> None:
    # Codes that separate x * fl32(1/d) from x / d, half-even from half-away
    # rounding and the fp32 d from its fp16 rounding, as literals.
    row, expected = _q8_0_kat_row()
    _check_q8_0_blocks(quantize_q8_0(dev(row)).cpu().numpy()[0], expected)


def test_rows_int8_known_answer_rows_bit_exact() -> None:
    # True division at a non-unit scale (a reciprocal product changes four
    # codes), half-even ties, the 1/127 floor and the mode without it.
    import q8_0_kats

    for name, row, floor, scale_bits, codes in q8_0_kats.row_kats():
        q, s = quantize_rows_int8(dev(row[None, :]), floor=floor)
        np.testing.assert_array_equal(q.cpu().numpy()[0].astype(np.int64),
                                      q8_0_kats.expected_codes(codes, row.size), err_msg=name)
        assert int(s.cpu().numpy().view(np.uint32)[0]) == scale_bits, name


def _selector_q4_0_weights(blocks: int) -> np.ndarray:
    """Q4_0 weights [32 B, B, 18], d = 1: column n picks element n % 32 of block n // 32 (code 9 = +1, else 0)."""
    n = 32 * blocks
    codes = np.full((n, blocks, 32), 8, np.int64)
    codes[np.arange(n), np.arange(n) // 32, np.arange(n) % 32] = 9
    return oracle.pack_q4_0_blocks(np.ones((n, blocks), np.float16), codes)


def _selected(expected, rows: int) -> np.ndarray:
    """y[r, n] = code of element n % 32 of block n // 32 times that block's fp16 scale (exact in fp32)."""
    y = np.concatenate([np.asarray(codes, np.float32) * np.float32(np.array([bits], np.uint16).view(np.float16)[0])
                        for _, bits, codes in expected])
    return np.repeat(y[None, :], rows, axis=0)


@pytest.mark.parametrize("path", ["prefetch_m1", "fused_m4", "prepass"])
def test_batch_quantisers_known_answers_through_selector_weights(path: str) -> None:
    # The Q4_0 batch kernels quantise fp32 activations to Q8_0 themselves
    # (inside each workgroup, or in a pre-pass launch for large batches).
    # Selector weights make every output one code times its block's fp16
    # scale, so the literal codes and scales are read back exactly.
    from qpu_xla_amd import _lib
    from qpu_xla_amd.kernels import ggml_q4_0 as q4

    row, expected = _q8_0_kat_row()
    # The batch kernels take K % 256 == 0: the known-answer blocks twice over.
    row, expected = np.concatenate([row, row], axis=1), expected + expected
    rows = 4 if path == "fused_m4" else 1
    x = dev(np.repeat(row, rows, axis=0))
    blocks = row.shape[1] // 32
    w = dev(_selector_q4_0_weights(blocks))
    y = torch.full((rows, 32 * blocks), float("nan"), device="cuda")
    tasks = [{"x": x, "weight": w, "destination": y}]
    if path == "prepass":
        # A filler linear of many column tiles pushes the batch past the
        # in-workgroup limit, so the activations go through the pre-pass.
        # (Its bytes are random codes with fp16 scales of 1/64; its output is not checked.)
        rng = np.random.default_rng(5)
        filler = rng.integers(0, 256, (65536, 64, 18), dtype=np.uint8)
        filler[..., 0:2] = np.array([2.0**-6], np.float16).view(np.uint8)
        tasks.append({"x": dev(rng.standard_normal((1, 2048), dtype=np.float32)), "weight": dev(filler),
                      "destination": torch.empty((1, 65536), device="cuda")})
    with q4.Q4_0LinearBatch(tasks) as batch:
        assert (batch.work_items > 1024) == (path == "prepass")
        with _lib.launch_timing() as timing:
            batch.launch()
            torch.cuda.synchronize()
    names = [name for name, _ in timing.records]
    assert names == (["q8_0_prepass_kernel", "q4_0_batch_kernel"] if path == "prepass" else ["q4_0_batch_kernel"])
    np.testing.assert_array_equal(y.cpu().numpy(), _selected(expected, rows))


def test_geglu_producer_known_answers() -> None:
    # gate = 4.0, whose fp16 GELU entry is 4.0 exactly: v = fl32(4 up) = 4 up,
    # so the producer's Q8_0 codes are the known answers of `up` and every
    # scale is 4 times the known one.
    from qpu_xla_amd.kernels.ggml_geglu_q8 import ggml_geglu_q8_0, ggml_gelu_fp16_table

    table = ggml_gelu_fp16_table()
    assert int(table.view(torch.int16)[0x4400]) & 0xFFFF == 0x4400
    row, expected = _q8_0_kat_row()
    gate = dev(np.full_like(row, 4.0))
    blocks = ggml_geglu_q8_0(gate, dev(row)).cpu().numpy()[0]
    _check_q8_0_blocks(blocks, expected, scale_shift=2)


def test_hbm_read_probe_reads_every_word_once() -> None:
    # The xor of the per-workgroup partials is the xor of every 32-bit word:
    # each 16-byte chunk was read exactly once (an even count would cancel).
    from qpu_xla_amd import _lib

    rng = np.random.default_rng(77)
    for nbytes in (16, 4096 + 48, (3 << 20) + 16 * 2047):
        host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
        src = torch.from_numpy(host.view(np.int32)).to("cuda")
        partials = torch.zeros(2048, dtype=torch.int32, device="cuda")
        _lib.call("qxt_hbm_read_probe", ctypes.c_void_p(src.data_ptr()), nbytes, ctypes.c_void_p(partials.data_ptr()),
                  None)
        got = np.bitwise_xor.reduce(partials.cpu().numpy().view(np.uint32))
        assert got == np.bitwise_xor.reduce(host)
