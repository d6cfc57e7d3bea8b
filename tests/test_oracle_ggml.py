"""Pin the NumPy oracle of the GGML path against closed forms, KATs and brute force."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle
import q4_0_kats
import q8_0_kats
from conftest import load_golden


def test_codec_extremes_match_reference_cases() -> None:
    # tests/test_qpu_xla_ggml_q4_0.py:25-44 in the reference.
    g = load_golden("codec_extremes")
    blocks = oracle.pack_q4_0_blocks(g["q4_scales"], g["q4_codes"])
    scales, values = oracle.unpack_q4_0_blocks(blocks)
    np.testing.assert_array_equal(scales, g["q4_scales"].astype(np.float32))
    np.testing.assert_array_equal(values, g["q4_codes"].astype(np.int8) - 8)
    q8 = oracle.pack_q8_0_blocks(g["q8_scales"], g["q8_values"])
    s8, v8 = oracle.unpack_q8_0_blocks(q8)
    np.testing.assert_array_equal(s8, g["q8_scales"].astype(np.float32))
    np.testing.assert_array_equal(v8, g["q8_values"].astype(np.int8))


def test_q4_0_byte_layout_low_nibble_is_element_j_high_is_j_plus_16() -> None:
    codes = np.arange(32, dtype=np.uint8) % 16
    codes[16:] = 15 - codes[16:]
    block = oracle.pack_q4_0_blocks(np.array([1.0], np.float16), codes[None])[0]
    assert block[0] == 0x00 and block[1] == 0x3C  # little-endian fp16 1.0
    for j in range(16):
        assert block[2 + j] & 0x0F == codes[j]
        assert block[2 + j] >> 4 == codes[16 + j]


def test_codec_round_trip_random() -> None:
    rng = np.random.default_rng(7)
    scales = rng.uniform(-2, 2, size=(5, 7)).astype(np.float16)
    codes = rng.integers(0, 16, size=(5, 7, 32), dtype=np.uint8)
    s, v = oracle.unpack_q4_0_blocks(oracle.pack_q4_0_blocks(scales, codes))
    np.testing.assert_array_equal(s, scales.astype(np.float32))
    np.testing.assert_array_equal(v.astype(np.int16) + 8, codes)
    values = rng.integers(-128, 128, size=(3, 4, 32), dtype=np.int16)
    s8, v8 = oracle.unpack_q8_0_blocks(oracle.pack_q8_0_blocks(scales[:3, :4], values))
    np.testing.assert_array_equal(v8, values.astype(np.int8))


@pytest.mark.parametrize("name", ["kat_q4_0_m1", "kat_q4_0_m4", "kat_q4_0_mx"])
def test_q4_0_reference_matches_native_smoke_kats(name: str) -> None:
    g = load_golden(name)
    actual = oracle.q4_0_q8_0_reference(g["activation"], g["weight"])
    np.testing.assert_array_equal(actual, g["expected"])


def test_q4_0_block_dots_match_dequantised_brute_force() -> None:
    rng = np.random.default_rng(11)
    rows, blocks, outputs = 3, 4, 5
    act = oracle.pack_q8_0_blocks(
        rng.uniform(-0.1, 0.1, (rows, blocks)).astype(np.float16), rng.integers(-128, 128, (rows, blocks, 32))
    )
    wt = oracle.pack_q4_0_blocks(
        rng.uniform(-0.2, 0.2, (outputs, blocks)).astype(np.float16), rng.integers(0, 16, (outputs, blocks, 32))
    )
    dots = oracle.q4_0_q8_0_block_dots(act, wt)
    for m in range(rows):
        for n in range(outputs):
            for b in range(blocks):
                a = [int(np.int8(x)) for x in act[m, b, 2:].view(np.int8)]
                w = [(int(wt[n, b, 2 + j]) & 15) - 8 for j in range(16)] + [(int(wt[n, b, 2 + j]) >> 4) - 8 for j in range(16)]
                assert dots[m, n, b] == sum(x * y for x, y in zip(a, w))


def test_q4_0_reference_matches_float64_dequantised_sum() -> None:
    rng = np.random.default_rng(4850)
    rows, blocks, outputs = 4, 9, 7
    act = oracle.pack_q8_0_blocks(
        rng.uniform(-0.1, 0.1, (rows, blocks)).astype(np.float16), rng.integers(-128, 128, (rows, blocks, 32))
    )
    wt = oracle.pack_q4_0_blocks(
        rng.uniform(-0.2, 0.2, (outputs, blocks)).astype(np.float16), rng.integers(0, 16, (outputs, blocks, 32))
    )
    sa, va = oracle.unpack_q8_0_blocks(act)
    sw, vw = oracle.unpack_q4_0_blocks(wt)
    a = sa.astype(np.float64)[..., None] * va.astype(np.float64)
    w = sw.astype(np.float64)[..., None] * vw.astype(np.float64)
    expected = np.einsum("rbk,obk->ro", a, w)
    actual = oracle.q4_0_q8_0_reference(act, wt)
    np.testing.assert_allclose(actual, expected, rtol=2e-5, atol=2e-5 * np.abs(expected).max())


def test_q4_0_reference_power_of_two_scales_are_exact() -> None:
    rng = np.random.default_rng(3)
    rows, blocks, outputs = 2, 6, 9
    a_scales = (2.0 ** rng.integers(-6, 2, (rows, blocks))).astype(np.float16)
    w_scales = (2.0 ** rng.integers(-6, 2, (outputs, blocks)) * rng.choice([-1, 1], (outputs, blocks))).astype(np.float16)
    act = oracle.pack_q8_0_blocks(a_scales, rng.integers(-128, 128, (rows, blocks, 32)))
    wt = oracle.pack_q4_0_blocks(w_scales, rng.integers(0, 16, (outputs, blocks, 32)))
    dots = oracle.q4_0_q8_0_block_dots(act, wt).astype(np.float64)
    expected = np.einsum("mnb,nb,mb->mn", dots, w_scales.astype(np.float64), a_scales.astype(np.float64))
    np.testing.assert_array_equal(oracle.q4_0_q8_0_reference(act, wt), expected.astype(np.float32))


def test_q4_0_reference_sums_blocks_sequentially() -> None:
    # c_0 = 1, c_1 = 2**-24, c_2 = -1: ((0 + 1) + 2**-24) - 1 == 0 in fp32 (the
    # middle add ties to even), while any other association gives 2**-24.
    act = np.zeros((1, 3, 34), np.uint8)
    wt = np.zeros((1, 3, 18), np.uint8)
    codes = np.full((1, 3, 32), 8, np.uint8)
    codes[0, :, 0] = 9  # element 0 contributes +1 per unit activation
    a_vals = np.zeros((1, 3, 32), np.int16)
    a_vals[0, :, 0] = [1, 1, -1]
    act[:] = oracle.pack_q8_0_blocks(np.array([[1.0, 2.0**-12, 1.0]], np.float16), a_vals)
    wt[:] = oracle.pack_q4_0_blocks(np.array([[1.0, 2.0**-12, 1.0]], np.float16), codes)
    assert oracle.q4_0_q8_0_reference(act, wt)[0, 0] == np.float32(0.0)


def test_q8_0_quantiser_invariants() -> None:
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 512), dtype=np.float32) * np.float32(3.0)
    x[2, 64:96] = 0.0
    scale_bits, codes = oracle.quantize_q8_0_split(x)
    g = x.reshape(6, 16, 32)
    q = codes.reshape(6, 16, 32).astype(np.int32)
    d16 = scale_bits.view(np.float16)
    amax = np.abs(g).max(axis=2)
    d32 = amax / np.float32(127.0)
    np.testing.assert_array_equal(d16, d32.astype(np.float16))  # fp16 RNE storage
    assert np.all(np.abs(q) <= 127)
    nz = amax > 0
    hit = np.take_along_axis(q, np.abs(g).argmax(axis=2)[..., None], axis=2)[..., 0]
    assert np.all(np.abs(hit[nz]) == 127)
    np.testing.assert_array_equal(q[~nz], 0)
    err = np.abs(g - q * d32[..., None])
    assert np.all(err <= d32[..., None] * 0.5000001 + 1e-12)


def test_q8_0_quantiser_rounds_half_to_even() -> None:
    x = np.zeros((1, 32), np.float32)
    x[0, :6] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5]  # absmax 127 -> d = 1, inv = 1
    _, codes = oracle.quantize_q8_0_split(x)
    np.testing.assert_array_equal(codes[0, :6], [127, 2, 4, -2, -4, 0])


@pytest.mark.parametrize("kat", q8_0_kats.q8_0_kat_blocks(), ids=lambda k: k[0])
def test_q8_0_quantiser_known_answer_blocks(kat) -> None:
    # Literal codes and fp16 scale bits (tests/q8_0_kats.py gives the fp32
    # quotient each literal rounds).
    name, values, scale_bits, codes = kat
    bits, got = oracle.quantize_q8_0_split(values[None, :])
    assert int(bits[0, 0]) == scale_bits, f"{name}: fp16 scale bits {int(bits[0, 0]):#06x}"
    np.testing.assert_array_equal(got[0].astype(np.int64), q8_0_kats.expected_codes(codes, 32), err_msg=name)


@pytest.mark.parametrize("kat", q8_0_kats.q8_0_kat_blocks(), ids=lambda k: k[0])
def test_q8_0_known_answers_agree_with_exact_arithmetic(kat) -> None:
    name, values, scale_bits, codes = kat
    d, exact = q8_0_kats.exact_q8_0(values)
    assert exact == q8_0_kats.expected_codes(codes, 32), name
    assert int(np.float16(float(d)).view(np.uint16)) == scale_bits, name


def test_q8_0_known_answers_reject_the_plausible_mistakes() -> None:
    # Dividing by d instead of multiplying by fl32(1/d), quantising with the
    # fp16-rounded d, or rounding half away from zero each changes at least
    # one literal code (checked in exact arithmetic, so the oracle cannot pass
    # the known answers with any of these mistakes).
    name, values, _, codes = q8_0_kats.q8_0_kat_blocks()[0]
    want = q8_0_kats.expected_codes(codes, 32)
    for mistake in ("divide", "fp16_scale", "half_away"):
        _, wrong = q8_0_kats.exact_q8_0(values, **{mistake: True})
        assert wrong != want, mistake
    # ... and a signed maximum instead of |x| flips the scale's sign bit.
    assert q8_0_kats.q8_0_kat_blocks()[1][2] & 0x8000 == 0


def test_q8_0_quantiser_random_blocks_match_exact_arithmetic() -> None:
    rng = np.random.default_rng(31)
    x = rng.standard_normal((3, 256), dtype=np.float32) * np.float32(2.5)
    x[1] *= np.float32(1e-4)
    bits, codes = oracle.quantize_q8_0_split(x)
    for r in range(x.shape[0]):
        for b in range(x.shape[1] // 32):
            d, exact = q8_0_kats.exact_q8_0(x[r, 32 * b : 32 * b + 32])
            np.testing.assert_array_equal(codes[r, 32 * b : 32 * b + 32].astype(np.int64), exact)
            assert int(bits[r, b]) == int(np.float16(float(d)).view(np.uint16))


def test_q8_0_blocks_equal_split_form() -> None:
    g = load_golden("oracle_quantizers_seed2024")
    bits, codes = oracle.quantize_q8_0_split(g["x"])
    blocks = g["q8_0_blocks"]
    np.testing.assert_array_equal(blocks[..., 0:2].copy().view("<u2")[..., 0], bits)
    np.testing.assert_array_equal(blocks[..., 2:].reshape(codes.shape).view(np.int8), codes)


@pytest.mark.parametrize("kat", q4_0_kats.kat_blocks(), ids=lambda k: k[0])
def test_q4_0_quantiser_known_answer_blocks(kat) -> None:
    # Literal codes worked by hand from ggml's quantize_row_q4_0_ref rule.
    name, values, scale_bits, codes, fill = kat
    blocks = oracle.quantize_q4_0_blocks(values[None, :])
    d, v = oracle.unpack_q4_0_blocks(blocks)
    got = v[0, 0].astype(np.int64) + 8
    want = np.full(32, fill, dtype=np.int64)
    for index, code in codes.items():
        want[index] = code
    np.testing.assert_array_equal(got, want, err_msg=name)
    bits = int(blocks[0, 0, 0]) | (int(blocks[0, 0, 1]) << 8)
    if scale_bits is not None:
        assert bits == scale_bits, f"{name}: fp16 scale bits {bits:#06x}, want {scale_bits:#06x}"


@pytest.mark.parametrize("kat", q4_0_kats.kat_blocks(), ids=lambda k: k[0])
def test_q4_0_known_answer_blocks_agree_with_exact_arithmetic(kat) -> None:
    # The literal codes themselves, re-derived with exact rationals and explicit
    # round-to-fp32 steps (independent of NumPy's float32 arithmetic).
    name, values, _, codes, fill = kat
    d, exact = q4_0_kats.exact_codes(values)
    want = [codes.get(i, fill) for i in range(32)]
    assert exact == want, name
    blocks = oracle.quantize_q4_0_blocks(values[None, :])
    assert float(np.float16(float(d))) == float(oracle.unpack_q4_0_blocks(blocks)[0][0, 0])


def test_q4_0_separators_distinguish_the_plausible_mistakes() -> None:
    # The two separator blocks really separate: dividing by d, or using the
    # fp16-rounded d, changes their second code (checked in exact arithmetic).
    from fractions import Fraction

    rn = q4_0_kats._rn32
    for name, values, _, codes, _ in q4_0_kats.kat_blocks():
        if name not in ("reciprocal_not_division", "fp32_scale_not_fp16"):
            continue
        m, x = Fraction(float(values[0])), Fraction(float(values[1]))
        d = rn(m / -8)
        if name == "reciprocal_not_division":
            wrong = min(15, int(rn(rn(x / d) + Fraction(17, 2))))
        else:
            d16 = Fraction(float(np.float16(float(d))))
            wrong = min(15, int(rn(rn(x * rn(1 / d16)) + Fraction(17, 2))))
        assert wrong != codes[1], name


def test_q4_0_quantiser_random_blocks_match_exact_arithmetic() -> None:
    rng = np.random.default_rng(77)
    w = rng.standard_normal((6, 128), dtype=np.float32) * np.float32(0.02)
    w[2, 32:64] *= np.float32(1e-3)  # small scales
    blocks = oracle.quantize_q4_0_blocks(w)
    d, v = oracle.unpack_q4_0_blocks(blocks)
    for r in range(w.shape[0]):
        for b in range(w.shape[1] // 32):
            exact_d, exact = q4_0_kats.exact_codes(w[r, 32 * b : 32 * b + 32])
            np.testing.assert_array_equal(v[r, b].astype(np.int64) + 8, exact)
            assert float(np.float16(float(exact_d))) == float(d[r, b])


def test_q4_0_quantiser_half_step_reconstruction_bound() -> None:
    # Round-half-up of x/d: every element not clamped at code 15 lies within
    # half a step of its code (in units of the fp32 d the codes were made with);
    # trunc(x/d + 8) would miss this by up to a whole step.
    rng = np.random.default_rng(9)
    w = rng.standard_normal((16, 512), dtype=np.float32) * np.float32(0.02)
    blocks = oracle.quantize_q4_0_blocks(w)
    _, v = oracle.unpack_q4_0_blocks(blocks)
    g = w.reshape(16, 16, 32).astype(np.float64)
    first = np.abs(g).argmax(axis=2)
    d32 = np.take_along_axis(g, first[..., None], axis=2) / -8.0  # exact: division by 8
    ratio = g / d32
    codes = v.astype(np.int64) + 8
    inner = codes < 15
    err = np.abs(ratio - (codes - 8))
    assert np.all(err[inner] <= 0.5 + 1e-5)
    assert np.all(ratio[~inner] >= 6.5 - 1e-5)  # clamped elements sit in the top half step or above
    np.testing.assert_array_equal(np.take_along_axis(codes, first[..., None], axis=2), 0)


def test_q4_0_quantiser_invariants() -> None:
    rng = np.random.default_rng(9)
    w = rng.standard_normal((8, 256), dtype=np.float32) * np.float32(0.02)
    w[3, :32] = 0.0
    blocks = oracle.quantize_q4_0_blocks(w)
    d, v = oracle.unpack_q4_0_blocks(blocks)
    g = w.reshape(8, 8, 32)
    first = np.abs(g).argmax(axis=2)
    signed_max = np.take_along_axis(g, first[..., None], axis=2)[..., 0]
    np.testing.assert_array_equal(d, (signed_max / np.float32(-8)).astype(np.float16).astype(np.float32))
    codes = v.astype(np.int32) + 8
    assert codes.min() >= 0 and codes.max() <= 15
    nz = np.abs(signed_max) > 0
    np.testing.assert_array_equal(np.take_along_axis(codes, first[..., None], axis=2)[..., 0][nz], 0)
    dq = v.astype(np.float32) * d[..., None]
    step = np.abs(d)[..., None]
    assert np.all(np.abs(dq - g) <= step * 1.01 + 1e-9)
    # All-zero block: d = -0.0 (fp16 0x8000) and every code 8, as ggml's rule gives.
    assert blocks[3, 0, 0] == 0x00 and blocks[3, 0, 1] == 0x80
    np.testing.assert_array_equal(codes[3, 0], 8)


def test_tiled_weight_words_hold_element_quads_of_each_block() -> None:
    # Layout of pack_ggml_q4_0_tiled_weights (reference ggml_q4_0.py:844-855),
    # checked element by element against the native block bytes.
    rng = np.random.default_rng(11)
    outputs, blocks = 5, 3
    scales = rng.uniform(-1, 1, size=(outputs, blocks)).astype(np.float16)
    codes = rng.integers(0, 16, size=(outputs, blocks, 32), dtype=np.uint8)
    native = oracle.pack_q4_0_blocks(scales, codes)
    scale_bits, words = oracle.pack_q4_0_tiled_weights(native)
    assert scale_bits.dtype == np.uint16 and scale_bits.shape == (blocks, outputs)
    assert words.dtype == np.uint32 and words.shape == (blocks * 8, outputs)
    for n in range(outputs):
        for b in range(blocks):
            assert int(scale_bits[b, n]) == int(native[n, b, 0]) | (int(native[n, b, 1]) << 8)
            for g in range(8):
                word = int(words[b * 8 + g, n])
                for i in range(4):
                    byte = (word >> (8 * i)) & 0xFF
                    signed = byte - 256 if byte > 127 else byte
                    assert signed == int(codes[n, b, 4 * g + i]) - 8


def test_split_q8_0_blocks_inverts_packing() -> None:
    rng = np.random.default_rng(12)
    scales = rng.uniform(0.001, 0.2, size=(4, 6)).astype(np.float16)
    values = rng.integers(-128, 128, size=(4, 6, 32))
    native = oracle.pack_q8_0_blocks(scales, values)
    scale_bits, q = oracle.split_q8_0_blocks(native)
    assert q.shape == (4, 192)
    np.testing.assert_array_equal(scale_bits.view(np.float16), scales)
    np.testing.assert_array_equal(q.view(np.int8).reshape(4, 6, 32), values.astype(np.int8))


# --------------------------------------------------------- CPU_REPACK layouts


def test_repack_q4_0x4_inverts_exactly_both_ways() -> None:
    rng = np.random.default_rng(44)
    native = rng.integers(0, 256, size=(12, 3, oracle.Q4_0_BLOCK_BYTES), dtype=np.uint8)
    groups = oracle.pack_q4_0x4(native)
    assert groups.shape == (3, 3, 72)
    np.testing.assert_array_equal(oracle.unpack_q4_0x4(groups), native)
    raw = rng.integers(0, 256, size=(2, 5, 72), dtype=np.uint8)
    np.testing.assert_array_equal(oracle.pack_q4_0x4(oracle.unpack_q4_0x4(raw)), raw)


def test_repack_q4_0x4_nibbles_are_signed_values() -> None:
    # ggml's repacked Q4_0 stores each element as a two's-complement nibble of
    # (code - 8): that is what the 0x88 mask means.  Check every nibble of a
    # packed group against the element it must carry.
    rng = np.random.default_rng(45)
    codes = rng.integers(0, 16, size=(4, 2, oracle.QK))
    scales = rng.standard_normal((4, 2)).astype(np.float16)
    groups = oracle.pack_q4_0x4(oracle.pack_q4_0_blocks(scales, codes))

    def signed(nibble: np.ndarray) -> np.ndarray:
        return np.where(nibble >= 8, nibble.astype(int) - 16, nibble.astype(int))

    for column in range(4):
        np.testing.assert_array_equal(groups[0, :, 2 * column:2 * column + 2].copy().view("<f2")[:, 0], scales[column])
        for chunk in range(4):
            word = groups[0, :, 8 + (chunk * 4 + column) * 4:8 + (chunk * 4 + column) * 4 + 4]
            for byte in range(4):
                element = 4 * chunk + byte
                np.testing.assert_array_equal(signed(word[:, byte] & 0xF), codes[column, :, element] - 8)
                np.testing.assert_array_equal(signed(word[:, byte] >> 4), codes[column, :, element + 16] - 8)


@pytest.mark.parametrize("interleave", [4, 8])
@pytest.mark.parametrize("rows", [1, 3, 4, 5, 8, 9])
def test_q8_0x4_interleave_round_trip(rows: int, interleave: int) -> None:
    rng = np.random.default_rng(rows * 10 + interleave)
    native = rng.integers(0, 256, size=(rows, 2, oracle.Q8_0_BLOCK_BYTES), dtype=np.uint8)
    packed = oracle.interleave_q8_0x4(native, interleave)
    assert packed.size == native.size
    np.testing.assert_array_equal(oracle.deinterleave_q8_0x4(packed, rows, 2, interleave), native)
    tail = rows - rows % 4
    row_bytes = 2 * oracle.Q8_0_BLOCK_BYTES
    np.testing.assert_array_equal(packed[tail * row_bytes:], native[tail:].reshape(-1))
    if rows >= 4:
        # Each group is a permutation of its four native rows' bytes.
        group = packed[:4 * row_bytes]
        assert sorted(group.tolist()) == sorted(native[:4].reshape(-1).tolist())
        assert not np.array_equal(group, native[:4].reshape(-1))


@pytest.mark.parametrize("interleave", [4, 8])
def test_q8_0x4_positions_cover_each_value_once(interleave: int) -> None:
    from oracle.ggml import _interleaved_index

    positions = sorted(_interleaved_index(i, lane, interleave) for lane in range(4) for i in range(oracle.QK))
    assert positions == list(range(4 * oracle.QK))
    # Runs of ``interleave`` consecutive values of one row stay contiguous.
    assert all(_interleaved_index(i + 1, 2, interleave) == _interleaved_index(i, 2, interleave) + 1
               for i in range(oracle.QK - 1) if (i + 1) % interleave)


@pytest.mark.parametrize("n,blocks", [(1, 8), (5, 16), (64, 8), (37, 176), (130, 24)])
def test_lane_layout_places_every_chunk_and_inverts(n: int, blocks: int) -> None:
    rng = np.random.default_rng(n * blocks)
    native = rng.integers(0, 256, size=(n, blocks, oracle.Q4_0_BLOCK_BYTES), dtype=np.uint8)
    packed = oracle.pack_q4_0_lanes(native)
    units = native.reshape(-1, 144)
    groups = -(-units.shape[0] // 64)
    assert packed.size == groups * 64 * 144
    for unit in range(units.shape[0]):
        q, lane = divmod(unit, 64)
        for v in range(9):
            at = q * 9216 + (v * 64 + lane) * 16
            np.testing.assert_array_equal(packed[at:at + 16], units[unit, 16 * v:16 * v + 16])
    tail = units.shape[0] % 64
    if tail:  # padding units of the last group are zero
        last = packed[(groups - 1) * 9216:].reshape(9, 64, 16)
        assert not last[:, tail:].any()
    np.testing.assert_array_equal(oracle.unpack_q4_0_lanes(packed, n, blocks), native)


# ------------------------------------------------------------ Q8_0 x Q8_0


def _q8_operands(seed: int, rows: int, outputs: int, blocks: int, a_range=(-0.1, 0.1), w_range=(-0.2, 0.2)):
    rng = np.random.default_rng(seed)
    a_scales = rng.uniform(*a_range, size=(rows, blocks)).astype(np.float16)
    a_values = rng.integers(-128, 128, size=(rows, blocks, 32), dtype=np.int16)
    w_scales = rng.uniform(*w_range, size=(outputs, blocks)).astype(np.float16)
    w_values = rng.integers(-128, 128, size=(outputs, blocks, 32), dtype=np.int16)
    return (oracle.pack_q8_0_blocks(a_scales, a_values), oracle.pack_q8_0_blocks(w_scales, w_values),
            a_scales, a_values, w_scales, w_values)


def test_q8_0_reference_matches_the_explicit_dequantized_dot() -> None:
    # tests/test_qpu_xla_ggml_q8_0.py:16-31 of the reference (seed 4850, same tolerance).
    act, wt, a_s, a_v, w_s, w_v = _q8_operands(4850, 4, 3, 3)
    actual = oracle.q8_0_q8_0_reference(act, wt)
    activation = a_s.astype(np.float32)[..., None] * a_v.astype(np.float32)
    weights = w_s.astype(np.float32)[..., None] * w_v.astype(np.float32)
    expected = np.einsum("rbk,obk->ro", activation, weights, dtype=np.float32)
    np.testing.assert_allclose(actual, expected, rtol=2e-5, atol=2e-3)


def test_q8_0_reference_exact_with_power_of_two_scales() -> None:
    rng = np.random.default_rng(4851)
    rows, outputs, blocks = 3, 5, 4
    a_s = (2.0 ** rng.integers(-6, 2, size=(rows, blocks))).astype(np.float16)
    w_s = (2.0 ** rng.integers(-6, 2, size=(outputs, blocks))).astype(np.float16)
    a_v = rng.integers(-128, 128, size=(rows, blocks, 32))
    w_v = rng.integers(-128, 128, size=(outputs, blocks, 32))
    got = oracle.q8_0_q8_0_reference(oracle.pack_q8_0_blocks(a_s, a_v), oracle.pack_q8_0_blocks(w_s, w_v))
    for r in range(rows):
        for o in range(outputs):
            exact = sum(int(np.dot(a_v[r, b], w_v[o, b])) * float(a_s[r, b]) * float(w_s[o, b]) for b in range(blocks))
            assert got[r, o] == np.float32(exact)  # every partial sum is exact in fp32 here


def test_q8_0_reference_scales_by_the_activation_first() -> None:
    # Find operands where fl(fl(dot*da)*dw) != fl(fl(dot*dw)*da): the oracle must give the first.
    for seed in range(200):
        act, wt, *_ = _q8_operands(seed, 1, 1, 1, a_range=(-1.0, 1.0), w_range=(-1.0, 1.0))
        da, qa = oracle.unpack_q8_0_blocks(act)
        dw, qw = oracle.unpack_q8_0_blocks(wt)
        dot = float(np.dot(qa[0, 0].astype(np.int64), qw[0, 0].astype(np.int64)))
        a_first = np.float32(np.float32(dot * float(da[0, 0])) * float(dw[0, 0]))
        w_first = np.float32(np.float32(dot * float(dw[0, 0])) * float(da[0, 0]))
        if a_first != w_first:
            assert oracle.q8_0_q8_0_reference(act, wt)[0, 0] == a_first
            return
    pytest.fail("no order-sensitive case found")


def test_real_activation_fixture_quantises_within_the_q8_0_invariants() -> None:
    # tests/golden/mtp_activation.f32: the reference's captured K=256 activation
    # (artifact/evidence/mtp/activation.f32), 256 little-endian fp32 values.
    x = np.fromfile(Path(__file__).resolve().parent / "golden" / "mtp_activation.f32", dtype="<f4")
    assert x.shape == (256,) and np.all(np.isfinite(x))
    scale_bits, codes = oracle.quantize_q8_0_split(x.reshape(1, 256))
    d = scale_bits.view(np.float16).astype(np.float32).reshape(8)
    blocks = x.reshape(8, 32)
    q = codes.reshape(8, 32).astype(np.int32)
    assert np.all(np.abs(q) <= 127)
    # the absmax element of every block maps to +-127 and the reconstruction is within half a step
    assert np.all(np.abs(q[np.arange(8), np.argmax(np.abs(blocks), axis=1)]) == 127)
    step = np.abs(blocks).max(axis=1) / 127
    assert np.all(np.abs(blocks - q * step[:, None]) <= 0.5 * step[:, None] * (1 + 1e-6))
    np.testing.assert_allclose(d, (np.abs(blocks).max(axis=1) / np.float32(127)).astype(np.float16), rtol=0)
