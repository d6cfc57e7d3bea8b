"""NumPy oracle for the GGML Q4_0 / Q8_0 block formats and their block-dot linear.

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py`` for who may import it.

Block formats (reference ``src/qpu_xla/kernels/ggml_q4_0.py:21-25``):

* Q4_0, 18 bytes: little-endian fp16 scale ``d``, then 16 bytes whose byte
  ``j`` holds element ``j`` in the low nibble and element ``j + 16`` in the
  high nibble; value = code - 8.
* Q8_0, 34 bytes: little-endian fp16 scale ``d``, then 32 signed bytes.
"""

from __future__ import annotations

import math
from functools import lru_cache

import numpy as np

QK = 32
Q4_0_BLOCK_BYTES = 18
Q8_0_BLOCK_BYTES = 34


def pack_q4_0_blocks(scales: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """Pack explicit 0..15 codes plus fp16 scales into 18-byte Q4_0 blocks.

    Follows ``src/qpu_xla/kernels/ggml_q4_0.py:28-40``.
    """
    scales = np.asarray(scales, dtype=np.float16)
    codes = np.asarray(codes)
    if codes.shape != (*scales.shape, QK):
        raise ValueError("Q4_0 codes must have shape scales.shape + (32,)")
    if np.any((codes < 0) | (codes > 15)):
        raise ValueError("Q4_0 codes must lie in 0..15")
    out = np.empty((*scales.shape, Q4_0_BLOCK_BYTES), dtype=np.uint8)
    out[..., 0:2] = scales.astype("<f2").view(np.uint8).reshape(*scales.shape, 2)
    low = codes[..., :16].astype(np.uint8)
    high = codes[..., 16:].astype(np.uint8)
    out[..., 2:] = low | (high << 4)
    return out


def pack_q8_0_blocks(scales: np.ndarray, values: np.ndarray) -> np.ndarray:
    """Pack signed bytes plus fp16 scales into 34-byte Q8_0 blocks.

    Follows ``src/qpu_xla/kernels/ggml_q4_0.py:43-55``.
    """
    scales = np.asarray(scales, dtype=np.float16)
    values = np.asarray(values)
    if values.shape != (*scales.shape, QK):
        raise ValueError("Q8_0 values must have shape scales.shape + (32,)")
    if np.any((values < -128) | (values > 127)):
        raise ValueError("Q8_0 values must lie in -128..127")
    out = np.empty((*scales.shape, Q8_0_BLOCK_BYTES), dtype=np.uint8)
    out[..., 0:2] = scales.astype("<f2").view(np.uint8).reshape(*scales.shape, 2)
    out[..., 2:] = values.astype(np.int8).view(np.uint8)
    return out


def _fp16_field(blocks: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(blocks[..., 0:2])
    return raw.view("<f2").reshape(blocks.shape[:-1])


def unpack_q4_0_blocks(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Decode Q4_0 blocks to (fp32 scales, int8 values in -8..7).

    Follows ``src/qpu_xla/kernels/ggml_q4_0.py:58-68``.
    """
    blocks = np.asarray(blocks)
    if blocks.dtype != np.uint8 or blocks.ndim < 1 or blocks.shape[-1] != Q4_0_BLOCK_BYTES:
        raise ValueError("Q4_0 blocks must be uint8 with a trailing extent of 18")
    scales = _fp16_field(blocks).astype(np.float32)
    qs = blocks[..., 2:]
    values = np.empty((*blocks.shape[:-1], QK), dtype=np.int8)
    values[..., :16] = (qs & 0x0F).astype(np.int8) - 8
    values[..., 16:] = (qs >> 4).astype(np.int8) - 8
    return scales, values


def unpack_q8_0_blocks(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Decode Q8_0 blocks to (fp32 scales, int8 values).

    Follows ``src/qpu_xla/kernels/ggml_q4_0.py:71-78``.
    """
    blocks = np.asarray(blocks)
    if blocks.dtype != np.uint8 or blocks.ndim < 1 or blocks.shape[-1] != Q8_0_BLOCK_BYTES:
        raise ValueError("Q8_0 blocks must be uint8 with a trailing extent of 34")
    scales = _fp16_field(blocks).astype(np.float32)
    values = np.ascontiguousarray(blocks[..., 2:]).view(np.int8)
    return scales, values


def _check_linear_operands(activation_blocks: np.ndarray, weight_blocks: np.ndarray) -> None:
    if activation_blocks.ndim != 3 or weight_blocks.ndim != 3:
        raise ValueError("activation and weight blocks must both be rank three")
    if activation_blocks.shape[2] != Q8_0_BLOCK_BYTES or weight_blocks.shape[2] != Q4_0_BLOCK_BYTES:
        raise ValueError("activation blocks must be Q8_0 (34 B) and weight blocks Q4_0 (18 B)")
    if activation_blocks.shape[1] != weight_blocks.shape[1]:
        raise ValueError("activation and weight reduction block counts differ")


def q4_0_q8_0_block_dots(activation_blocks: np.ndarray, weight_blocks: np.ndarray) -> np.ndarray:
    """Exact int32 per-block dots ``dot[m, n, b] = sum_k a[m,b,k] * (code[n,b,k] - 8)``.

    These are the integer terms of ``src/qpu_xla/kernels/ggml_q4_0.py:96``.
    Shapes: activation u8 [M, B, 34], weight u8 [N, B, 18] -> int32 [M, N, B].
    """
    _check_linear_operands(activation_blocks, weight_blocks)
    _, a = unpack_q8_0_blocks(activation_blocks)
    _, w = unpack_q4_0_blocks(weight_blocks)
    return np.einsum("mbk,nbk->mnb", a.astype(np.int32), w.astype(np.int32)).astype(np.int32)


def q4_0_q8_0_reference(activation_blocks: np.ndarray, weight_blocks: np.ndarray) -> np.ndarray:
    """Q4_0 x Q8_0 linear: ``y[m, n] = sum_b fl32(fl32(dot * dw[n,b]) * da[m,b])``.

    Follows ``src/qpu_xla/kernels/ggml_q4_0.py:81-100`` op for op: per block
    an exact int32 dot, converted to fp32, multiplied by the weight scale,
    then by the activation scale, and added to an fp32 accumulator in block
    order ``((0 + c_0) + c_1) + ...``.  NumPy float32 arithmetic performs
    each multiply and add with its own rounding (no fused multiply-add).
    """
    _check_linear_operands(activation_blocks, weight_blocks)
    a_scale, a = unpack_q8_0_blocks(activation_blocks)
    w_scale, w = unpack_q4_0_blocks(weight_blocks)
    rows, blocks = a_scale.shape
    outputs = w_scale.shape[0]
    result = np.zeros((rows, outputs), dtype=np.float32)
    for b in range(blocks):
        dots = a[:, b].astype(np.int32) @ w[:, b].astype(np.int32).T
        term = dots.astype(np.float32) * w_scale[None, :, b]
        term *= a_scale[:, b, None]
        result += term
    return result


def quantize_q8_0_split(values: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Quantise fp32 rows to Q8_0: (fp16 scale bits u16 [M, K/32], int8 codes [M, K]).

    Follows the repository's own quantiser,
    ``examples/benchmark_llama_cpp_qpu_persistent_q4.py:42-53``:
    ``d = fl32(absmax / 127)``; ``inv = fl32(1 / d)`` (0 when d == 0);
    ``q = clip(rint(fl32(x * inv)), -127, 127)`` with round-half-even;
    ``d`` stored as fp16 with round-to-nearest-even.
    """
    values = np.asarray(values, dtype=np.float32)
    if values.ndim != 2 or values.shape[1] % QK:
        raise ValueError("Q8_0 quantisation needs rank-2 rows whose length is a multiple of 32")
    rows, columns = values.shape
    grouped = values.reshape(rows, columns // QK, QK)
    scales = np.max(np.abs(grouped), axis=2).astype(np.float32) / np.float32(127.0)
    inverse = np.zeros_like(scales)
    np.divide(np.float32(1.0), scales, out=inverse, where=scales != 0.0)
    codes = np.clip(np.rint(grouped * inverse[..., None]), -127, 127).astype(np.int8)
    return (
        np.ascontiguousarray(scales.astype(np.float16).view(np.uint16)),
        np.ascontiguousarray(codes.reshape(rows, columns)),
    )


def quantize_q8_0_blocks(values: np.ndarray) -> np.ndarray:
    """Quantise fp32 rows [M, K] into native Q8_0 blocks u8 [M, K/32, 34] (same math as above)."""
    scale_bits, codes = quantize_q8_0_split(values)
    rows, columns = codes.shape
    out = np.empty((rows, columns // QK, Q8_0_BLOCK_BYTES), dtype=np.uint8)
    out[..., 0:2] = scale_bits.astype("<u2").view(np.uint8).reshape(rows, columns // QK, 2)
    out[..., 2:] = codes.reshape(rows, columns // QK, QK).view(np.uint8)
    return out


def quantize_q4_0_blocks(weights: np.ndarray) -> np.ndarray:
    """Quantise fp32 rows [N, K] into native Q4_0 blocks u8 [N, K/32, 18].

    Restates ggml's published reference quantiser ``quantize_row_q4_0_ref``
    (the reference has no Python Q4_0 quantiser and calls ggml's
    ``quantize_row_q4_0`` only from native tests,
    ``integrations/llama_cpp/tests/qpu_ggml_backend_smoke.cpp:119``; llama.cpp
    pinned at 91d2fc387529940230555abd297a8b5e99737d3f, not vendored), the
    BASELINE formula ``d = signed_absmax / -8``, ``q = clamp(round(x/d) + 8, 0, 15)``
    with ggml's rounding.  Pinned by the known-answer blocks of
    ``tests/q4_0_kats.py`` (literal codes) and by exact rational arithmetic:

    * ``max`` = the first element of largest magnitude (+0.0 for an all-zero block),
    * ``d = fl32(max / -8)``, ``id = fl32(1 / d)`` or 0 when d == 0,
    * ``q = min(15, trunc(fl32(fl32(x * id) + 8.5)))``, ``d`` stored as fp16 (RNE).
    """
    weights = np.asarray(weights, dtype=np.float32)
    if weights.ndim != 2 or weights.shape[1] % QK:
        raise ValueError("Q4_0 quantisation needs rank-2 rows whose length is a multiple of 32")
    rows, columns = weights.shape
    grouped = weights.reshape(rows, columns // QK, QK)
    first = np.argmax(np.abs(grouped), axis=2)
    signed_max = np.take_along_axis(grouped, first[..., None], axis=2)[..., 0]
    signed_max = np.where(np.abs(signed_max) > 0, signed_max, np.float32(0.0)).astype(np.float32)
    d = signed_max / np.float32(-8.0)
    inverse = np.zeros_like(d)
    np.divide(np.float32(1.0), d, out=inverse, where=d != 0.0)
    shifted = (grouped * inverse[..., None]) + np.float32(8.5)
    codes = np.minimum(np.trunc(shifted), 15).astype(np.uint8)
    return pack_q4_0_blocks(d.astype(np.float16), codes)


def pack_q4_0_tiled_weights(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Native Q4_0 weights [N, B, 18] -> (fp16 scale bits uint16 [B, N], uint32 words [B * 8, N]).

    Follows ``src/qpu_xla/kernels/ggml_q4_0.py:844-855``: word ``(8 b + g, n)``
    holds the signed values ``code - 8`` of elements ``4 g .. 4 g + 3`` of
    block ``b`` of output ``n`` as little-endian int8 bytes.
    """
    scales, values = unpack_q4_0_blocks(blocks)
    if blocks.ndim != 3:
        raise ValueError("native Q4_0 weights must have shape (outputs, blocks, 18)")
    scale_words = np.ascontiguousarray(scales.astype(np.float16).T.view(np.uint16))
    outputs, reduction_blocks, _ = values.shape
    groups = np.ascontiguousarray(values.astype(np.int8).reshape(outputs, reduction_blocks, 8, 4).transpose(1, 2, 0, 3))
    return scale_words, np.ascontiguousarray(groups.view(np.uint32).reshape(reduction_blocks * 8, outputs))


def split_q8_0_blocks(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Native Q8_0 activations [M, B, 34] -> (fp16 scale bits uint16 [M, B], int8 values as uint8 [M, B * 32]).

    The split activation operands of the reference's tiled tests
    (``tests/test_qpu_xla_ggml_q4_0.py:97-98``).
    """
    rows, nblocks, _ = blocks.shape
    scales = np.ascontiguousarray(blocks[..., :2]).view(np.uint16).reshape(rows, nblocks)
    values = np.ascontiguousarray(blocks[..., 2:].reshape(rows, nblocks * QK))
    return scales, values



# ------------------------------------------------ llama.cpp CPU_REPACK layouts

REPACK_GROUP_BYTES = 4 * Q4_0_BLOCK_BYTES      # block_q4_0x4: 4 fp16 scales + 64 code bytes
INTERLEAVED_BLOCK_BYTES = 4 * Q8_0_BLOCK_BYTES  # block_q8_0x4: 4 fp16 scales + 128 values


def unpack_q4_0x4(groups: np.ndarray) -> np.ndarray:
    """CPU_REPACK ``block_q4_0x4`` groups [N/4, B, 72] -> native Q4_0 blocks [N, B, 18].

    Follows ``unpack_q4_0_4x4`` (``integrations/llama_cpp/backend/ggml-qpu.cpp:250-284``):
    scale of column r at bytes 2r..2r+1; code bytes 4c..4c+3 of column r in
    word 4c + r of the 64 code bytes, each byte XOR 0x88.
    """
    groups = np.asarray(groups, dtype=np.uint8)
    if groups.ndim != 3 or groups.shape[2] != REPACK_GROUP_BYTES:
        raise ValueError("CPU_REPACK groups must have shape [N/4, blocks, 72]")
    n4, blocks, _ = groups.shape
    out = np.empty((n4, 4, blocks, Q4_0_BLOCK_BYTES), dtype=np.uint8)
    for row in range(4):
        out[:, row, :, 0:2] = groups[:, :, 2 * row:2 * row + 2]
        for chunk in range(4):
            word = 8 + (chunk * 4 + row) * 4
            out[:, row, :, 2 + 4 * chunk:6 + 4 * chunk] = groups[:, :, word:word + 4] ^ np.uint8(0x88)
    return out.reshape(n4 * 4, blocks, Q4_0_BLOCK_BYTES)


def pack_q4_0x4(blocks: np.ndarray) -> np.ndarray:
    """Native Q4_0 blocks [N, B, 18] (N % 4 == 0) -> CPU_REPACK groups: the inverse of ``unpack_q4_0x4``."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    if blocks.ndim != 3 or blocks.shape[2] != Q4_0_BLOCK_BYTES or blocks.shape[0] % 4:
        raise ValueError("native Q4_0 blocks must have shape [N, blocks, 18] with N % 4 == 0")
    n, nb, _ = blocks.shape
    cols = blocks.reshape(n // 4, 4, nb, Q4_0_BLOCK_BYTES)
    out = np.empty((n // 4, nb, REPACK_GROUP_BYTES), dtype=np.uint8)
    for row in range(4):
        out[:, :, 2 * row:2 * row + 2] = cols[:, row, :, 0:2]
        for chunk in range(4):
            word = 8 + (chunk * 4 + row) * 4
            out[:, :, word:word + 4] = cols[:, row, :, 2 + 4 * chunk:6 + 4 * chunk] ^ np.uint8(0x88)
    return out


def _interleaved_index(index: int, lane: int, interleave: int) -> int:
    # Position of value ``index`` of row ``lane`` inside a block_q8_0x4's 128 values
    # (qpu_llama_q4_0.c:189-203).
    return (index // interleave) * 4 * interleave + lane * interleave + index % interleave


def interleave_q8_0x4(rows: np.ndarray, interleave: int) -> np.ndarray:
    """Native Q8_0 rows [M, B, 34] -> CPU_REPACK activation bytes (same total size).

    Follows the packer of ``integrations/llama_cpp/tests/qpu_llama_q4_0_mx_smoke.c:23-45``:
    rows below M - M % 4 form block_q8_0x4 groups (the four scales, then the
    values at ``_interleaved_index``); the remaining rows stay native.
    """
    rows = np.asarray(rows, dtype=np.uint8)
    if interleave not in (4, 8) or rows.ndim != 3 or rows.shape[2] != Q8_0_BLOCK_BYTES:
        raise ValueError("interleave must be 4 or 8 and rows [M, blocks, 34]")
    m, nb, _ = rows.shape
    out = rows.reshape(m, nb * Q8_0_BLOCK_BYTES).copy()
    grouped = m - m % 4
    perm = np.array([[_interleaved_index(i, lane, interleave) for i in range(QK)] for lane in range(4)])
    for base in range(0, grouped, 4):
        group = np.empty((nb, INTERLEAVED_BLOCK_BYTES), dtype=np.uint8)
        for lane in range(4):
            native = rows[base + lane]
            group[:, 2 * lane:2 * lane + 2] = native[:, 0:2]
            group[:, 8 + perm[lane]] = native[:, 2:]
        out[base:base + 4] = group.reshape(4, nb * Q8_0_BLOCK_BYTES)
    return out.reshape(-1)


def deinterleave_q8_0x4(packed: np.ndarray, rows: int, blocks: int, interleave: int) -> np.ndarray:
    """CPU_REPACK activation bytes -> native Q8_0 rows [M, B, 34].

    Follows ``q8_0_source_block`` / ``q8_0_source_value``
    (``integrations/llama_cpp/src/qpu_llama_q4_0.c:160-203``).
    """
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    row_bytes = blocks * Q8_0_BLOCK_BYTES
    if interleave not in (4, 8) or packed.size < rows * row_bytes:
        raise ValueError("interleave must be 4 or 8 and the buffer must hold M rows")
    out = np.empty((rows, blocks, Q8_0_BLOCK_BYTES), dtype=np.uint8)
    grouped = rows - rows % 4
    for row in range(rows):
        for block in range(blocks):
            if row < grouped:
                group = (row // 4) * 4 * row_bytes + block * INTERLEAVED_BLOCK_BYTES
                lane = row % 4
                out[row, block, 0:2] = packed[group + 2 * lane:group + 2 * lane + 2]
                for index in range(QK):
                    out[row, block, 2 + index] = packed[group + 8 + _interleaved_index(index, lane, interleave)]
            else:
                start = row * row_bytes + block * Q8_0_BLOCK_BYTES
                out[row, block] = packed[start:start + Q8_0_BLOCK_BYTES]
    return out


# ------------------------------------------------------ lane layout (decode)

LANE_GROUP_UNITS = 64
LANE_UNIT_BYTES = 8 * Q4_0_BLOCK_BYTES  # 144: 8 blocks of one column


def pack_q4_0_lanes(blocks: np.ndarray) -> np.ndarray:
    """Native Q4_0 blocks [N, B, 18] (B % 8 == 0) -> the lane layout (flat uint8).

    The GPU library's decode-path weight layout (no reference counterpart; the
    reference re-lays weights out for its own kernels at prepare time,
    ``integrations/llama_cpp/src/qpu_llama_q4_0.c:343-395``): units of 144
    bytes (8 blocks of one column, native order), groups of 64 units, chunk v
    (16 bytes) of unit l of group q at ``q * 9216 + (v * 64 + l) * 16``; the
    last group is zero-padded.
    """
    blocks = np.asarray(blocks, dtype=np.uint8)
    if blocks.ndim != 3 or blocks.shape[2] != Q4_0_BLOCK_BYTES or blocks.shape[1] % 8:
        raise ValueError("lane layout needs blocks [N, B, 18] with B % 8 == 0")
    units = blocks.reshape(-1, LANE_UNIT_BYTES)
    groups = -(-units.shape[0] // LANE_GROUP_UNITS)
    padded = np.zeros((groups * LANE_GROUP_UNITS, LANE_UNIT_BYTES), dtype=np.uint8)
    padded[: units.shape[0]] = units
    chunks = padded.reshape(groups, LANE_GROUP_UNITS, 9, 16)
    return np.ascontiguousarray(chunks.transpose(0, 2, 1, 3)).reshape(-1)


def unpack_q4_0_lanes(packed: np.ndarray, columns: int, blocks: int) -> np.ndarray:
    """Inverse of ``pack_q4_0_lanes``."""
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    units = columns * (blocks // 8)
    groups = -(-units // LANE_GROUP_UNITS)
    chunks = packed[: groups * LANE_GROUP_UNITS * LANE_UNIT_BYTES].reshape(groups, 9, LANE_GROUP_UNITS, 16)
    unit_rows = chunks.transpose(0, 2, 1, 3).reshape(-1, LANE_UNIT_BYTES)[:units]
    return np.ascontiguousarray(unit_rows).reshape(columns, blocks, Q4_0_BLOCK_BYTES)


# ------------------------------------------------------------ Q8_0 x Q8_0


def q8_0_q8_0_reference(activation_blocks: np.ndarray, weight_blocks: np.ndarray) -> np.ndarray:
    """Q8_0 x Q8_0 linear: exact int32 block dots, scaled by da then dw, summed in block order.

    Follows ``ggml_q8_0_q8_0_reference`` (``src/qpu_xla/kernels/ggml_q8_0.py:26-51``):
    ``contribution = float32(dots); contribution *= da; contribution *= dw;
    result += contribution`` per block, all in float32.
    """
    activation_blocks = np.asarray(activation_blocks, dtype=np.uint8)
    weight_blocks = np.asarray(weight_blocks, dtype=np.uint8)
    if activation_blocks.ndim != 3 or weight_blocks.ndim != 3:
        raise ValueError("activation and weight blocks must both be rank three")
    rows, blocks, a_bytes = activation_blocks.shape
    outputs, w_blocks, w_bytes = weight_blocks.shape
    if a_bytes != Q8_0_BLOCK_BYTES or w_bytes != Q8_0_BLOCK_BYTES or blocks != w_blocks:
        raise ValueError("native Q8_0 block extents or counts do not match")
    da, qa = unpack_q8_0_blocks(activation_blocks)
    dw, qw = unpack_q8_0_blocks(weight_blocks)
    da = da.astype(np.float32)
    dw = dw.astype(np.float32)
    result = np.zeros((rows, outputs), dtype=np.float32)
    for b in range(blocks):
        dots = qa[:, b].astype(np.int32) @ qw[:, b].astype(np.int32).T
        term = dots.astype(np.float32)
        term *= da[:, b, None]
        term *= dw[None, :, b]
        result += term
    return result


# ------------------------------------------------------------ GEGLU -> Q8_0


def gelu_fp16_table() -> np.ndarray:
    """GGML's exact-GELU fp16 lookup table, u16 [65536] (a fresh copy per call).

    Follows ``ggml_gelu_fp16_table`` (``src/qpu_xla/kernels/ggml_geglu_q8.py:26-34``):
    entry ``i`` is ``0.5 x (1 + erf(x / sqrt 2))`` for ``x`` = the fp16 value
    with bits ``i``, evaluated in Python double arithmetic, stored into a
    float32 array (first rounding), then converted to float16 (second
    rounding, both to nearest even).
    """
    return _gelu_fp16_table().copy()


@lru_cache(maxsize=1)
def _gelu_fp16_table() -> np.ndarray:
    inputs = np.arange(1 << 16, dtype=np.uint16).view(np.float16).astype(np.float32)
    out = np.empty_like(inputs)
    root2 = math.sqrt(2.0)
    with np.errstate(invalid="ignore"):
        for index, value in enumerate(inputs):
            x = float(value)
            out[index] = 0.5 * x * (1.0 + math.erf(x / root2))
        table = np.ascontiguousarray(out.astype(np.float16).view(np.uint16))
    table.flags.writeable = False
    return table


def geglu_activate(gate: np.ndarray, up: np.ndarray, table: np.ndarray | None = None) -> np.ndarray:
    """``fl32(table[fp16(gate)] * up)``, fp32 [M, K] (``ggml_geglu_q8.py:46-48``)."""
    gate = np.asarray(gate, dtype=np.float32)
    up = np.asarray(up, dtype=np.float32)
    if gate.shape != up.shape or gate.ndim != 2 or gate.shape[1] % QK:
        raise ValueError("gate/up must be equal rank-two F32 arrays with K divisible by 32")
    lut = (_gelu_fp16_table() if table is None else np.asarray(table, dtype=np.uint16)).view(np.float16)
    with np.errstate(invalid="ignore", over="ignore"):
        return lut[gate.astype(np.float16).view(np.uint16)].astype(np.float32) * up


def geglu_q8_0_reference(gate: np.ndarray, up: np.ndarray, table: np.ndarray | None = None) -> np.ndarray:
    """Table GEGLU quantised straight to native Q8_0 blocks u8 [M, K/32, 34].

    Follows ``ggml_geglu_q8_0_reference`` (``src/qpu_xla/kernels/ggml_geglu_q8.py:37-59``):
    the activation of :func:`geglu_activate`, then per 32-element block
    ``d = fl32(absmax / 127)``, ``inverse = fl32(1 / d)`` (0 when d == 0),
    ``q = clip(rint(v * inverse), +-127)``, ``d`` stored as fp16 -- the rule
    of :func:`quantize_q8_0_split`, applied here to the activation.
    """
    return quantize_q8_0_blocks(geglu_activate(gate, up, table))


def geglu_q8_0_split_reference(
    gate: np.ndarray, up: np.ndarray, table: np.ndarray | None = None
) -> tuple[np.ndarray, np.ndarray]:
    """Split planes of :func:`geglu_q8_0_reference`: (scale words u32 [M, K/32], values int8 [M, K]).

    The scale word is the fp16 bits zero-extended, as the reference's split
    producer stores it (``ggml_geglu_q8.py:186-192``) and its test reads it
    (``tests/test_qpu_xla_ggml_geglu_q8.py:126-133``).
    """
    scale_bits, values = quantize_q8_0_split(geglu_activate(gate, up, table))
    return scale_bits.astype(np.uint32), values
