"""CPU oracle for the quantized-linear hot path (TEST INFRASTRUCTURE ONLY).

This package is a NumPy restatement of the reference's CPU algorithms for the
Q4_0 x Q8_0 block-dot linear, the Q8_0 / Q4_0 / per-row int8 quantisers and
the dynamic W8A8 int8 GEMM with its dequant + bias epilogue.  Every function
cites the reference file:line it follows (paths are relative to the
``yiannisha/qpu-xla-triton`` source tree).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and only as the checker / the timed CPU baseline.  The
product package (``qpu_xla_amd``) never imports or calls it: the product
path is the HIP library and fails loudly when that library is missing.

Pinning status (what each function is checked against, in ``tests/``):

* block codecs: round trips plus the reference's extreme-value cases
  (tests/test_qpu_xla_ggml_q4_0.py:25-44 in the reference).
* ``q4_0_q8_0_reference``: closed-form integer KATs of the native smokes
  (integrations/llama_cpp/tests/qpu_llama_q4_0_smoke.c:15-36,
  qpu_llama_q4_0_m4_smoke.c:17-40), exact power-of-two-scale cases, and a
  float64 dequantised brute force.
* ``quantize_q8_0_*``: invariants (|q| <= 127, absmax maps to +-127, fp16
  RNE scale) and exact half-way ties that separate ``rint`` from ``round``.
* W8A8: closed-form KAT (qpu_llama_w8a8_smoke.c:58-66), int64 brute force,
  quantiser invariants including the 1/127 scale floor.
* ``pack_q4_0_tiled_weights`` / ``split_q8_0_blocks``: byte-level checks of
  the word layout against the native blocks and exact inversion.
* CPU_REPACK layouts (``unpack_q4_0x4`` / ``pack_q4_0x4``,
  ``deinterleave_q8_0x4`` / ``interleave_q8_0x4``): exact inversion both
  ways, the signed-nibble meaning of the 0x88 mask (each packed nibble is the
  two's-complement 4-bit value code - 8), and the native-smoke expectation
  that an interleaved activation gives the native result
  (qpu_llama_q4_0_mx_smoke.c:47-180).
* ``q8_0_q8_0_reference``: the reference's own check against the explicit
  dequantised float dot (tests/test_qpu_xla_ggml_q8_0.py:16-31), a Python
  brute force of the int32 block dots with power-of-two scales (exact), and
  a case where scaling by dw first would round differently.
* ``pack_q4_0_lanes``: exact inversion and the byte position of every
  16-byte chunk (a layout of this library, checked against its definition
  chunk by chunk; the kernels' parity is then pinned by the linear's oracle).
* ``gelu_fp16_table``: every entry against the same two roundings of an
  independent erf (SciPy's), textbook values of the normal CDF
  (x * Phi(x) at x = +-1, +-2, +-3), gelu(x) = x exactly for large x and the
  odd-part identity gelu(x) - gelu(-x) = x within fp16 rounding.
* ``geglu_q8_0_reference`` / ``geglu_q8_0_split_reference``: the reference's
  own layout test (tests/test_qpu_xla_ggml_geglu_q8.py:24-30); the fp16
  table index checked against torch's half conversion on exact fp16 ties;
  cases that reduce to the pinned Q8_0 quantiser (up = 1 with gates where
  gelu is the identity or exactly zero); dequantised blocks within half a
  step of gelu(gate) * up computed in float64; the split planes against the
  native blocks byte for byte.
* ``oracle/llama_approx.py`` (the bridge's COLUMN_W8 / ROWCOL_W8A8 modes):
  hand-worked columns and rows whose literal codes separate half-away
  rounding from half-even and exact rounding (the fp32 ``+ 0.5`` before the
  truncation), zero columns and rows, random data re-derived in exact
  rational arithmetic (on data where a reciprocal multiply would differ),
  power-of-two-scale linears that are exact, and a case where applying the
  column scale per block rounds differently from applying it once.
* ``quantize_q4_0_blocks``: ggml's published ``quantize_row_q4_0_ref`` rule
  (upstream ggml is not vendored in the reference, so there is no runnable
  copy); pinned by hand-worked known-answer blocks whose literal codes and
  fp16 scale bits separate the plausible mistakes (half-way values round up,
  not to even and not by truncating x/d + 8; the first element of largest
  magnitude sets the sign; x * fl32(1/d), not x / d; codes from the fp32 d,
  not its fp16 rounding; -0.0 scale of a zero block; fp16-subnormal scales),
  by the same blocks and random blocks re-derived in exact rational
  arithmetic with explicit round-to-fp32 steps, and by the half-step
  reconstruction bound (``tests/test_oracle_ggml.py``).
"""

from oracle.ggml import (  # noqa: F401
    Q4_0_BLOCK_BYTES,
    Q8_0_BLOCK_BYTES,
    QK,
    deinterleave_q8_0x4,
    gelu_fp16_table,
    geglu_activate,
    geglu_q8_0_reference,
    geglu_q8_0_split_reference,
    interleave_q8_0x4,
    pack_q4_0_blocks,
    pack_q4_0_lanes,
    pack_q4_0x4,
    pack_q4_0_tiled_weights,
    pack_q8_0_blocks,
    q4_0_q8_0_block_dots,
    q4_0_q8_0_reference,
    q8_0_q8_0_reference,
    quantize_q4_0_blocks,
    quantize_q8_0_blocks,
    quantize_q8_0_split,
    split_q8_0_blocks,
    unpack_q4_0_blocks,
    unpack_q4_0_lanes,
    unpack_q4_0x4,
    unpack_q8_0_blocks,
)
from oracle.w8a8 import (  # noqa: F401
    SCALE_FLOOR,
    dequantize_epilogue,
    int8_gemm_i32,
    pack_int8_gemm_operands,
    pack_int8_quads,
    quantize_per_output_channel_int8,
    quantize_rows_int8,
    w8a8_linear_reference,
)
