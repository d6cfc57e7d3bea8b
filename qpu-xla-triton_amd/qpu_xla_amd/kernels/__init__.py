"""gfx950 kernels of the quantized-linear path, one module per reference kernel module."""

from qpu_xla_amd.kernels.gemm_int8 import (  # noqa: F401
    TILED_W8A8_GEMM_DEQUANTIZE_KERNEL,
    TILED_W8A8_GEMM_KERNEL,
    pack_int8_gemm_operands,
    pack_int8_quads,
    supports_tiled_w8a8_gemm,
    supports_tiled_w8a8_gemm_dequantize,
    w8a8_gemm_dequantize,
    w8a8_gemm_i32,
)
from qpu_xla_amd.kernels.gemv_int8 import W8A8_GEMV_KERNEL, supports_w8a8_gemv  # noqa: F401
from qpu_xla_amd.kernels.ggml_geglu_q8 import (  # noqa: F401
    GGML_GEGLU_Q8_0_KERNEL,
    GGML_GEGLU_Q8_0_SPLIT_KERNEL,
    ggml_geglu_q8_0,
    ggml_geglu_q8_0_split,
    ggml_gelu_fp16_table,
    supports_ggml_geglu_q8_0,
    supports_ggml_geglu_q8_0_split,
)
from qpu_xla_amd.kernels.ggml_q4_0 import (  # noqa: F401
    GGML_Q4_0_Q8_0_LINEAR_KERNEL,
    GGML_Q4_0_Q8_0_TILED_LINEAR_KERNEL,
    Q4_0LaneWeights,
    Q4_0LinearBatch,
    ggml_q4_0_q8_0_block_dots,
    ggml_q4_0_q8_0_lane_linear,
    ggml_q4_0_q8_0_linear,
    ggml_q4_0_q8_0_tiled_linear,
    pack_ggml_q4_0_blocks,
    pack_ggml_q4_0_lane_weights,
    pack_ggml_q4_0_tiled_weights,
    pack_ggml_q8_0_blocks,
    split_ggml_q8_0_blocks,
    supports_ggml_q4_0_q8_0_linear,
    supports_ggml_q4_0_q8_0_tiled_linear,
    unpack_ggml_q4_0_blocks,
    unpack_ggml_q8_0_blocks,
)
from qpu_xla_amd.kernels.ggml_q8_0 import (  # noqa: F401
    GGML_Q8_0_Q8_0_LINEAR_M4_KERNEL,
    ggml_q8_0_q8_0_linear,
    supports_ggml_q8_0_q8_0_linear_m4,
)
from qpu_xla_amd.kernels.quantize import quantize_q4_0, quantize_q8_0, quantize_rows_int8  # noqa: F401
from qpu_xla_amd.kernels.w8a8_epilogue import W8A8_DEQUANTIZE_KERNEL, supports_w8a8_dequantize, w8a8_dequantize  # noqa: F401
