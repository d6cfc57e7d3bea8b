"""Python view of the ggml CPU_REPACK M=1 hooks (``include/qxt_ggml_hooks.h``).

llama.cpp binds the C symbols itself (weak references in its patched
``repack.cpp``, ``integrations/llama_cpp/patches/0002-ggml-cpu-inline-m1-q4-hook.patch:9-29``);
these wrappers call the same symbols through ctypes for tests and tools.
Registration and execution are opt-in through the reference's environment
variables ``GGML_QPU_M1_INLINE`` and ``GGML_QPU_M1_TENSORS``.
"""

from __future__ import annotations

import numpy as np

from qpu_xla_amd import _lib


def _host(buffer: np.ndarray) -> int:
    if not isinstance(buffer, np.ndarray) or not buffer.flags["C_CONTIGUOUS"]:
        raise ValueError("hook buffers must be C-contiguous NumPy arrays")
    return int(buffer.ctypes.data)


def register_q4_0(name: str, weights: np.ndarray, input_columns: int, output_columns: int) -> bool:
    """``ggml_qpu_m1_register_q4_0`` on native ggml Q4_0 rows; True when registered."""
    lib = _lib.load()
    return lib.ggml_qpu_m1_register_q4_0(name.encode(), _host(weights), weights.nbytes, input_columns,
                                         output_columns) == 1


def weight_registered(name: str) -> bool:
    return _lib.load().ggml_qpu_m1_weight_registered(name.encode()) == 1


def execute(name: str, activation_q8_0: np.ndarray, destination: np.ndarray, input_columns: int,
            output_columns: int, activation_interleave: int = 0, rows: int = 1) -> bool:
    """``ggml_qpu_m1_execute``: one Q8_0 row times the registered weight into ``destination`` (fp32)."""
    if destination.dtype != np.float32:
        raise ValueError("destination must be float32")
    return _lib.load().ggml_qpu_m1_execute(name.encode(), _host(activation_q8_0), activation_q8_0.nbytes,
                                           _host(destination), rows, input_columns, output_columns,
                                           activation_interleave) == 1


def cpu_columns_for(name: str) -> int:
    return int(_lib.load().ggml_qpu_m1_cpu_columns_for(name.encode()))


def dispatch_count() -> int:
    return int(_lib.load().ggml_qpu_m1_dispatch_count())


def release() -> None:
    _lib.load().ggml_qpu_m1_release()
