"""ctypes binding of ``libqxt_gfx950.so`` (declared in ``include/qxt_gfx950.h``,
``include/qxt_llama_q4_0.h`` and ``include/qxt_ggml_hooks.h``).

The library is built in-tree by ``qpu-xla-triton_amd/build.py``.  There is no
fallback: when the library is missing every entry point raises
``LibraryMissingError``.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import (
    POINTER,
    Structure,
    c_char,
    c_char_p,
    c_int,
    c_int32,
    c_int64,
    c_size_t,
    c_uint32,
    c_uint64,
    c_void_p,
)
from pathlib import Path
from typing import Any

LIBRARY_PATH = Path(__file__).with_name("libqxt_gfx950.so")

# Status codes (values of qpu_llama_status, integrations/llama_cpp/include/qpu_llama_runtime.h:16-27).
OK = 0
INVALID_ARGUMENT = 1
DEVICE_UNAVAILABLE = 2
CAPABILITY_MISSING = 3
ALLOCATION_FAILED = 4
IO_FAILED = 5
SUBMISSION_FAILED = 6
TIMEOUT = 7
HASH_MISMATCH = 8
INTERNAL_ERROR = 9

# Failure-injection bits (qpu_llama_failure_point, qpu_llama_runtime.h:29-36).
FAIL_NONE = 0
FAIL_DEVICE_OPEN = 1 << 0
FAIL_ALLOCATION = 1 << 1
FAIL_SUBMISSION = 1 << 2
FAIL_WAIT = 1 << 3
FAIL_SOURCE_HASH = 1 << 4  # llama bridge contexts only

QUANT_NO_SCALE_FLOOR = 1
Q4_0_LAYOUT_NATIVE = 0
Q4_0_LAYOUT_LANES = 1
WEIGHT_NK = 0
WEIGHT_K4N = 1


class DeviceInfo(Structure):
    _fields_ = [
        ("arch", c_char * 64),
        ("compute_units", c_int32),
        ("clock_khz", c_int32),
        ("memory_clock_khz", c_int32),
        ("memory_bus_width", c_int32),
        ("total_memory", c_int64),
        ("l2_bytes", c_int32),
        ("lds_bytes_per_cu", c_int32),
    ]


class LaunchRecord(Structure):
    _fields_ = [("kernel", c_char * 48), ("ms", ctypes.c_float)]


class Q4Task(Structure):
    """``qxt_q4_0_task``: one linear of a Q4_0 batch."""

    _fields_ = [
        ("x", c_void_p),
        ("x_row_stride", c_size_t),
        ("activation", c_void_p),
        ("activation_row_stride", c_size_t),
        ("weight", c_void_p),
        ("weight_row_stride", c_size_t),
        ("destination", c_void_p),
        ("destination_row_stride", c_size_t),
        ("rows", c_uint32),
        ("blocks", c_uint32),
        ("weight_column_start", c_uint32),
        ("output_column_start", c_uint32),
        ("column_count", c_uint32),
        ("weight_layout", c_uint32),
    ]


class LlamaContextConfig(Structure):
    """``qxt_llama_context_config``."""

    _fields_ = [("device", c_int32), ("timeout_ns", c_uint64), ("failure_mask", c_uint32)]


class LlamaQ4_0LinearDesc(Structure):
    """``qxt_llama_q4_0_linear_desc`` (fields of qpu_llama_q4_0_linear_desc + weight_format)."""

    _fields_ = [
        ("weights", c_void_p),
        ("weight_size", c_size_t),
        ("input_columns", c_uint32),
        ("output_columns", c_uint32),
        ("rows", c_uint32),
        ("resident_column_start", c_uint32),
        ("resident_column_count", c_uint32),
        ("weight_mode", c_int),
        ("workgroups_per_supergroup", c_uint32),
        ("expected_source_hash", c_char_p),
        ("weight_format", c_int),
    ]


class LlamaQ4_0Execution(Structure):
    """``qxt_llama_q4_0_execution`` (fields of qpu_llama_q4_0_execution)."""

    _fields_ = [
        ("activation", c_void_p),
        ("activation_size", c_size_t),
        ("activation_offset", c_size_t),
        ("destination", c_void_p),
        ("destination_size", c_size_t),
        ("destination_offset", c_size_t),
        ("column_start", c_uint32),
        ("column_count", c_uint32),
        ("rows", c_uint32),
        ("activation_interleave", c_uint32),
    ]


class LlamaQ4_0Timing(Structure):
    """``qxt_llama_q4_0_timing`` (fields of qpu_llama_q4_0_timing), nanoseconds."""

    _fields_ = [(name, c_uint64) for name in (
        "input_access_ns", "input_pack_ns", "input_sync_ns", "input_copy_ns", "submit_ns", "wait_ns",
        "submit_wait_ns", "output_sync_ns", "output_copy_ns", "complete_ns",
    )]


_P = c_void_p
_SZ = c_size_t
_U = c_uint32

SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "qxt_abi_version": (c_int, []),
    "qxt_status_string": (c_char_p, [c_int]),
    "qxt_last_error": (c_char_p, []),
    "qxt_set_failure_mask": (None, [_U]),
    "qxt_get_failure_mask": (_U, []),
    "qxt_allocation_count": (c_uint64, []),
    "qxt_device_query": (c_int, [POINTER(DeviceInfo)]),
    "qxt_stream_wait": (c_int, [_P]),
    "qxt_timing_begin": (c_int, []),
    "qxt_timing_end": (c_int, [POINTER(LaunchRecord), _U, POINTER(_U)]),
    "qxt_quantize_q8_0": (c_int, [_P, _SZ, _P, _SZ, _U, _U, _P]),
    "qxt_q8_0_scale_check": (c_int, [_P, _P]),
    "qxt_hbm_read_probe": (c_int, [_P, c_size_t, _P, _P]),
    "qxt_quantize_rows_int8": (c_int, [_P, _SZ, _P, _SZ, _P, _U, _U, _U, _U, _P]),
    "qxt_quantize_q4_0": (c_int, [_P, _SZ, _P, _SZ, _U, _U, _P]),
    "qxt_ggml_gelu_fp16_table": (c_int, [_P]),
    "qxt_ggml_geglu_q8_0": (c_int, [_P, _SZ, _P, _SZ, _P, _P, _SZ, _U, _U, _P]),
    "qxt_ggml_geglu_q8_0_split": (c_int, [_P, _SZ, _P, _SZ, _P, _P, _SZ, _U, _P, _SZ, _U, _U, _P]),
    "qxt_ggml_q4_0_q8_0_linear": (c_int, [_P, _SZ, _P, _SZ, _P, _SZ, _U, _U, _U, _U, _U, _P]),
    "qxt_ggml_q4_0_q8_0_block_dots": (c_int, [_P, _SZ, _P, _SZ, _P, _U, _U, _U, _U, _P]),
    "qxt_ggml_q8_0_q8_0_linear": (c_int, [_P, _SZ, _P, _SZ, _P, _SZ, _U, _U, _U, _U, _U, _P]),
    "qxt_q4_0_lanes_bytes": (_SZ, [_U, _U]),
    "qxt_q4_0_pack_lanes": (c_int, [_P, _SZ, _P, _SZ, _U, _U, _P]),
    "qxt_ggml_q4_0_q8_0_linear_lanes": (c_int, [_P, _SZ, _P, _U, _P, _SZ, _U, _U, _U, _U, _U, _P]),
    "qxt_ggml_q4_0_q8_0_tiled_linear": (c_int, [_P, _SZ, _P, _SZ, _U, _P, _SZ, _P, _SZ, _P, _SZ, _U, _U, _U, _P]),
    "qxt_q4_0_batch_prepare": (c_int, [POINTER(Q4Task), _U, POINTER(c_void_p)]),
    "qxt_q4_0_batch_launch": (c_int, [_P, _P]),
    "qxt_q4_0_batch_work_items": (_U, [_P]),
    "qxt_q4_0_batch_destroy": (None, [_P]),
    "qxt_w8a8_gemm_i32": (c_int, [_P, _SZ, _P, _SZ, _P, _SZ, _U, _U, _U, _U, _P]),
    "qxt_w8a8_gemm_dequantize": (c_int, [_P, _SZ, _P, _SZ, _P, _P, _P, _P, _SZ, _U, _U, _U, _U, _P]),
    "qxt_w8a8_dequantize": (c_int, [_P, _SZ, _P, _P, _P, _P, _SZ, _U, _U, _P]),
    "qxt_w8a8_linear": (c_int, [_P, _SZ, _P, _SZ, _P, _P, _SZ, _P, _P, _P, _SZ, _U, _U, _U, _U, _U, _P]),
    "qxt_w8a8_linear_noalloc": (c_int, [_P, _SZ, _P, _SZ, _P, _P, _P, _SZ, _U, _U, _U, _U, _U, _P]),
    "qxt_llama_context_create": (c_int, [POINTER(LlamaContextConfig), POINTER(c_void_p)]),
    "qxt_llama_context_destroy": (None, [_P]),
    "qxt_llama_context_last_error": (c_char_p, [_P]),
    "qxt_llama_context_set_failure_mask": (None, [_P, _U]),
    "qxt_llama_q4_0_source_hash": (c_char_p, []),
    "qxt_llama_q4_0_linear_prepare": (c_int, [_P, POINTER(LlamaQ4_0LinearDesc), POINTER(c_void_p)]),
    "qxt_llama_q4_0_linear_destroy": (None, [_P]),
    "qxt_llama_q4_0_linear_resident_bytes": (_SZ, [_P]),
    "qxt_llama_q4_0_linear_submit": (c_int, [_P, POINTER(LlamaQ4_0Execution), POINTER(c_void_p)]),
    "qxt_llama_q4_0_submission_wait": (c_int, [_P, POINTER(LlamaQ4_0Timing)]),
    "qxt_llama_q4_0_submission_destroy": (None, [_P]),
    "qxt_llama_q4_0_linear_execute": (c_int, [_P, POINTER(LlamaQ4_0Execution), POINTER(LlamaQ4_0Timing)]),
    "qxt_llama_q4_0_submission_cpu_fallback": (c_int, [_P]),
    "qxt_llama_status_string": (c_char_p, [c_int]),
    # ggml CPU_REPACK M=1 hooks (include/qxt_ggml_hooks.h)
    "ggml_qpu_m1_register_q4_0": (c_int, [c_char_p, _P, _SZ, c_uint64, c_uint64]),
    "ggml_qpu_m1_weight_registered": (c_int, [c_char_p]),
    "ggml_qpu_m1_execute": (c_int, [c_char_p, _P, _SZ, _P, c_uint64, c_uint64, c_uint64, c_uint64]),
    "ggml_qpu_m1_cpu_columns_for": (c_uint64, [c_char_p]),
    "ggml_qpu_m1_dispatch_count": (c_uint64, []),
    "ggml_qpu_m1_release": (None, []),
}


class LibraryMissingError(RuntimeError):
    """The gfx950 library has not been built; there is no CPU fallback."""


class QxtError(RuntimeError):
    """A library call returned a non-OK status."""

    def __init__(self, status: int, message: str) -> None:
        super().__init__(f"{status_string(status)} ({status}): {message}")
        self.status = status
        self.message = message


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library with typed signatures."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.exists():
            raise LibraryMissingError(
                f"{LIBRARY_PATH} is missing: build it with `python qpu-xla-triton_amd/build.py` "
                "(the quantized-linear path has no CPU fallback)"
            )
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def status_string(status: int) -> str:
    try:
        return load().qxt_status_string(status).decode()
    except LibraryMissingError:
        return f"status {status}"


def last_error() -> str:
    raw = load().qxt_last_error()
    return raw.decode() if raw else ""


def check(status: int) -> None:
    """Raise ``QxtError`` for a non-OK status."""
    if status != OK:
        raise QxtError(status, last_error())


def call(name: str, *args: Any) -> None:
    """Call an entry point and raise on a non-OK status."""
    check(getattr(load(), name)(*args))


def set_failure_mask(mask: int) -> None:
    load().qxt_set_failure_mask(mask)


def get_failure_mask() -> int:
    return int(load().qxt_get_failure_mask())


def allocation_count() -> int:
    """Device and pinned-host allocations the library has made in this process."""
    return int(load().qxt_allocation_count())


def device_info() -> DeviceInfo:
    info = DeviceInfo()
    check(load().qxt_device_query(ctypes.byref(info)))
    return info


class launch_timing:
    """Context manager collecting device time of every kernel launched inside it.

    ``records`` holds ``(kernel_name, milliseconds)`` in launch order after exit.
    Uses the library's per-launch start/stop events (not usable under graph capture).
    """

    def __init__(self, capacity: int = 65536) -> None:
        self.capacity = capacity
        self.records: list[tuple[str, float]] = []

    def __enter__(self) -> "launch_timing":
        check(load().qxt_timing_begin())
        return self

    def __exit__(self, *exc: object) -> None:
        buf = (LaunchRecord * self.capacity)()
        count = c_uint32(0)
        check(load().qxt_timing_end(buf, self.capacity, ctypes.byref(count)))
        n = min(int(count.value), self.capacity)
        self.records = [(buf[i].kernel.decode(), float(buf[i].ms)) for i in range(n)]
