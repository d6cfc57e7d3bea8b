"""Python handle over the llama.cpp-facing C bridge (``include/qxt_llama_q4_0.h``).

Mirrors the reference's native bridge ``qpu_llama_q4_0_*``
(``integrations/llama_cpp/include/qpu_llama_q4_0.h:63-82``): host buffers in,
host buffers out, status codes instead of exceptions where the caller asks
for them.  Buffers are NumPy arrays (or anything exposing a writable host
pointer through ``ctypes``); the library copies them through pinned staging.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any

import numpy as np

from qpu_xla_amd import _lib

WEIGHT_EXACT = 0
WEIGHT_COLUMN_W8 = 1
WEIGHT_ROWCOL_W8A8 = 2
FORMAT_NATIVE = 0
FORMAT_REPACK_4X4 = 1


def source_hash() -> str:
    """The value ``expected_source_hash`` must carry for this build."""
    return _lib.load().qxt_llama_q4_0_source_hash().decode()


def status_string(status: int) -> str:
    """``qxt_llama_status_string`` (the reference's ``qpu_llama_status_string`` texts)."""
    return _lib.load().qxt_llama_status_string(status).decode()


def _host_pointer(buffer: np.ndarray) -> int:
    if not isinstance(buffer, np.ndarray) or not buffer.flags["C_CONTIGUOUS"]:
        raise ValueError("bridge buffers must be C-contiguous NumPy arrays")
    return int(buffer.ctypes.data)


class LlamaContext:
    """``qxt_llama_context``: one HIP device and stream, failure mask, last error."""

    def __init__(self, device: int = 0, *, timeout_ns: int = 0, failure_mask: int = 0) -> None:
        config = _lib.LlamaContextConfig(device, timeout_ns, failure_mask)
        handle = ctypes.c_void_p()
        _lib.check(_lib.load().qxt_llama_context_create(ctypes.byref(config), ctypes.byref(handle)))
        self.handle = handle

    def __enter__(self) -> "LlamaContext":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def close(self) -> None:
        if self.handle:
            _lib.load().qxt_llama_context_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    @property
    def last_error(self) -> str:
        return _lib.load().qxt_llama_context_last_error(self.handle).decode()

    def set_failure_mask(self, mask: int) -> None:
        _lib.load().qxt_llama_context_set_failure_mask(self.handle, mask)


@dataclass
class Execution:
    """Arguments of one submission (``qxt_llama_q4_0_execution``)."""

    activation: np.ndarray
    destination: np.ndarray
    column_start: int
    column_count: int
    rows: int = 0
    activation_interleave: int = 0
    activation_offset: int = 0
    destination_offset: int = 0
    activation_size: int | None = None
    destination_size: int | None = None

    def to_c(self) -> _lib.LlamaQ4_0Execution:
        return _lib.LlamaQ4_0Execution(
            _host_pointer(self.activation),
            self.activation.nbytes if self.activation_size is None else self.activation_size,
            self.activation_offset,
            _host_pointer(self.destination),
            self.destination.nbytes if self.destination_size is None else self.destination_size,
            self.destination_offset,
            self.column_start, self.column_count, self.rows, self.activation_interleave,
        )


class LlamaQ4_0Linear:
    """``qxt_llama_q4_0_linear``: resident Q4_0 weight columns on the GPU."""

    def __init__(
        self,
        context: LlamaContext,
        weights: np.ndarray,
        *,
        input_columns: int,
        output_columns: int,
        rows: int,
        resident_column_start: int = 0,
        resident_column_count: int | None = None,
        weight_mode: int = WEIGHT_EXACT,
        weight_format: int = FORMAT_NATIVE,
        expected_source_hash: str | None = None,
        weight_size: int | None = None,
    ) -> None:
        status, handle = self.prepare_status(
            context, weights, input_columns=input_columns, output_columns=output_columns, rows=rows,
            resident_column_start=resident_column_start,
            resident_column_count=output_columns - resident_column_start
            if resident_column_count is None else resident_column_count,
            weight_mode=weight_mode, weight_format=weight_format, expected_source_hash=expected_source_hash,
            weight_size=weight_size,
        )
        if status != _lib.OK:
            raise _lib.QxtError(status, context.last_error)
        self.context = context
        self.handle = handle

    @staticmethod
    def prepare_status(context: LlamaContext, weights: np.ndarray, **desc: Any) -> tuple[int, ctypes.c_void_p]:
        """Call ``qxt_llama_q4_0_linear_prepare`` and return (status, handle) without raising."""
        expected = desc.get("expected_source_hash")
        c_desc = _lib.LlamaQ4_0LinearDesc(
            _host_pointer(weights),
            weights.nbytes if desc.get("weight_size") is None else desc["weight_size"],
            desc["input_columns"], desc["output_columns"], desc["rows"],
            desc["resident_column_start"], desc["resident_column_count"],
            desc.get("weight_mode", WEIGHT_EXACT), 0,
            (source_hash() if expected is None else expected).encode(),
            desc.get("weight_format", FORMAT_NATIVE),
        )
        handle = ctypes.c_void_p()
        status = _lib.load().qxt_llama_q4_0_linear_prepare(context.handle, ctypes.byref(c_desc), ctypes.byref(handle))
        return int(status), handle

    def __enter__(self) -> "LlamaQ4_0Linear":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def close(self) -> None:
        if self.handle:
            _lib.load().qxt_llama_q4_0_linear_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    @property
    def resident_bytes(self) -> int:
        return int(_lib.load().qxt_llama_q4_0_linear_resident_bytes(self.handle))

    def execute_status(self, execution: Execution) -> tuple[int, _lib.LlamaQ4_0Timing]:
        """``qxt_llama_q4_0_linear_execute``: (status, timing) without raising."""
        timing = _lib.LlamaQ4_0Timing()
        c_exec = execution.to_c()
        status = _lib.load().qxt_llama_q4_0_linear_execute(self.handle, ctypes.byref(c_exec), ctypes.byref(timing))
        return int(status), timing

    def execute(self, execution: Execution) -> _lib.LlamaQ4_0Timing:
        status, timing = self.execute_status(execution)
        if status != _lib.OK:
            raise _lib.QxtError(status, self.context.last_error)
        return timing

    def submit_status(self, execution: Execution) -> tuple[int, "Submission | None"]:
        handle = ctypes.c_void_p()
        c_exec = execution.to_c()
        status = _lib.load().qxt_llama_q4_0_linear_submit(self.handle, ctypes.byref(c_exec), ctypes.byref(handle))
        return int(status), (Submission(handle) if status == _lib.OK else None)


class Submission:
    """``qxt_llama_q4_0_submission``: wait once, then destroy."""

    def __init__(self, handle: ctypes.c_void_p) -> None:
        self.handle = handle

    def wait_status(self) -> tuple[int, _lib.LlamaQ4_0Timing]:
        timing = _lib.LlamaQ4_0Timing()
        status = _lib.load().qxt_llama_q4_0_submission_wait(self.handle, ctypes.byref(timing))
        return int(status), timing

    def cpu_fallback_status(self) -> int:
        """``qxt_llama_q4_0_submission_cpu_fallback``: always CAPABILITY_MISSING (no CPU compute path)."""
        return int(_lib.load().qxt_llama_q4_0_submission_cpu_fallback(self.handle))

    def destroy(self) -> None:
        if self.handle:
            _lib.load().qxt_llama_q4_0_submission_destroy(self.handle)
            self.handle = ctypes.c_void_p()
