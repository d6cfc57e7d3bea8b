"""The C-ABI library loads, exports every declared symbol and validates on the host.

No test here launches GPU work: validation and failure injection return before
any HIP call, so these run in the GPU-less container.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from qpu_xla_amd import _lib

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_functions() -> list[str]:
    names: set[str] = set()
    for header in HEADERS:
        text = header.read_text()
        names.update(
            re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*((?:qxt|ggml_qpu)_\w+)\s*\(", text, flags=re.MULTILINE)
        )
    return sorted(names)


def test_header_declares_the_boundary() -> None:
    names = declared_functions()
    for required in (
        "qxt_quantize_q8_0",
        "qxt_quantize_rows_int8",
        "qxt_ggml_q4_0_q8_0_linear",
        "qxt_w8a8_gemm_dequantize",
        "qxt_w8a8_linear",
    ):
        assert required in names


def test_library_exports_every_declared_symbol() -> None:
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"


def test_binding_covers_exactly_the_header() -> None:
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_status_strings_and_version() -> None:
    lib = _lib.load()
    assert lib.qxt_abi_version() == 2
    assert _lib.status_string(_lib.OK) == "ok"
    assert _lib.status_string(_lib.SUBMISSION_FAILED) == "submission failed"
    assert _lib.status_string(_lib.TIMEOUT) == "timeout"
    assert _lib.status_string(99) == "unknown status"


def test_failure_mask_round_trip() -> None:
    _lib.set_failure_mask(_lib.FAIL_SUBMISSION | _lib.FAIL_WAIT)
    try:
        assert _lib.get_failure_mask() == _lib.FAIL_SUBMISSION | _lib.FAIL_WAIT
    finally:
        _lib.set_failure_mask(_lib.FAIL_NONE)
    assert _lib.get_failure_mask() == 0


FAKE = ctypes.c_void_p(1 << 20)  # 16-byte aligned, never dereferenced: validation or injection returns first


@pytest.mark.parametrize(
    "name,args,fragment",
    [
        ("qxt_quantize_q8_0", (None, 128, FAKE, 34, 1, 32, None), "null pointer"),
        ("qxt_quantize_q8_0", (FAKE, 128, FAKE, 34, 1, 40, None), "multiple of 32"),
        ("qxt_q8_0_scale_check", (None, None), "bad counter"),
        ("qxt_q8_0_scale_check", (ctypes.c_void_p((1 << 20) + 4), None), "bad counter"),
        ("qxt_hbm_read_probe", (None, 16, FAKE, None), "null or misaligned"),
        ("qxt_hbm_read_probe", (FAKE, 24, FAKE, None), "multiple of 16"),
        ("qxt_quantize_rows_int8", (FAKE, 64, FAKE, 8, FAKE, 1, 16, 8, 0, None), "padded_columns"),
        ("qxt_quantize_rows_int8", (FAKE, 64, FAKE, 16, FAKE, 1, 16, 16, 8, None), "unknown flags"),
        ("qxt_ggml_q4_0_q8_0_linear", (FAKE, 34, FAKE, 18, FAKE, 64, 0, 1, 0, 0, 16, None), "positive"),
        ("qxt_ggml_q4_0_q8_0_linear", (FAKE, 33, FAKE, 18, FAKE, 64, 1, 1, 0, 0, 16, None), "strides"),
        ("qxt_w8a8_gemm_i32", (FAKE, 16, FAKE, 16, FAKE, 64, 16, 16, 24, 0, None), "multiple of 16"),
        ("qxt_w8a8_gemm_i32", (FAKE, 16, FAKE, 16, FAKE, 64, 16, 16, 16, 7, None), "layout"),
        ("qxt_w8a8_gemm_i32", (FAKE, 2**20, FAKE, 2**20, FAKE, 2**20, 16, 16, 140000, 0, None), "overflow"),
        ("qxt_w8a8_gemm_dequantize", (FAKE, 16, FAKE, 16, None, FAKE, None, FAKE, 64, 16, 16, 16, 0, None), "null"),
        ("qxt_w8a8_dequantize", (FAKE, 64, FAKE, FAKE, None, FAKE, 32, 1, 16, None), "stride"),
        ("qxt_ggml_gelu_fp16_table", (None,), "null pointer"),
        ("qxt_ggml_geglu_q8_0", (FAKE, 256, FAKE, 256, None, FAKE, 68, 1, 64, None), "null pointer"),
        ("qxt_ggml_geglu_q8_0", (FAKE, 256, FAKE, 256, FAKE, FAKE, 68, 1, 48, None), "multiple of 32"),
        ("qxt_ggml_geglu_q8_0", (FAKE, 256, FAKE, 128, FAKE, FAKE, 68, 2, 64, None), "strides"),
        ("qxt_ggml_geglu_q8_0", (FAKE, 256, FAKE, 256, FAKE, FAKE, 67, 1, 64, None), "block stride"),
        ("qxt_ggml_geglu_q8_0_split", (FAKE, 256, FAKE, 256, FAKE, FAKE, 8, 3, FAKE, 64, 1, 64, None), "scale_bytes"),
        ("qxt_ggml_geglu_q8_0_split", (FAKE, 256, FAKE, 256, FAKE, FAKE, 8, 4, FAKE, 62, 1, 64, None), "strides"),
    ],
)
def test_invalid_arguments_are_rejected_on_the_host(name, args, fragment) -> None:
    status = getattr(_lib.load(), name)(*args)
    assert status == _lib.INVALID_ARGUMENT
    assert fragment in _lib.last_error()


def test_injected_submission_failure_returns_before_launch() -> None:
    lib = _lib.load()
    _lib.set_failure_mask(_lib.FAIL_SUBMISSION)
    try:
        status = lib.qxt_ggml_q4_0_q8_0_linear(FAKE, 34, FAKE, 18, FAKE, 64, 1, 1, 0, 0, 16, None)
        assert status == _lib.SUBMISSION_FAILED
        assert "injected" in _lib.last_error()
        status = lib.qxt_w8a8_gemm_i32(FAKE, 16, FAKE, 16, FAKE, 64, 16, 16, 16, 0, None)
        assert status == _lib.SUBMISSION_FAILED
        status = lib.qxt_ggml_geglu_q8_0(FAKE, 256, FAKE, 256, FAKE, FAKE, 68, 1, 64, None)
        assert status == _lib.SUBMISSION_FAILED
    finally:
        _lib.set_failure_mask(_lib.FAIL_NONE)


def test_injected_wait_failure_maps_to_timeout() -> None:
    lib = _lib.load()
    _lib.set_failure_mask(_lib.FAIL_WAIT)
    try:
        assert lib.qxt_stream_wait(None) == _lib.TIMEOUT
    finally:
        _lib.set_failure_mask(_lib.FAIL_NONE)


def test_qxt_error_carries_status_and_message() -> None:
    with pytest.raises(_lib.QxtError) as info:
        _lib.call("qxt_quantize_q8_0", None, 128, FAKE, 34, 1, 32, None)
    assert info.value.status == _lib.INVALID_ARGUMENT
    assert "null pointer" in str(info.value)


def test_q4_0_linear_rejects_k_beyond_the_lds_budget_before_launch() -> None:
    # K = 131072 needs more than 64 KB of LDS for the staged activation row.
    status = _lib.load().qxt_ggml_q4_0_q8_0_linear(FAKE, 4096 * 34, FAKE, 4096 * 18, FAKE, 64, 1, 4096, 0, 0, 16, None)
    assert status == _lib.CAPABILITY_MISSING
    assert "LDS" in _lib.last_error()


def test_llama_bridge_source_hash_is_the_build_hash() -> None:
    import importlib.util

    spec = importlib.util.spec_from_file_location("qxt_build", Path(__file__).resolve().parents[1] / "qpu-xla-triton_amd" / "build.py")
    builder = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(builder)
    from qpu_xla_amd import llama_bridge

    value = llama_bridge.source_hash()
    assert re.fullmatch(r"[0-9a-f]{64}", value)
    assert value == builder.source_hash(), "library is stale: rebuild before testing"


def test_llama_bridge_validates_on_the_host() -> None:
    lib = _lib.load()
    handle = ctypes.c_void_p()
    assert lib.qxt_llama_context_create(None, None) == _lib.INVALID_ARGUMENT
    injected = _lib.LlamaContextConfig(0, 0, _lib.FAIL_DEVICE_OPEN)
    assert lib.qxt_llama_context_create(ctypes.byref(injected), ctypes.byref(handle)) == _lib.DEVICE_UNAVAILABLE
    assert not handle.value
    unknown = _lib.LlamaContextConfig(0, 0, 1 << 9)
    assert lib.qxt_llama_context_create(ctypes.byref(unknown), ctypes.byref(handle)) == _lib.INVALID_ARGUMENT
    desc = _lib.LlamaQ4_0LinearDesc()
    assert lib.qxt_llama_q4_0_linear_prepare(None, ctypes.byref(desc), ctypes.byref(handle)) == _lib.INVALID_ARGUMENT
    execution = _lib.LlamaQ4_0Execution()
    assert lib.qxt_llama_q4_0_linear_submit(None, ctypes.byref(execution), ctypes.byref(handle)) == _lib.INVALID_ARGUMENT
    assert lib.qxt_llama_q4_0_submission_wait(None, None) == _lib.INVALID_ARGUMENT
    assert lib.qxt_llama_q4_0_linear_execute(None, None, None) == _lib.INVALID_ARGUMENT
    assert lib.qxt_llama_q4_0_linear_resident_bytes(None) == 0
    assert lib.qxt_llama_context_last_error(None) == b"no context"
    lib.qxt_llama_q4_0_linear_destroy(None)
    lib.qxt_llama_q4_0_submission_destroy(None)
    lib.qxt_llama_context_destroy(None)


def test_llama_status_string_matches_the_reference_texts() -> None:
    from qpu_xla_amd.llama_bridge import status_string

    # qpu_llama_runtime.c:751-765.
    texts = ["ok", "invalid argument", "device unavailable", "capability missing", "allocation failed",
             "I/O failed", "submission failed", "timeout", "hash mismatch", "internal error"]
    for status, text in enumerate(texts):
        assert status_string(status) == text
    assert status_string(42) == "unknown status"


def test_cpu_fallback_of_no_submission_is_invalid() -> None:
    assert _lib.load().qxt_llama_q4_0_submission_cpu_fallback(None) == _lib.INVALID_ARGUMENT


def test_ggml_m1_hooks_decline_without_opt_in(monkeypatch) -> None:
    # Disabled or unselected tensors are declined before any HIP call.
    from qpu_xla_amd import ggml_hooks

    weights = np.zeros((16, 1, 18), np.uint8)
    monkeypatch.delenv("GGML_QPU_M1_INLINE", raising=False)
    monkeypatch.setenv("GGML_QPU_M1_TENSORS", "ffn_up")
    assert not ggml_hooks.register_q4_0("blk.0.ffn_up.weight", weights, 32, 16)
    monkeypatch.setenv("GGML_QPU_M1_INLINE", "1")
    assert not ggml_hooks.register_q4_0("blk.0.attn_q.weight", weights, 32, 16)  # not selected
    monkeypatch.setenv("GGML_QPU_M1_TENSORS", "")
    assert not ggml_hooks.register_q4_0("blk.0.ffn_up.weight", weights, 32, 16)  # empty selection
    monkeypatch.setenv("GGML_QPU_M1_TENSORS", "attn,ffn_up")
    assert not ggml_hooks.register_q4_0("blk.0.ffn_up.weight", weights, 40, 16)  # K % 32
    assert not ggml_hooks.register_q4_0("blk.0.ffn_up.weight", weights, 32, 24)  # N % 16
    assert not ggml_hooks.weight_registered("blk.0.ffn_up.weight")
    destination = np.zeros(16, np.float32)
    activation = np.zeros((1, 34), np.uint8)
    assert not ggml_hooks.execute("blk.0.ffn_up.weight", activation, destination, 32, 16)
    assert ggml_hooks.cpu_columns_for("blk.0.ffn_up.weight") == 0
    assert ggml_hooks.dispatch_count() == 0
    lib = _lib.load()
    assert lib.ggml_qpu_m1_weight_registered(None) == 0
    assert lib.ggml_qpu_m1_cpu_columns_for(None) == 0


def test_q4_0_linear_k_limits_per_row_count_before_launch() -> None:
    # Four rows at K = 32768 need ~192 KB of LDS (> the 160 KB of a workgroup):
    # rejected with CAPABILITY_MISSING before anything is enqueued.
    lib = _lib.load()
    blocks = 32768 // 32
    status = lib.qxt_ggml_q4_0_q8_0_linear(FAKE, blocks * 34, FAKE, blocks * 18, FAKE, 64, 4, blocks, 0, 0, 16, None)
    assert status == _lib.CAPABILITY_MISSING
    assert "LDS" in _lib.last_error() and "4 rows" in _lib.last_error()


def test_w8a8_linear_noalloc_rejects_sizes_beyond_its_workspace_before_launch() -> None:
    lib = _lib.load()
    # m * k = 4096 * 16400 bytes > 64 MiB; m = 65537 rows > 65,536 scales.
    status = lib.qxt_w8a8_linear_noalloc(FAKE, 16400 * 4, FAKE, 16400, FAKE, None, FAKE, 64, 4096, 16, 16400, 0, 0, None)
    assert status == _lib.INVALID_ARGUMENT and "static workspace" in _lib.last_error()
    status = lib.qxt_w8a8_linear_noalloc(FAKE, 64, FAKE, 16, FAKE, None, FAKE, 64, 65537, 16, 16, 0, 0, None)
    assert status == _lib.INVALID_ARGUMENT and "static workspace" in _lib.last_error()
    status = lib.qxt_w8a8_linear_noalloc(FAKE, 64, FAKE, 16, FAKE, None, FAKE, 64, 4, 16, 24, 0, 0, None)
    assert status == _lib.INVALID_ARGUMENT and "multiple of 16" in _lib.last_error()


def test_allocation_count_is_a_host_counter() -> None:
    # Nothing in the host-only tests allocates device memory through the library.
    assert _lib.allocation_count() == 0
