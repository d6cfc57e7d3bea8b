"""GPU tests of the llama.cpp-facing bridge (``include/qxt_llama_q4_0.h``), called through the C ABI.

They restate the reference's native smokes
(integrations/llama_cpp/tests/qpu_llama_q4_0_smoke.c, qpu_llama_q4_0_m4_smoke.c,
qpu_llama_q4_0_mx_smoke.c, qpu_llama_native_safety_smoke.c): closed-form
KATs, resident partitions with sentinels, guard bytes around host buffers,
invalid descriptors and executions, failure injection without partial output,
CPU_REPACK weights and Q8_0x4 activations.  Results are bit-exact against the
oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import load_golden
from qpu_xla_amd import _lib
from qpu_xla_amd.llama_bridge import (
    FORMAT_REPACK_4X4,
    WEIGHT_COLUMN_W8,
    WEIGHT_ROWCOL_W8A8,
    Execution,
    LlamaContext,
    LlamaQ4_0Linear,
)

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(123456.0)
GUARD = 64
GUARD_VALUE = 0xA5


def _desc(weights: np.ndarray, *, k: int, n: int, rows: int, start: int = 0, count: int | None = None, **extra):
    return dict(input_columns=k, output_columns=n, rows=rows, resident_column_start=start,
                resident_column_count=n - start if count is None else count, **extra)


@pytest.mark.parametrize("name", ["kat_q4_0_m1", "kat_q4_0_m4", "kat_q4_0_mx"])
def test_native_smoke_kats_with_hash_allocation_and_failure_injection(name: str) -> None:
    # qpu_llama_q4_0_smoke.c:15-143 (M=1), _m4_smoke.c (M=4), _mx_smoke.c (M=5, two blocks).
    g = load_golden(name)
    act, weight, expected = g["activation"], g["weight"], g["expected"]
    rows, blocks = act.shape[0], act.shape[1]
    n, start, count = weight.shape[0], int(g["resident_start"]), int(g["resident_count"])
    k = blocks * oracle.QK
    with LlamaContext() as ctx:
        desc = _desc(weight, k=k, n=n, rows=rows, start=start, count=count)
        status, handle = LlamaQ4_0Linear.prepare_status(ctx, weight, expected_source_hash="0" * 64, **desc)
        assert status == _lib.HASH_MISMATCH and not handle.value
        ctx.set_failure_mask(_lib.FAIL_ALLOCATION)
        status, handle = LlamaQ4_0Linear.prepare_status(ctx, weight, **desc)
        ctx.set_failure_mask(_lib.FAIL_NONE)
        assert status == _lib.ALLOCATION_FAILED and not handle.value
        ctx.set_failure_mask(_lib.FAIL_SOURCE_HASH)
        status, handle = LlamaQ4_0Linear.prepare_status(ctx, weight, **desc)
        ctx.set_failure_mask(_lib.FAIL_NONE)
        assert status == _lib.HASH_MISMATCH and not handle.value

        with LlamaQ4_0Linear(ctx, weight, **desc) as linear:
            assert linear.resident_bytes >= count * blocks * oracle.Q4_0_BLOCK_BYTES
            destination = np.full((rows, n), SENTINEL, dtype=np.float32)
            run = Execution(act, destination, start, count)
            timing = linear.execute(run)
            assert timing.complete_ns > 0 and timing.submit_wait_ns > 0
            np.testing.assert_array_equal(destination[:, :start], SENTINEL)
            np.testing.assert_array_equal(destination[:, start:], expected[:, start:])

            destination[:, start:] = -777.0
            ctx.set_failure_mask(_lib.FAIL_SUBMISSION)
            status, _ = linear.execute_status(run)
            ctx.set_failure_mask(_lib.FAIL_NONE)
            assert status == _lib.SUBMISSION_FAILED
            np.testing.assert_array_equal(destination[:, start:], -777.0)
            ctx.set_failure_mask(_lib.FAIL_WAIT)
            status, _ = linear.execute_status(run)
            ctx.set_failure_mask(_lib.FAIL_NONE)
            assert status == _lib.TIMEOUT
            np.testing.assert_array_equal(destination[:, start:], -777.0)
            # A failed wait poisons the context, as the reference runtime does.
            status, _ = linear.execute_status(run)
            assert status == _lib.IO_FAILED
            assert "poisoned" in ctx.last_error


def _guarded(payload: np.ndarray) -> np.ndarray:
    raw = np.full(GUARD + payload.nbytes + GUARD, GUARD_VALUE, dtype=np.uint8)
    raw[GUARD:GUARD + payload.nbytes] = payload.reshape(-1).view(np.uint8)
    return raw


@pytest.mark.parametrize("rows", [1, 4])
def test_native_safety_matrix(rows: int) -> None:
    # qpu_llama_native_safety_smoke.c:216-716 for the Q4_0 formats: zero weights and
    # activations, 48 output columns, guard bytes around every host buffer.
    n, k, tile = 48, 32, 16
    weights = _guarded(np.zeros((n, 1, oracle.Q4_0_BLOCK_BYTES), np.uint8))
    activation = _guarded(np.zeros((rows, 1, oracle.Q8_0_BLOCK_BYTES), np.uint8))
    w_bytes, a_bytes, d_bytes = n * 18, rows * 34, rows * n * 4
    dest_raw = np.empty(GUARD + d_bytes + GUARD, dtype=np.uint8)

    def reset() -> None:
        dest_raw[:] = GUARD_VALUE
        dest_raw[GUARD:GUARD + d_bytes].view(np.float32)[:] = SENTINEL

    def check(start: int, count: int, expect_output: bool) -> None:
        assert np.all(weights[:GUARD] == GUARD_VALUE) and np.all(weights[GUARD + w_bytes:] == GUARD_VALUE)
        assert not weights[GUARD:GUARD + w_bytes].any()
        assert np.all(activation[:GUARD] == GUARD_VALUE) and np.all(activation[GUARD + a_bytes:] == GUARD_VALUE)
        assert not activation[GUARD:GUARD + a_bytes].any()
        assert np.all(dest_raw[:GUARD] == GUARD_VALUE) and np.all(dest_raw[GUARD + d_bytes:] == GUARD_VALUE)
        out = dest_raw[GUARD:GUARD + d_bytes].view(np.float32).reshape(rows, n)
        want = np.full((rows, n), SENTINEL, np.float32)
        if expect_output:
            want[:, start:start + count] = 0.0
        np.testing.assert_array_equal(out, want)

    with LlamaContext() as ctx:
        base = dict(k=k, n=n, rows=rows)
        for bad in (dict(k=k - 1), dict(start=1, count=tile), dict(start=tile - 1, count=tile), dict(count=tile - 1),
                    dict(count=tile + 1), dict(count=0)):
            args = {**base, **bad}
            desc = _desc(weights, k=args["k"], n=n, rows=rows, start=args.get("start", 0), count=args.get("count"))
            status, handle = LlamaQ4_0Linear.prepare_status(ctx, weights[GUARD:GUARD + w_bytes], **desc)
            assert status == _lib.INVALID_ARGUMENT and not handle.value, bad
        status, handle = LlamaQ4_0Linear.prepare_status(ctx, weights[GUARD:GUARD + w_bytes],
                                                        weight_size=w_bytes - 1, **_desc(weights, **base))
        assert status == _lib.INVALID_ARGUMENT and not handle.value
        # The approximate weight modes need more than four rows (qpu_llama_q4_0.c:219).
        for mode in (WEIGHT_COLUMN_W8, WEIGHT_ROWCOL_W8A8):
            status, handle = LlamaQ4_0Linear.prepare_status(ctx, weights[GUARD:GUARD + w_bytes], weight_mode=mode,
                                                            **_desc(weights, k=k, n=n, rows=4))
            assert status == _lib.INVALID_ARGUMENT and not handle.value

        with LlamaQ4_0Linear(ctx, weights[GUARD:GUARD + w_bytes], **_desc(weights, **base)) as linear:
            def run(start: int, count: int, *, a_size: int = GUARD + a_bytes, d_size: int = GUARD + d_bytes) -> int:
                reset()
                status, _ = linear.execute_status(Execution(
                    activation, dest_raw, start, count, activation_offset=GUARD, destination_offset=GUARD,
                    activation_size=a_size, destination_size=d_size))
                return status

            partitions = [(0, n), (0, tile), (0, n - tile), (tile, tile), (tile, n - tile), (n - tile, tile)]
            for i in range(100 + len(partitions)):
                start, count = partitions[i % len(partitions)]
                assert run(start, count) == _lib.OK
                check(start, count, True)
            for start, count in ((0, 0), (0, tile - 1), (0, tile + 1), (1, tile)):
                assert run(start, count) == _lib.INVALID_ARGUMENT
                check(start, count, False)
            assert run(0, tile, a_size=GUARD + a_bytes - 1) == _lib.INVALID_ARGUMENT
            check(0, tile, False)
            assert run(0, tile, d_size=GUARD + d_bytes - 1) == _lib.INVALID_ARGUMENT
            check(0, tile, False)
            ctx.set_failure_mask(_lib.FAIL_SUBMISSION)
            assert run(0, n) == _lib.SUBMISSION_FAILED
            check(0, n, False)
            ctx.set_failure_mask(_lib.FAIL_WAIT)
            assert run(0, n) == _lib.TIMEOUT
            check(0, n, False)
            ctx.set_failure_mask(_lib.FAIL_NONE)


@pytest.mark.parametrize("interleave", [4, 8])
def test_interleaved_q8_0x4_activation_matches_native_rows(interleave: int) -> None:
    # qpu_llama_q4_0_mx_smoke.c: 5 rows (one group of four + one native row), two blocks.
    g = load_golden("kat_q4_0_mx")
    act, weight, expected = g["activation"], g["weight"], g["expected"]
    rows, blocks = act.shape[:2]
    n, start, count = weight.shape[0], int(g["resident_start"]), int(g["resident_count"])
    packed = oracle.interleave_q8_0x4(act, interleave)
    with LlamaContext() as ctx, LlamaQ4_0Linear(
            ctx, weight, **_desc(weight, k=blocks * 32, n=n, rows=rows, start=start, count=count)) as linear:
        destination = np.full((rows, n), SENTINEL, dtype=np.float32)
        status, submission = linear.submit_status(Execution(packed, destination, start, count, rows=rows,
                                                            activation_interleave=interleave))
        assert status == _lib.OK
        # One in-flight submission per linear.
        status2, _ = linear.submit_status(Execution(packed, destination, start, count))
        assert status2 == _lib.INTERNAL_ERROR
        status, _ = submission.wait_status()
        submission.destroy()
        assert status == _lib.OK
        np.testing.assert_array_equal(destination[:, :start], SENTINEL)
        np.testing.assert_array_equal(destination[:, start:], expected[:, start:])
        bad = Execution(packed, destination, start, count, activation_interleave=2)
        assert linear.execute_status(bad)[0] == _lib.INVALID_ARGUMENT


def _random_case(seed: int, rows: int, k: int, n: int):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((rows, k), dtype=np.float32)
    wq = oracle.quantize_q4_0_blocks(w)
    xq = oracle.quantize_q8_0_blocks(x)
    return xq, wq, oracle.q4_0_q8_0_reference(xq, wq)


@pytest.mark.parametrize("rows,k,n,start,count,run_rows", [
    (1, 2048, 5632, 0, 5632, 0),        # cfg0 decode shape
    (4, 4096, 4096, 1024, 2048, 0),     # cfg2 row count, a resident sub-range
    (32, 1024, 512, 0, 512, 19),        # prefill capacity, fewer rows submitted
])
def test_random_shapes_bit_exact_native_and_cpu_repack_weights(rows, k, n, start, count, run_rows) -> None:
    xq, wq, expected = _random_case(4000 + rows, rows, k, n)
    submitted = run_rows or rows
    with LlamaContext() as ctx:
        for fmt, weights in ((0, wq), (FORMAT_REPACK_4X4, oracle.pack_q4_0x4(wq))):
            with LlamaQ4_0Linear(ctx, np.ascontiguousarray(weights), weight_format=fmt,
                                 **_desc(wq, k=k, n=n, rows=rows, start=start, count=count)) as linear:
                destination = np.full((submitted, n), SENTINEL, dtype=np.float32)
                linear.execute(Execution(np.ascontiguousarray(xq[:submitted]), destination, start, count,
                                         rows=run_rows))
                np.testing.assert_array_equal(destination[:, :start], SENTINEL)
                np.testing.assert_array_equal(destination[:, start + count:], SENTINEL)
                np.testing.assert_array_equal(destination[:, start:start + count],
                                              expected[:submitted, start:start + count])


def test_repack_weight_format_requires_whole_groups() -> None:
    _, wq, _ = _random_case(7, 1, 64, 48)
    with LlamaContext() as ctx:
        status, handle = LlamaQ4_0Linear.prepare_status(
            ctx, np.ascontiguousarray(wq[:46]), weight_format=FORMAT_REPACK_4X4, **_desc(wq, k=64, n=46, rows=1, count=32))
        assert status == _lib.INVALID_ARGUMENT and not handle.value


def test_prepare_rejects_k_the_submit_path_cannot_run_and_runs_k14336_at_four_rows() -> None:
    rng = np.random.default_rng(7300)
    with LlamaContext() as ctx:
        k, n = 32768, 32  # four rows at K = 32768 exceed a workgroup's LDS
        weight = np.zeros((n, k // 32, 18), np.uint8)
        status, handle = LlamaQ4_0Linear.prepare_status(ctx, weight, **_desc(weight, k=k, n=n, rows=4))
        assert status == _lib.CAPABILITY_MISSING and not handle.value
        assert "LDS" in ctx.last_error
        status, handle = LlamaQ4_0Linear.prepare_status(ctx, weight, **_desc(weight, k=k, n=n, rows=1))
        assert status == _lib.OK  # one row fits
        _lib.load().qxt_llama_q4_0_linear_destroy(handle)

        k, n, rows = 14336, 256, 4
        w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        x = rng.standard_normal((rows, k), dtype=np.float32)
        wq, xq = oracle.quantize_q4_0_blocks(w), oracle.quantize_q8_0_blocks(x)
        with LlamaQ4_0Linear(ctx, wq, **_desc(wq, k=k, n=n, rows=rows)) as linear:
            destination = np.full((rows, n), SENTINEL, dtype=np.float32)
            linear.execute(Execution(xq, destination, 0, n))
            np.testing.assert_array_equal(destination, oracle.q4_0_q8_0_reference(xq, wq))


def test_cpu_fallback_after_a_failed_wait_computes_nothing() -> None:
    # The reference's M=1 hook calls the fallback after a failed wait
    # (ggml-qpu-up-inline.cpp:379-388); here it reports CAPABILITY_MISSING and
    # the destination keeps its bytes.
    g = load_golden("kat_q4_0_m1")
    act, weight = g["activation"], g["weight"]
    rows, blocks, n = act.shape[0], act.shape[1], weight.shape[0]
    with LlamaContext() as ctx, LlamaQ4_0Linear(ctx, weight, **_desc(weight, k=blocks * 32, n=n, rows=rows)) as linear:
        destination = np.full((rows, n), -777.0, dtype=np.float32)
        ctx.set_failure_mask(_lib.FAIL_WAIT)
        status, submission = linear.submit_status(Execution(act, destination, 0, n))
        assert status == _lib.OK
        status, _ = submission.wait_status()
        assert status == _lib.TIMEOUT
        assert submission.cpu_fallback_status() == _lib.CAPABILITY_MISSING
        assert "no CPU compute path" in ctx.last_error
        submission.destroy()
        np.testing.assert_array_equal(destination, -777.0)


def test_ggml_m1_hooks_register_by_name_and_execute(monkeypatch) -> None:
    # Patch 0002's call sequence: set_tensor registers native Q4_0 rows by
    # tensor name; forward_mul_mat executes one Q8_0 row (native, or passed
    # with INTER_SIZE 4 / 8 as CPU_REPACK does for a single row) and asks how
    # many columns the CPU must still compute.
    from qpu_xla_amd import ggml_hooks

    monkeypatch.setenv("GGML_QPU_M1_INLINE", "1")
    monkeypatch.setenv("GGML_QPU_M1_TENSORS", "ffn_up,attn_k")
    monkeypatch.setenv("GGML_QPU_TELEMETRY", "0")
    ggml_hooks.release()
    rng = np.random.default_rng(0)
    try:
        shapes = {"blk.3.ffn_up.weight": (2048, 5632), "blk.3.attn_k.weight": (2048, 256)}
        cases = {}
        for name, (k, n) in shapes.items():
            w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
            x = rng.standard_normal((1, k), dtype=np.float32)
            wq, xq = oracle.quantize_q4_0_blocks(w), oracle.quantize_q8_0_blocks(x)
            cases[name] = (k, n, wq, xq, oracle.q4_0_q8_0_reference(xq, wq)[0])
            assert ggml_hooks.register_q4_0(name, wq, k, n)
            assert ggml_hooks.register_q4_0(name, wq, k, n)  # already registered
            assert ggml_hooks.weight_registered(name)
        assert not ggml_hooks.register_q4_0("blk.3.ffn_down.weight", cases["blk.3.attn_k.weight"][2], 2048, 256)
        assert not ggml_hooks.weight_registered("blk.3.ffn_down.weight")
        base = ggml_hooks.dispatch_count()
        for interleave in (0, 4, 8):
            for name, (k, n, wq, xq, want) in cases.items():
                destination = np.full(n, np.nan, dtype=np.float32)
                assert ggml_hooks.execute(name, xq, destination, k, n, interleave)
                np.testing.assert_array_equal(destination, want)
                assert ggml_hooks.cpu_columns_for(name) == 0
                assert ggml_hooks.cpu_columns_for("blk.9.attn_q.weight") == 0
        assert ggml_hooks.dispatch_count() == base + 6

        k, n, wq, xq, want = cases["blk.3.ffn_up.weight"]
        destination = np.full(n, -5.0, dtype=np.float32)
        assert not ggml_hooks.execute("blk.3.ffn_up.weight", xq, destination, k, n + 16)  # shape mismatch
        assert not ggml_hooks.execute("blk.3.ffn_up.weight", xq, destination, k, n, rows=2)
        assert not ggml_hooks.execute("blk.3.ffn_up.weight", xq[:, :10], destination, k, n)  # short activation
        np.testing.assert_array_equal(destination, -5.0)
        assert ggml_hooks.cpu_columns_for("blk.3.ffn_up.weight") == n  # the CPU computes every column
        monkeypatch.setenv("GGML_QPU_M1_INLINE", "0")
        assert not ggml_hooks.execute("blk.3.ffn_up.weight", xq, destination, k, n)
        assert ggml_hooks.cpu_columns_for("blk.3.ffn_up.weight") == n
        np.testing.assert_array_equal(destination, -5.0)
        assert ggml_hooks.dispatch_count() == base + 6
    finally:
        ggml_hooks.release()
    assert not ggml_hooks.weight_registered("blk.3.ffn_up.weight")
