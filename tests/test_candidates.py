"""Candidate archive (JSON compatibility, evidence gates) and W8A8 dispatch selection (host logic)."""

from __future__ import annotations

import json

import pytest

from qpu_xla_amd.candidates import (
    CandidateRecord,
    CandidateRegistry,
    CandidateStatus,
    CorrectnessEvidence,
    PartitionEvidence,
    PerformanceEvidence,
    QualityEvidence,
)
from qpu_xla_amd.placement import Placement
from qpu_xla_amd.quantization import W8A8_DTYPE, W8A8_LAYOUT, select_w8a8_dispatch, w8a8_shape_class


def _exact() -> CorrectnessEvidence:
    return CorrectnessEvidence("oracle-int64", 8, True, 0.0, 0.0, 0.0, 0.0)


def _linear(name: str, shape: str, candidate_s: float, *, placement: str = "gpu",
            partition: PartitionEvidence | None = None, status=CandidateStatus.SUPPORTED_WIN) -> CandidateRecord:
    return CandidateRecord(
        name, "linear", W8A8_DTYPE, W8A8_LAYOUT, shape, "src", status, _exact(),
        PerformanceEvidence("numpy-int32", (0.010,), (candidate_s,)),
        placement=placement, partition=partition,
    )


def test_registry_round_trips_winners_and_slower_candidates(tmp_path) -> None:
    winning = CandidateRecord(
        "packed-gemm-h2048", "w8a8-gemm", "int8-int32", "packed-k4", "llama-h2048-prefill", "abc123",
        CandidateStatus.SUPPORTED_WIN, _exact(), PerformanceEvidence("torch", (0.010, 0.011), (0.008, 0.009)),
    )
    slower = CandidateRecord(
        "packed-gemv-h2048", "w8a8-gemv", "int8-int32", "packed-k4", "llama-h2048-decode", "def456",
        CandidateStatus.EXPERIMENTAL_CORRECT_SLOWER, _exact(), PerformanceEvidence("numpy", (0.001,), (0.002,)),
        "correct but slower on this shape",
    )
    path = tmp_path / "candidates.json"
    CandidateRegistry((winning, slower)).save(path)
    restored = CandidateRegistry.load(path)
    assert [r.name for r in restored.supported] == ["packed-gemm-h2048"]
    assert restored.records == (winning, slower)
    assert restored.supported_for(operation="w8a8-gemm", dtype="int8-int32", layout="packed-k4",
                                  shape_class="llama-h2048-prefill") == (winning,)
    assert not restored.supported_for(operation="w8a8-gemv", dtype="int8-int32", layout="packed-k4",
                                      shape_class="llama-h2048-decode")
    assert CandidateRegistry.combine(CandidateRegistry((winning,)), CandidateRegistry((slower,))).records == (
        winning, slower)
    with pytest.raises(ValueError, match="duplicate candidate name"):
        CandidateRegistry((winning, winning))


def test_registry_round_trips_partition_quality_and_same_contract(tmp_path) -> None:
    hybrid = CandidateRecord(
        "w8a8-hybrid", "linear", W8A8_DTYPE, W8A8_LAYOUT, "64x1024x2816", "source", CandidateStatus.SUPPORTED_WIN,
        _exact(), PerformanceEvidence("numpy-fp32", (0.010,), (0.008,), host_prep_seconds=(0.001,),
                                      kernel_seconds=(0.005,)),
        placement="hybrid", kernels=("gfx950.w8a8_linear", "gfx950.w8a8_linear"),
        partition=PartitionEvidence("rows", 16, 64, 16), quality=QualityEvidence("numpy-fp32", 0.08, 0.995),
    )
    same = CandidateRecord(
        "same-contract-only", "linear", W8A8_DTYPE, W8A8_LAYOUT, "64x64x64", "hash",
        CandidateStatus.SAME_CONTRACT_WIN, _exact(),
        PerformanceEvidence("torch-fp32", (0.0005,), (0.001,), dequantization_seconds=(0.0001,),
                            same_contract_reference="numpy-int32-dynamic-w8a8", same_contract_seconds=(0.002,)),
        quality=QualityEvidence("numpy-fp32", 0.02, 0.999, max_abs_error=0.1, top1_agreement=1.0),
    )
    path = tmp_path / "hybrid.json"
    CandidateRegistry((hybrid, same)).save(path)
    restored = CandidateRegistry.load(path)
    assert restored.records == (hybrid, same)
    assert restored.records[0].quality.passes_default_gate
    assert restored.supported == (hybrid,)
    assert restored.records[1].performance.same_contract_win
    assert restored.records[1].performance.same_contract_speedup == 2.0
    payload = json.loads(path.read_text())
    assert payload["schema_version"] == 3
    assert payload["records"][0]["status"] == "supported-win"
    assert payload["records"][0]["partition"] == {"axis": "rows", "qpu_units": 16, "total_units": 64, "alignment": 16}


def test_registry_loads_older_schemas_and_qpu_records() -> None:
    # A schema-1 archive as the reference wrote it: no placement/kernels/partition/quality keys.
    payload = {
        "schema_version": 1,
        "records": [{
            "name": "vc7-linear", "operation": "linear", "dtype": W8A8_DTYPE, "layout": W8A8_LAYOUT,
            "shape_class": "16x16x16", "source_hash": "abc", "status": "supported-win",
            "correctness": {"reference": "numpy", "cases": 1, "exact": True, "max_abs_error": 0.0,
                            "mean_abs_error": 0.0, "p99_abs_error": 0.0, "max_relative_error": 0.0},
            "performance": {"cpu_reference": "torch", "cpu_seconds": [0.002], "candidate_seconds": [0.001]},
            "reason": "",
        }],
    }
    registry = CandidateRegistry.from_dict(payload)
    (record,) = registry.records
    assert record.placement == "qpu" and record.performance.cpu_seconds == (0.002,)
    assert registry.to_dict()["records"][0]["placement"] == "qpu"
    with pytest.raises(ValueError, match="schema_version must be 1, 2 or 3"):
        CandidateRegistry.from_dict({"schema_version": 4, "records": []})
    with pytest.raises(ValueError, match="must be a JSON list"):
        CandidateRegistry.from_dict({"schema_version": 3, "records": {}})
    broken = json.loads(json.dumps(payload))
    broken["records"][0]["status"] = "promoted"
    with pytest.raises(ValueError, match="is malformed"):
        CandidateRegistry.from_dict(broken)


def test_evidence_gates() -> None:
    with pytest.raises(ValueError, match="needs correctness evidence and a measured win"):
        _linear("slow", "1x16x16", 0.0099)  # 1.01x: below the 5 % gate
    assert _linear("fast", "1x16x16", 0.0095).performance.measured_win  # 1.053x
    fused = CandidateRecord("fused", "linear", W8A8_DTYPE, W8A8_LAYOUT, "1x16x16", "h",
                            CandidateStatus.SUPPORTED_WIN, _exact(),
                            PerformanceEvidence("torch", (0.001,), (0.002,), fused_model_win=True))
    assert fused.performance.speedup == 0.5 and fused.performance.measured_win
    with pytest.raises(ValueError, match="NaN or Inf"):
        CandidateRecord("nan", "linear", W8A8_DTYPE, W8A8_LAYOUT, "1x16x16", "h", CandidateStatus.SUPPORTED_WIN,
                        CorrectnessEvidence("numpy", 1, False, 1.0, 1.0, 1.0, 1.0, nan_count=1),
                        PerformanceEvidence("torch", (0.002,), (0.001,)))
    with pytest.raises(ValueError, match="needs a reason"):
        CandidateRecord("bad", "linear", W8A8_DTYPE, W8A8_LAYOUT, "s", "h", CandidateStatus.QUARANTINED_INCORRECT)
    with pytest.raises(ValueError, match="needs partition evidence"):
        _linear("h", "1x16x16", 0.001, placement="hybrid")
    with pytest.raises(ValueError, match="hybrid records only"):
        _linear("g", "1x16x16", 0.001, partition=PartitionEvidence("rows", 16, 32, 16))
    with pytest.raises(ValueError, match="placement must be"):
        _linear("x", "1x16x16", 0.001, placement="npu")
    with pytest.raises(ValueError, match="both partitions must be non-empty"):
        PartitionEvidence("rows", 32, 32, 16)
    with pytest.raises(ValueError, match="alignment"):
        PartitionEvidence("outputs", 8, 32, 16)
    with pytest.raises(ValueError, match="> 0 seconds"):
        PerformanceEvidence("torch", (0.0,), (0.001,))
    with pytest.raises(ValueError, match="cosine"):
        QualityEvidence("numpy", 0.1, 1.5)


def _registry() -> CandidateRegistry:
    shape = w8a8_shape_class(32, 16, 32)
    return CandidateRegistry((
        _linear("gpu", shape, 0.004),
        _linear("hybrid-rows", shape, 0.001, placement="hybrid", partition=PartitionEvidence("rows", 16, 32, 16)),
        _linear("hybrid-outputs", shape, 0.002, placement="hybrid",
                partition=PartitionEvidence("outputs", 16, 32, 16)),
        _linear("vc7", shape, 0.0001, placement="qpu"),
        CandidateRecord("slower", "linear", W8A8_DTYPE, W8A8_LAYOUT, shape, "src",
                        CandidateStatus.EXPERIMENTAL_CORRECT_SLOWER, _exact(),
                        PerformanceEvidence("numpy-int32", (0.001,), (0.0000001,)), placement="gpu"),
        _linear("other-shape", w8a8_shape_class(16, 16, 32), 0.00001),
    ))


def test_dispatch_auto_takes_the_fastest_executable_record() -> None:
    reg = _registry()
    pick = select_w8a8_dispatch(reg, batch=32, features=16, outputs=32, partition_queue=True)
    assert (pick.record.name, pick.placement, pick.axis, pick.units) == ("hybrid-rows", Placement.HYBRID, "rows", 16)
    # Without a second queue the partitioned records are not executable; "qpu" records never are.
    pick = select_w8a8_dispatch(reg, batch=32, features=16, outputs=32)
    assert (pick.record.name, pick.placement) == ("gpu", Placement.GPU)
    pick = select_w8a8_dispatch(reg, batch=32, features=16, outputs=32, qpu_outputs=16, partition_queue=True)
    assert pick.record.name == "hybrid-outputs" and pick.axis == "outputs"
    pick = select_w8a8_dispatch(reg, batch=32, features=16, outputs=32, placement=Placement.GPU, partition_queue=True)
    assert pick.record.name == "gpu"
    pick = select_w8a8_dispatch(reg, batch=32, features=16, outputs=32, placement=Placement.HYBRID,
                                partition_queue=True)
    assert pick.record.name == "hybrid-rows"


def test_dispatch_rejections() -> None:
    reg = _registry()
    kw = dict(batch=32, features=16, outputs=32, partition_queue=True)
    with pytest.raises(ValueError, match="mutually exclusive"):
        select_w8a8_dispatch(reg, qpu_rows=16, qpu_outputs=16, **kw)
    with pytest.raises(ValueError, match="require HYBRID or AUTO"):
        select_w8a8_dispatch(reg, placement=Placement.GPU, qpu_rows=16, **kw)
    with pytest.raises(ValueError, match="no CPU placement"):
        select_w8a8_dispatch(reg, placement=Placement.CPU, **kw)
    with pytest.raises(ValueError, match="QPU placement does not exist"):
        select_w8a8_dispatch(reg, placement=Placement.QPU, **kw)
    with pytest.raises(ValueError, match="partition matches"):
        select_w8a8_dispatch(reg, qpu_rows=8, **kw)
    with pytest.raises(ValueError, match="hybrid candidate"):
        select_w8a8_dispatch(reg, batch=32, features=16, outputs=32, placement=Placement.HYBRID)
    with pytest.raises(ValueError, match="no CPU reference fallback"):
        select_w8a8_dispatch(reg, batch=31, features=16, outputs=32)
    vc7_only = CandidateRegistry((_linear("vc7", w8a8_shape_class(4, 16, 16), 0.001, placement="qpu"),))
    with pytest.raises(ValueError, match="no CPU reference fallback"):
        select_w8a8_dispatch(vc7_only, batch=4, features=16, outputs=16)
    with pytest.raises(ValueError, match="GPU candidate"):
        select_w8a8_dispatch(vc7_only, batch=4, features=16, outputs=16, placement=Placement.GPU)


def test_archive_format_is_preserved_key_for_key() -> None:
    # A schema-3 archive in the reference's layout loads and saves back to the
    # same JSON (every field, nested evidence objects, tuples as lists).
    record = {
        "name": "w8a8-rows", "operation": "linear", "dtype": W8A8_DTYPE, "layout": W8A8_LAYOUT,
        "shape_class": "64x1024x2816", "source_hash": "f00d", "status": "supported-win", "reason": "",
        "placement": "hybrid", "kernels": ["a", "b"],
        "correctness": {"reference": "numpy", "cases": 3, "exact": True, "max_abs_error": 0.0,
                        "mean_abs_error": 0.0, "p99_abs_error": 0.0, "max_relative_error": 0.0,
                        "saturation_count": 0, "nan_count": 0, "inf_count": 0},
        "performance": {"cpu_reference": "torch", "cpu_seconds": [0.003, 0.002], "candidate_seconds": [0.001],
                        "fused_model_win": False, "host_prep_seconds": [], "kernel_seconds": [0.0005],
                        "cold_start_seconds": [], "dequantization_seconds": [], "same_contract_reference": "",
                        "same_contract_seconds": []},
        "partition": {"axis": "rows", "qpu_units": 32, "total_units": 64, "alignment": 16},
        "quality": {"reference": "fp32", "normalized_rmse": 0.01, "cosine_similarity": 0.999,
                    "max_abs_error": 0.1, "mean_abs_error": 0.01, "p99_abs_error": 0.05, "nan_count": 0,
                    "inf_count": 0, "top1_agreement": None},
    }
    payload = {"schema_version": 3, "records": [record]}
    registry = CandidateRegistry.from_dict(json.loads(json.dumps(payload)))
    assert json.dumps(registry.to_dict(), sort_keys=True) == json.dumps(payload, sort_keys=True)
    assert registry.records[0].partition.trailing == 32
    with pytest.raises(ValueError, match="unknown keys"):
        CandidateRegistry.from_dict({"schema_version": 2, "records": [dict(record, promoted=True)]})
