"""Measured-candidate archive that gates automatic placement.

JSON-compatible with the reference's ``CandidateRegistry``
(``src/qpu_xla/benchmark/candidates.py:13-330``): the same record fields,
status strings, evidence gates and ``schema_version`` 1-3 payloads, so an
archive written by either side loads in the other.  The one extension is the
``"gpu"`` placement, which names records measured for this library's HIP
kernels; ``"qpu"`` records describe VideoCore programs and are kept (and
saved back) but never executed here.

A record is scheduler-visible only with status ``supported-win``, which
requires correctness evidence without NaN/Inf and a measured win (median
CPU time / median candidate time >= 1.05, or a fused-model win).
"""

from __future__ import annotations

import json
from dataclasses import asdict, dataclass, fields
from enum import Enum
from os import PathLike
from statistics import median
from typing import Any

SCHEMA_VERSION = 3
LOADABLE_SCHEMAS = (1, 2, 3)
PLACEMENTS = ("cpu", "qpu", "hybrid", "gpu")
WIN_THRESHOLD = 1.05


class CandidateStatus(Enum):
    """Lifecycle state of one candidate (values are the archive strings)."""

    SUPPORTED_WIN = "supported-win"
    SAME_CONTRACT_WIN = "same-contract-win"
    EXPERIMENTAL_CORRECT_SLOWER = "experimental-correct-slower"
    QUARANTINED_INCORRECT = "quarantined-incorrect"
    REFERENCE_ONLY = "reference-only"


def _nonnegative(*values: float) -> bool:
    return all(v >= 0 for v in values)


@dataclass(frozen=True, slots=True)
class CorrectnessEvidence:
    """Numerical comparison of a candidate against a named reference."""

    reference: str
    cases: int
    exact: bool
    max_abs_error: float
    mean_abs_error: float
    p99_abs_error: float
    max_relative_error: float
    saturation_count: int = 0
    nan_count: int = 0
    inf_count: int = 0

    def __post_init__(self) -> None:
        if not self.reference or self.cases <= 0:
            raise ValueError("correctness evidence requires a reference and at least one case")
        if not _nonnegative(self.max_abs_error, self.mean_abs_error, self.p99_abs_error, self.max_relative_error,
                            self.saturation_count, self.nan_count, self.inf_count):
            raise ValueError("correctness errors and counts cannot be negative")


@dataclass(frozen=True, slots=True)
class PerformanceEvidence:
    """Whole-operation wall-time samples (seconds) of a reference and a candidate."""

    cpu_reference: str
    cpu_seconds: tuple[float, ...]
    candidate_seconds: tuple[float, ...]
    fused_model_win: bool = False
    host_prep_seconds: tuple[float, ...] = ()
    kernel_seconds: tuple[float, ...] = ()
    cold_start_seconds: tuple[float, ...] = ()
    dequantization_seconds: tuple[float, ...] = ()
    same_contract_reference: str = ""
    same_contract_seconds: tuple[float, ...] = ()

    def __post_init__(self) -> None:
        if not self.cpu_reference or not self.cpu_seconds or not self.candidate_seconds:
            raise ValueError("performance evidence requires both CPU and candidate samples")
        samples = [
            *self.cpu_seconds, *self.candidate_seconds, *self.host_prep_seconds, *self.kernel_seconds,
            *self.cold_start_seconds, *self.dequantization_seconds, *self.same_contract_seconds,
        ]
        if any(s <= 0 for s in samples):
            raise ValueError("performance samples must be positive")
        if bool(self.same_contract_reference) != bool(self.same_contract_seconds):
            raise ValueError("same-contract performance requires both a reference and samples")

    @property
    def cpu_median_seconds(self) -> float:
        return float(median(self.cpu_seconds))

    @property
    def candidate_median_seconds(self) -> float:
        return float(median(self.candidate_seconds))

    @property
    def speedup(self) -> float:
        return self.cpu_median_seconds / self.candidate_median_seconds

    @property
    def measured_win(self) -> bool:
        """Clears the 5 % gate against the fastest CPU reference (or wins inside a fused model)."""
        return self.fused_model_win or self.speedup >= WIN_THRESHOLD

    @property
    def same_contract_speedup(self) -> float | None:
        if not self.same_contract_seconds:
            return None
        return float(median(self.same_contract_seconds)) / self.candidate_median_seconds

    @property
    def same_contract_win(self) -> bool:
        speedup = self.same_contract_speedup
        return speedup is not None and speedup >= WIN_THRESHOLD


@dataclass(frozen=True, slots=True)
class PartitionEvidence:
    """Split of one operator's work along ``axis`` ("rows" or "outputs").

    ``qpu_units`` is the size of the leading partition (the accelerator
    prefix in the reference); the remainder is the trailing partition.  Both
    must be non-empty and the prefix a multiple of ``alignment``.
    """

    axis: str
    qpu_units: int
    total_units: int
    alignment: int = 1

    def __post_init__(self) -> None:
        if not self.axis or self.total_units <= 0 or self.alignment <= 0:
            raise ValueError("partition evidence requires an axis and positive sizes")
        if not 0 < self.qpu_units < self.total_units:
            raise ValueError("partition evidence must retain work on both CPU and QPU")
        if self.qpu_units % self.alignment:
            raise ValueError("partition evidence does not satisfy its alignment")


@dataclass(frozen=True, slots=True)
class QualityEvidence:
    """Error of a quantized format against its fp32 source-domain reference."""

    reference: str
    normalized_rmse: float
    cosine_similarity: float
    max_abs_error: float = 0.0
    mean_abs_error: float = 0.0
    p99_abs_error: float = 0.0
    nan_count: int = 0
    inf_count: int = 0
    top1_agreement: float | None = None

    def __post_init__(self) -> None:
        if not self.reference or not _nonnegative(self.normalized_rmse, self.max_abs_error, self.mean_abs_error,
                                                  self.p99_abs_error):
            raise ValueError("quality evidence requires a reference and non-negative NRMSE")
        if not -1.0 <= self.cosine_similarity <= 1.0:
            raise ValueError("quality cosine similarity must be within [-1, 1]")
        if self.nan_count < 0 or self.inf_count < 0:
            raise ValueError("quality NaN and Inf counts cannot be negative")
        if self.top1_agreement is not None and not 0.0 <= self.top1_agreement <= 1.0:
            raise ValueError("quality top-1 agreement must be within [0, 1]")

    @property
    def passes_default_gate(self) -> bool:
        return (self.normalized_rmse <= 0.10 and self.cosine_similarity >= 0.99
                and self.nan_count == 0 and self.inf_count == 0)


@dataclass(frozen=True, slots=True)
class CandidateRecord:
    """One kernel specialisation for one exact operation class, with its evidence."""

    name: str
    operation: str
    dtype: str
    layout: str
    shape_class: str
    source_hash: str
    status: CandidateStatus
    correctness: CorrectnessEvidence | None = None
    performance: PerformanceEvidence | None = None
    reason: str = ""
    placement: str = "qpu"
    kernels: tuple[str, ...] = ()
    partition: PartitionEvidence | None = None
    quality: QualityEvidence | None = None

    def __post_init__(self) -> None:
        if not all((self.name, self.operation, self.dtype, self.layout, self.shape_class, self.source_hash)):
            raise ValueError("candidate identity fields must be non-empty")
        if self.placement not in PLACEMENTS:
            raise ValueError("candidate placement must be cpu, qpu, hybrid, or gpu")
        if (self.placement == "hybrid") != (self.partition is not None):
            if self.partition is None:
                raise ValueError("hybrid candidate records require partition evidence")
            raise ValueError("only hybrid candidate records may include partition evidence")
        clean = self.correctness is not None and not (self.correctness.nan_count or self.correctness.inf_count)
        if self.status is CandidateStatus.SUPPORTED_WIN:
            if self.correctness is None or self.performance is None or not self.performance.measured_win:
                raise ValueError("supported candidates require correctness and a measured or fused win")
            if not clean:
                raise ValueError("supported candidates cannot produce NaN or Inf outputs")
        elif self.status is CandidateStatus.SAME_CONTRACT_WIN:
            if self.correctness is None or self.performance is None or not self.performance.same_contract_win:
                raise ValueError("same-contract winners require correctness and a measured W8A8 CPU win")
            if not clean:
                raise ValueError("same-contract winners cannot produce NaN or Inf outputs")
        elif self.status is CandidateStatus.EXPERIMENTAL_CORRECT_SLOWER and self.correctness is None:
            raise ValueError("correct experimental candidates require correctness evidence")
        elif self.status is CandidateStatus.QUARANTINED_INCORRECT and not self.reason:
            raise ValueError("quarantined candidates require a failure reason")

    def to_json(self) -> dict[str, Any]:
        payload = asdict(self)
        payload["status"] = self.status.value
        return payload

    @classmethod
    def from_json(cls, raw: Any) -> "CandidateRecord":
        if not isinstance(raw, dict):
            raise ValueError("candidate registry records must be objects")
        item = dict(raw)
        item["status"] = CandidateStatus(item["status"])
        for key, evidence in (("correctness", CorrectnessEvidence), ("partition", PartitionEvidence),
                              ("quality", QualityEvidence)):
            if item.get(key) is not None:
                item[key] = evidence(**item[key])
        if item.get("performance") is not None:
            perf = dict(item["performance"])
            for f in fields(PerformanceEvidence):
                if f.name.endswith("_seconds") and f.name in perf:
                    perf[f.name] = tuple(perf[f.name])
            item["performance"] = PerformanceEvidence(**perf)
        if "kernels" in item:
            item["kernels"] = tuple(item["kernels"])
        return cls(**item)


class CandidateRegistry:
    """Ordered, uniquely named candidate archive; only measured winners are visible to dispatch."""

    def __init__(self, records: tuple[CandidateRecord, ...] = ()) -> None:
        self._by_name: dict[str, CandidateRecord] = {}
        for record in records:
            self.register(record)

    @property
    def records(self) -> tuple[CandidateRecord, ...]:
        return tuple(self._by_name.values())

    @property
    def supported(self) -> tuple[CandidateRecord, ...]:
        return tuple(r for r in self._by_name.values() if r.status is CandidateStatus.SUPPORTED_WIN)

    def supported_for(self, *, operation: str, dtype: str, layout: str, shape_class: str) -> tuple[CandidateRecord, ...]:
        """Supported winners for exactly this operation, dtype, layout and shape class."""
        key = (operation, dtype, layout, shape_class)
        return tuple(r for r in self.supported if (r.operation, r.dtype, r.layout, r.shape_class) == key)

    def register(self, record: CandidateRecord) -> None:
        if record.name in self._by_name:
            raise ValueError(f"candidate {record.name!r} is already registered")
        self._by_name[record.name] = record

    @classmethod
    def combine(cls, *registries: "CandidateRegistry") -> "CandidateRegistry":
        return cls(tuple(r for registry in registries for r in registry.records))

    def to_dict(self) -> dict[str, Any]:
        return {"schema_version": SCHEMA_VERSION, "records": [r.to_json() for r in self.records]}

    def save(self, path: str | PathLike[str]) -> None:
        with open(path, "w", encoding="utf-8") as out:
            json.dump(self.to_dict(), out, indent=2, sort_keys=True)

    @classmethod
    def from_dict(cls, payload: Any) -> "CandidateRegistry":
        if not isinstance(payload, dict) or payload.get("schema_version") not in LOADABLE_SCHEMAS:
            raise ValueError("unsupported candidate registry schema")
        raw_records = payload.get("records")
        if not isinstance(raw_records, list):
            raise ValueError("candidate registry records must be a list")
        records = []
        for raw in raw_records:
            try:
                records.append(CandidateRecord.from_json(raw))
            except (KeyError, TypeError, ValueError) as exc:
                raise ValueError("candidate registry contains an invalid record") from exc
        return cls(tuple(records))

    @classmethod
    def load(cls, path: str | PathLike[str]) -> "CandidateRegistry":
        with open(path, encoding="utf-8") as source:
            return cls.from_dict(json.load(source))


__all__ = [
    "CandidateRecord",
    "CandidateRegistry",
    "CandidateStatus",
    "CorrectnessEvidence",
    "PartitionEvidence",
    "PerformanceEvidence",
    "QualityEvidence",
]
