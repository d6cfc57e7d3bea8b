"""Archive of measured kernel candidates; only measured winners reach calibrated dispatch.

The on-disk format is the reference's candidate archive
(``src/qpu_xla/benchmark/candidates.py:13-330``) so that archives move between
the two libraries unchanged: a JSON object ``{"schema_version": 1 | 2 | 3,
"records": [...]}`` (written as version 3, sorted keys, two-space indent), each
record an object whose keys are the field names of :class:`CandidateRecord`
and whose evidence members are objects keyed by the fields of the evidence
classes below; status values are the strings of :class:`CandidateStatus`.
The evidence gates are the format's too: a record is dispatchable only as
``supported-win``, which needs exact-or-measured correctness without NaN/Inf
outputs and a median-over-median speedup of at least ``WIN_GATE`` (or a win
inside a fused model).

This module adds the ``"gpu"`` placement for records measured on this
library's HIP kernels.  ``"qpu"`` records describe VideoCore programs; they
load and save unchanged but nothing here executes them.

Structure: every class states its invariants as a table of (predicate,
message) rules checked at construction (``_enforce``), and one generic
decoder (``_decode``) turns JSON objects into the dataclasses, converting
lists to tuples for tuple-typed fields and nested objects to evidence.
"""

from __future__ import annotations

import json
from collections.abc import Callable, Mapping
from dataclasses import asdict, dataclass, fields
from enum import Enum
from os import PathLike
from statistics import median
from typing import Any

SCHEMA_VERSION = 3  # version written by save()
READABLE_SCHEMAS = frozenset({1, 2, 3})  # 1: no placement/kernels; 2: + partition; 3: + quality
PLACEMENTS = ("cpu", "qpu", "hybrid", "gpu")
WIN_GATE = 1.05  # minimum median baseline time / median candidate time
QUALITY_GATE = {"normalized_rmse": 0.10, "cosine_similarity": 0.99}

Rule = tuple[Callable[[Any], bool], str]


def _enforce(obj: Any, rules: tuple[Rule, ...]) -> None:
    for holds, message in rules:
        if not holds(obj):
            raise ValueError(f"{type(obj).__name__}: {message}")


def _all_at_least(values, bound: float) -> bool:
    return all(v >= bound for v in values)


class CandidateStatus(Enum):
    """Lifecycle state of a candidate; the values are the archive's strings."""

    SUPPORTED_WIN = "supported-win"
    SAME_CONTRACT_WIN = "same-contract-win"
    EXPERIMENTAL_CORRECT_SLOWER = "experimental-correct-slower"
    QUARANTINED_INCORRECT = "quarantined-incorrect"
    REFERENCE_ONLY = "reference-only"


# ---------------------------------------------------------------- evidence


@dataclass(frozen=True, slots=True)
class CorrectnessEvidence:
    """How a candidate's outputs compared with a named reference over ``cases`` inputs."""

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

    RULES = (
        (lambda e: bool(e.reference) and e.cases > 0, "needs a named reference and at least one compared case"),
        (lambda e: _all_at_least((e.max_abs_error, e.mean_abs_error, e.p99_abs_error, e.max_relative_error,
                                  e.saturation_count, e.nan_count, e.inf_count), 0),
         "error magnitudes and counts must be >= 0"),
    )

    def __post_init__(self) -> None:
        _enforce(self, self.RULES)

    @property
    def finite(self) -> bool:
        """No NaN or Inf output was observed."""
        return self.nan_count == 0 and self.inf_count == 0


@dataclass(frozen=True, slots=True)
class PerformanceEvidence:
    """Wall-time samples (seconds) of the fastest baseline and of the candidate, whole operation."""

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

    RULES = (
        (lambda p: bool(p.cpu_reference) and len(p.cpu_seconds) > 0 and len(p.candidate_seconds) > 0,
         "needs a baseline name plus baseline and candidate timings"),
        (lambda p: all(t > 0 for name in PerformanceEvidence.TIMINGS for t in getattr(p, name)),
         "every timing sample must be > 0 seconds"),
        (lambda p: bool(p.same_contract_reference) == bool(p.same_contract_seconds),
         "a same-contract baseline needs both its name and its timings"),
    )
    TIMINGS = ("cpu_seconds", "candidate_seconds", "host_prep_seconds", "kernel_seconds", "cold_start_seconds",
               "dequantization_seconds", "same_contract_seconds")

    def __post_init__(self) -> None:
        _enforce(self, self.RULES)

    @property
    def cpu_median_seconds(self) -> float:
        return float(median(self.cpu_seconds))

    @property
    def candidate_median_seconds(self) -> float:
        return float(median(self.candidate_seconds))

    @property
    def speedup(self) -> float:
        """Median baseline time over median candidate time."""
        return self.cpu_median_seconds / self.candidate_median_seconds

    @property
    def measured_win(self) -> bool:
        return self.fused_model_win or self.speedup >= WIN_GATE

    @property
    def same_contract_speedup(self) -> float | None:
        if not self.same_contract_seconds:
            return None
        return float(median(self.same_contract_seconds)) / self.candidate_median_seconds

    @property
    def same_contract_win(self) -> bool:
        ratio = self.same_contract_speedup
        return ratio is not None and ratio >= WIN_GATE


@dataclass(frozen=True, slots=True)
class PartitionEvidence:
    """Two-way split of one operator along ``axis`` (``"rows"`` or ``"outputs"``).

    ``qpu_units`` (the archive's name) is the size of the leading partition,
    run on the first queue; the trailing ``total_units - qpu_units`` run on
    the second.  Both are non-empty and the leading size is a multiple of
    ``alignment``.
    """

    axis: str
    qpu_units: int
    total_units: int
    alignment: int = 1

    RULES = (
        (lambda s: bool(s.axis) and s.total_units > 0 and s.alignment > 0,
         "needs an axis name and positive unit counts"),
        (lambda s: 0 < s.qpu_units < s.total_units, "both partitions must be non-empty (0 < leading < total)"),
        (lambda s: s.qpu_units % s.alignment == 0, "the leading partition must be a multiple of the alignment"),
    )

    def __post_init__(self) -> None:
        _enforce(self, self.RULES)

    @property
    def leading(self) -> int:
        return self.qpu_units

    @property
    def trailing(self) -> int:
        return self.total_units - self.qpu_units


@dataclass(frozen=True, slots=True)
class QualityEvidence:
    """Error of a quantised format against its fp32 source-domain result."""

    reference: str
    normalized_rmse: float
    cosine_similarity: float
    max_abs_error: float = 0.0
    mean_abs_error: float = 0.0
    p99_abs_error: float = 0.0
    nan_count: int = 0
    inf_count: int = 0
    top1_agreement: float | None = None

    RULES = (
        (lambda q: bool(q.reference) and _all_at_least(
            (q.normalized_rmse, q.max_abs_error, q.mean_abs_error, q.p99_abs_error), 0),
         "needs a reference and non-negative error figures"),
        (lambda q: -1.0 <= q.cosine_similarity <= 1.0, "cosine similarity lies in [-1, 1]"),
        (lambda q: q.nan_count >= 0 and q.inf_count >= 0, "NaN and Inf counts must be >= 0"),
        (lambda q: q.top1_agreement is None or 0.0 <= q.top1_agreement <= 1.0, "top-1 agreement lies in [0, 1]"),
    )

    def __post_init__(self) -> None:
        _enforce(self, self.RULES)

    @property
    def passes_default_gate(self) -> bool:
        return (self.normalized_rmse <= QUALITY_GATE["normalized_rmse"]
                and self.cosine_similarity >= QUALITY_GATE["cosine_similarity"]
                and self.nan_count == 0 and self.inf_count == 0)


# ------------------------------------------------------------------ records


def _dispatchable_evidence(record: "CandidateRecord", win: Callable[[PerformanceEvidence], bool]) -> bool:
    return record.correctness is not None and record.performance is not None and win(record.performance)


# What each status demands of a record's evidence, checked in order.
_STATUS_RULES: dict[CandidateStatus, tuple[Rule, ...]] = {
    CandidateStatus.SUPPORTED_WIN: (
        (lambda r: _dispatchable_evidence(r, lambda p: p.measured_win),
         f"supported-win needs correctness evidence and a measured win (>= {WIN_GATE}x or a fused-model win)"),
        (lambda r: r.correctness.finite, "a supported-win record must not have produced NaN or Inf"),
    ),
    CandidateStatus.SAME_CONTRACT_WIN: (
        (lambda r: _dispatchable_evidence(r, lambda p: p.same_contract_win),
         f"same-contract-win needs correctness evidence and >= {WIN_GATE}x over its same-contract baseline"),
        (lambda r: r.correctness.finite, "a same-contract-win record must not have produced NaN or Inf"),
    ),
    CandidateStatus.EXPERIMENTAL_CORRECT_SLOWER: (
        (lambda r: r.correctness is not None, "experimental-correct-slower needs correctness evidence"),
    ),
    CandidateStatus.QUARANTINED_INCORRECT: (
        (lambda r: bool(r.reason), "quarantined-incorrect needs a reason"),
    ),
    CandidateStatus.REFERENCE_ONLY: (),
}


@dataclass(frozen=True, slots=True)
class CandidateRecord:
    """One kernel specialisation for one exact (operation, dtype, layout, shape class), with its evidence."""

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
    placement: str = "qpu"  # archives of schema 1 carry no placement: VideoCore records
    kernels: tuple[str, ...] = ()
    partition: PartitionEvidence | None = None
    quality: QualityEvidence | None = None

    RULES = (
        (lambda r: all((r.name, r.operation, r.dtype, r.layout, r.shape_class, r.source_hash)),
         "identity fields (name, operation, dtype, layout, shape_class, source_hash) must all be set"),
        (lambda r: r.placement in PLACEMENTS, f"placement must be one of {', '.join(PLACEMENTS)}"),
        (lambda r: r.placement != "hybrid" or r.partition is not None, "a hybrid record needs partition evidence"),
        (lambda r: r.placement == "hybrid" or r.partition is None, "partition evidence belongs to hybrid records only"),
    )

    def __post_init__(self) -> None:
        _enforce(self, self.RULES)
        _enforce(self, _STATUS_RULES[self.status])

    @property
    def class_key(self) -> tuple[str, str, str, str]:
        """The exact operation class dispatch matches on."""
        return (self.operation, self.dtype, self.layout, self.shape_class)

    def to_json(self) -> dict[str, Any]:
        payload = asdict(self)
        payload["status"] = self.status.value
        return payload

    @classmethod
    def from_json(cls, raw: Any) -> "CandidateRecord":
        return _decode(cls, raw)


_NESTED = {"correctness": CorrectnessEvidence, "performance": PerformanceEvidence,
           "partition": PartitionEvidence, "quality": QualityEvidence}


def _decode(cls: type, raw: Any) -> Any:
    """Build ``cls`` from a JSON object: nested evidence, enum status, tuple-typed fields."""
    if not isinstance(raw, Mapping):
        raise ValueError(f"{cls.__name__} must be a JSON object")
    spec = {f.name: f for f in fields(cls)}
    unknown = sorted(set(raw) - set(spec))
    if unknown:
        raise ValueError(f"{cls.__name__} has unknown keys {unknown}")
    values = {}
    for key, value in raw.items():
        if key in _NESTED and cls is CandidateRecord:
            value = None if value is None else _decode(_NESTED[key], value)
        elif key == "status" and cls is CandidateRecord:
            value = CandidateStatus(value)
        elif str(spec[key].type).startswith("tuple") and isinstance(value, list):
            value = tuple(value)
        values[key] = value
    return cls(**values)


# ----------------------------------------------------------------- registry


class CandidateRegistry:
    """Uniquely named records in registration order; dispatch sees only ``supported-win`` ones."""

    def __init__(self, records: tuple[CandidateRecord, ...] = ()) -> None:
        self._records: dict[str, CandidateRecord] = {}
        for record in records:
            self.register(record)

    @property
    def records(self) -> tuple[CandidateRecord, ...]:
        return tuple(self._records.values())

    @property
    def supported(self) -> tuple[CandidateRecord, ...]:
        return tuple(r for r in self._records.values() if r.status is CandidateStatus.SUPPORTED_WIN)

    def supported_for(self, *, operation: str, dtype: str, layout: str, shape_class: str) -> tuple[CandidateRecord, ...]:
        """Dispatchable records of exactly this operation class."""
        key = (operation, dtype, layout, shape_class)
        return tuple(r for r in self.supported if r.class_key == key)

    def register(self, record: CandidateRecord) -> None:
        if record.name in self._records:
            raise ValueError(f"duplicate candidate name {record.name!r}")
        self._records[record.name] = record

    @classmethod
    def combine(cls, *registries: "CandidateRegistry") -> "CandidateRegistry":
        """One registry holding every record of ``registries`` (names must stay unique)."""
        return cls(tuple(r for registry in registries for r in registry.records))

    # ------------------------------------------------------------- archive

    def to_dict(self) -> dict[str, Any]:
        return {"schema_version": SCHEMA_VERSION, "records": [r.to_json() for r in self.records]}

    def save(self, path: str | PathLike[str]) -> None:
        """Write every record, slower and quarantined ones included."""
        with open(path, "w", encoding="utf-8") as out:
            json.dump(self.to_dict(), out, indent=2, sort_keys=True)

    @classmethod
    def from_dict(cls, payload: Any) -> "CandidateRegistry":
        if not isinstance(payload, Mapping) or payload.get("schema_version") not in READABLE_SCHEMAS:
            raise ValueError("candidate archive schema_version must be 1, 2 or 3")
        raw = payload.get("records")
        if not isinstance(raw, list):
            raise ValueError("candidate archive 'records' must be a JSON list")
        records = []
        for index, item in enumerate(raw):
            try:
                records.append(CandidateRecord.from_json(item))
            except (KeyError, TypeError, ValueError) as exc:
                raise ValueError(f"candidate archive record {index} is malformed: {exc}") from exc
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
