"""Placement values for operator dispatch.

The reference defines ``Placement{AUTO, CPU, QPU, HYBRID}``
(``src/qpu_xla/scheduler/placement.py:14-20``).  This library adds ``GPU``,
the MI355X placement, next to them; the other values keep their strings so
candidate records stay comparable.
"""

from __future__ import annotations

from enum import Enum


class Placement(Enum):
    """A requested or selected whole-operator execution strategy."""

    AUTO = "auto"
    CPU = "cpu"
    QPU = "qpu"
    HYBRID = "hybrid"
    GPU = "gpu"
