"""Kernel handles and launch grids.

Mirrors the reference's ``src/qpu_xla/kernel.py:12-38``: a ``Kernel`` is a
name plus an executor ``(stream, args, grid) -> None``; any exception other
than ``KernelError`` raised by the executor is wrapped in ``KernelError``.
The executor receives the HIP stream the owning queue submits on.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from typing import Any

from qpu_xla_amd.errors import KernelError

Executor = Callable[[Any, tuple[Any, ...], tuple[int, int, int]], None]


@dataclass(frozen=True, slots=True)
class LaunchConfig:
    """A three-dimensional launch grid for one kernel invocation."""

    grid: tuple[int, int, int] = (1, 1, 1)

    def __post_init__(self) -> None:
        if len(self.grid) != 3 or any(int(dim) <= 0 for dim in self.grid):
            raise KernelError("kernel grid must contain three positive dimensions")


@dataclass(frozen=True, slots=True)
class Kernel:
    """A named kernel with an explicit execution adapter."""

    name: str
    executor: Executor

    def execute(self, stream: Any, args: tuple[Any, ...], launch: LaunchConfig) -> None:
        try:
            self.executor(stream, args, launch.grid)
        except KernelError:
            raise
        except BaseException as exc:  # noqa: BLE001 - mirrors the reference's wrapping contract
            raise KernelError(f"kernel {self.name!r} failed") from exc
