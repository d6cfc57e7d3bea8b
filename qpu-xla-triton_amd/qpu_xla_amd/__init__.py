"""MI355X (gfx950) placement of qpu_xla's quantized-linear hot path.

Python host layer over ``libqxt_gfx950.so`` (hand-written HIP kernels behind a
C ABI, ``include/qxt_gfx950.h``).  Tensors are torch tensors on the HIP
device; there is no CPU fallback anywhere in this package.
"""

from qpu_xla_amd import _lib  # noqa: F401
from qpu_xla_amd.errors import (  # noqa: F401
    AllocationError,
    DependencyError,
    DeviceClosedError,
    EventCancelledError,
    EventTimeoutError,
    KernelError,
    QpuXlaError,
)
from qpu_xla_amd.kernel import Kernel, LaunchConfig  # noqa: F401
from qpu_xla_amd.placement import Placement  # noqa: F401
from qpu_xla_amd.queue import Event, EventStatus, Queue  # noqa: F401

__all__ = [
    "AllocationError",
    "DependencyError",
    "DeviceClosedError",
    "Event",
    "EventCancelledError",
    "EventStatus",
    "EventTimeoutError",
    "Kernel",
    "KernelError",
    "LaunchConfig",
    "Placement",
    "QpuXlaError",
    "Queue",
]
