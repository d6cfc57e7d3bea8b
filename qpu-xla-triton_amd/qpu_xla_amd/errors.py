"""Exception hierarchy; names and meanings follow the reference's
``src/qpu_xla/errors.py`` so callers catch the same types."""


class QpuXlaError(Exception):
    """Base class for all failures of this library."""


class DeviceClosedError(QpuXlaError):
    """Work was submitted to a queue that is closed."""


class AllocationError(QpuXlaError):
    """A buffer allocation or layout is invalid."""


class DependencyError(QpuXlaError):
    """An event dependency, queue binding or device pairing cannot be accepted."""


class EventTimeoutError(QpuXlaError):
    """Waiting for an event exceeded its timeout."""


class EventCancelledError(QpuXlaError):
    """The awaited event was cancelled before it ran."""


class KernelError(QpuXlaError):
    """A kernel cannot be launched or failed during execution."""
