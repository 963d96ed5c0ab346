"""Exception types of the reference API (exceptions.py:1-6)."""


class KernelError(RuntimeError):
    """Base error for kernel dispatch failures."""


class KernelNotAvailableError(KernelError):
    """Raised when metadata exists but the compiled kernel cannot be launched."""
