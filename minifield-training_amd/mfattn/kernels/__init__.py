"""Drop-in kernels with the reference's call signatures (HIP underneath)."""

from . import attention, bidirectional

__all__ = ["attention", "bidirectional"]
