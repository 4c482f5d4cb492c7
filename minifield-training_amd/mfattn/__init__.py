"""mfattn: MI355X-native packed-sequence attention.

``mfattn.kernels.attention`` and ``mfattn.kernels.bidirectional`` mirror the
reference's kernel modules; ``mfattn.ops`` is the tensor-level C-ABI binding.
Importing the package loads ``libmfattn.so`` and raises ``ImportError`` if it
is missing (build with ``python minifield-training_amd/mfattn/build.py``).
"""

from . import _lib, ops
from .kernels import attention, bidirectional

__all__ = ["attention", "bidirectional", "ops"]
__version__ = _lib.version()
