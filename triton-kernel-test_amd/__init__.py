"""MI355X-native compressed-activation kernels (encode / decode / fused backward).

Import with ``importlib.import_module("triton-kernel-test_amd")`` (the directory name is
not a Python identifier).  The HIP library liblrq.so must be built first; nothing here
falls back to a CPU implementation.
"""

from . import _lib, api, autograd, inputs, offload  # noqa: F401
from .api import *  # noqa: F401,F403
from .legacy import *  # noqa: F401,F403

__version__ = "0.1.0"
