"""tessera_amd: gfx950 kernels for tessera's matmul and attention hot path.

``abi`` binds libtessera_hip.so (the C ABI in include/tessera_hip.h); ``rules``
launches each kernel on torch device tensors under the reference rule names.
"""
from . import abi  # noqa: F401

__all__ = ["abi"]
