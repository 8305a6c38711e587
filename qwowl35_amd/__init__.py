"""qwowl35_amd — MI355X-native (gfx950) quantized matvec/matmul engine for the
Qwen3.5-9B projection path of EmilioSchi/qwowl35.

The product is ``libqw35_hip.so`` (hand-written HIP kernels + the C ABI in
``include/qw35_hip.h``).  ``runtime`` is the Python mirror of the reference's
per-op encoder API over that ABI; ``build`` compiles the library in-tree.
"""
from ._ffi import Qw35Error, load  # noqa: F401

__all__ = ["Qw35Error", "load"]
