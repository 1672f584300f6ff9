"""MI355X (gfx950) kernel nodes for the qwen36_layer / qwen36_lmhead8 bundle slots.

The compute lives in libq36.so (hand-written HIP, C-ABI in include/q36_abi.h); the Python
modules under qwen36_layer/ and qwen36_lmhead8/ mirror the reference bundle's operator
interface and only pass device pointers across that boundary.
"""
from ._lib import lib  # noqa: F401  (loading the library is the import-time check)

__all__ = ["lib"]
