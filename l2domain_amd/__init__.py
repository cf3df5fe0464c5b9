"""l2domain_amd -- XCD-domain-aware GEMV, histogram, hash and BFS kernels for MI355X (gfx950).

Python host mirror of the C ABI in include/xdom.h. Device buffers are torch tensors on a
ROCm device (torch is used only for device memory and streams); every compute call goes
to libxdom.so, and importing this package fails if that library is not built.
"""
from ._lib import (MODE_AWARE, MODE_OBLIVIOUS, MODE_ROTATED, MODES, XdomError, lib)  # noqa: F401

__all__ = ["MODE_AWARE", "MODE_OBLIVIOUS", "MODE_ROTATED", "MODES", "XdomError", "lib"]
