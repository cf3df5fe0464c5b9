"""l2domain_amd -- XCD-domain-aware GEMV, histogram, hash and BFS kernels for MI355X (gfx950).

Python host mirror of the C ABI in include/xdom.h. Device buffers are torch tensors on a
ROCm device (torch is used only for device memory and streams); every compute call goes
to libxdom.so. The library is loaded by the first module that needs it (l2domain_amd._lib)
and that import fails if the library is not built: there is no CPU fallback.
"""
MODE_OBLIVIOUS = 0
MODE_AWARE = 1
MODE_ROTATED = 2


def __getattr__(name):
    if name in ("lib", "XdomError", "MODES"):
        from . import _lib
        return getattr(_lib, name)
    raise AttributeError(name)
