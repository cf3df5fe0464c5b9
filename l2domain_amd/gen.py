"""Seeded input generators (host side, in libxdom). Fully specified: see include/xdom.h."""
from __future__ import annotations

import numpy as np

from . import _lib

SEED_GEMV_F32 = 4242      # applications/gemv/run.sh:80 passes seed 4242
SEED_GEMV_F16_W = 4243
SEED_GEMV_F16_X = 4244
X_SEED_OFFSET = 0x9E37    # x uses seed + 0x9e37, as init_data does (GEMV.cu:129)


def rand64(seed: int, index: int) -> int:
    return int(_lib.lib.xd_rand64(seed, index))


def uniform_f32(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _lib.call("xd_gen_uniform_f32", out.ctypes.data, n, seed)
    return out


def normal_f16(n: int, mean: float, stddev: float, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    _lib.call("xd_gen_normal_f16", out.ctypes.data, n, mean, stddev, seed)
    return out.view(np.float16)


def mix32_words(n: int, seed: int = 0) -> np.ndarray:
    """The reference histogram's data: words[i] = mix32(i ^ seed) (seed 0 there)."""
    out = np.empty(n, dtype=np.uint32)
    _lib.call("xd_gen_mix32_words", out.ctypes.data if n else None, n, seed)
    return out


def mix32_f32(n: int, seed: int, modulus: int = 0, offset: int = 0) -> np.ndarray:
    """The reference GEMV's init_data values: (h & 0xff)/255 - 0.5, or h % modulus - offset."""
    out = np.empty(n, dtype=np.float32)
    _lib.call("xd_gen_mix32_f32", out.ctypes.data if n else None, n, seed, modulus, offset)
    return out


def gemv_mix32_inputs(M: int, K: int, seed: int = SEED_GEMV_F32, integer: bool = False):
    """A[M,K], x[K] exactly as the reference's init_data draws them (GEMV.cu:118-139)."""
    if integer:
        return (mix32_f32(M * K, seed, 17, 8).reshape(M, K),
                mix32_f32(K, (seed + X_SEED_OFFSET) & 0xFFFFFFFF, 7, 3))
    return mix32_f32(M * K, seed).reshape(M, K), mix32_f32(K, (seed + X_SEED_OFFSET) & 0xFFFFFFFF)


def zipf_thresholds(num_bins: int, s: float = 1.1) -> np.ndarray:
    out = np.empty(num_bins, dtype=np.uint64)
    _lib.call("xd_zipf_thresholds", out.ctypes.data, num_bins, s)
    return out


def zipf_keys_device(n: int, num_bins: int, seed: int, s: float = 1.1, scramble: bool = True,
                     thresholds=None, out=None):
    """Draws n Zipf(s) keys on the current device (torch int32 tensor holding u32 keys)."""
    import torch
    from ._torch import stream_handle
    t = thresholds if thresholds is not None else torch.from_numpy(zipf_thresholds(num_bins, s).view(np.int64)).cuda()
    keys = out if out is not None else torch.empty(n, dtype=torch.int32, device="cuda")
    _lib.call("xd_gen_zipf_keys", keys.data_ptr() if n else None, n, t.data_ptr(), num_bins, seed,
              1 if scramble else 0, stream_handle())
    return keys


def gemv_f32_inputs(M: int, K: int, seed: int = SEED_GEMV_F32):
    """A[M,K], x[K]: U[-1,1) on a 2^-23 grid (configs[0] of the build)."""
    return uniform_f32(M * K, seed).reshape(M, K), uniform_f32(K, seed + X_SEED_OFFSET)


def gemv_f16_inputs(M: int, K: int, w_seed: int = SEED_GEMV_F16_W, x_seed: int = SEED_GEMV_F16_X):
    """W[M,K] ~ N(0, 0.02), x[K] ~ N(0, 1), both rounded to binary16."""
    return normal_f16(M * K, 0.0, 0.02, w_seed).reshape(M, K), normal_f16(K, 0.0, 1.0, x_seed)
