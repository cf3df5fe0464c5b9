"""ctypes binding of libxdom.so (the C ABI declared in include/xdom.h).

The library is loaded from the package directory only. There is no fallback: if the
shared object is missing or does not export a declared symbol, import fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

# torch ships its own HIP and HSA runtime libraries. In a process that uses both, torch has
# to be loaded before libxdom.so (which links /opt/rocm's): loaded the other way round, the
# library's HIP calls report hipErrorNoDevice once torch has initialised the device.
try:
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - the library itself does not need torch
    pass

PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("XDOM_LIB", PKG / "libxdom.so"))

XD_OK = 0
XD_ERR_INVALID_ARG = -1
XD_ERR_HIP = -2
XD_ERR_WORKSPACE = -3
XD_ERR_UNSUPPORTED = -4
XD_ERR_TABLE_FULL = -5
XD_ERR_INCOMPLETE = -6

MODE_OBLIVIOUS = 0
MODE_AWARE = 1
MODE_ROTATED = 2
MODES = {"oblivious": MODE_OBLIVIOUS, "baseline": MODE_OBLIVIOUS, "aware": MODE_AWARE,
         "rotated": MODE_ROTATED, "swapped": MODE_ROTATED}

_ERR_NAMES = {XD_ERR_INVALID_ARG: "XD_ERR_INVALID_ARG", XD_ERR_HIP: "XD_ERR_HIP",
              XD_ERR_WORKSPACE: "XD_ERR_WORKSPACE", XD_ERR_UNSUPPORTED: "XD_ERR_UNSUPPORTED",
              XD_ERR_TABLE_FULL: "XD_ERR_TABLE_FULL", XD_ERR_INCOMPLETE: "XD_ERR_INCOMPLETE"}


class XdomError(RuntimeError):
    def __init__(self, code: int, fn: str, msg: str):
        super().__init__(f"{fn} failed with {_ERR_NAMES.get(code, code)}: {msg}")
        self.code = code


class BfsStats(C.Structure):
    _fields_ = [("levels", C.c_int32), ("topdown_steps", C.c_int32), ("bottomup_steps", C.c_int32),
                ("reached_vertices", C.c_int64), ("reached_edges", C.c_int64)]


class Topology(C.Structure):
    _fields_ = [("device", C.c_int), ("num_cu", C.c_int), ("num_xcd", C.c_int),
                ("cu_per_xcd", C.c_int), ("wave_size", C.c_int), ("clock_khz", C.c_int),
                ("l2_bytes", C.c_longlong), ("lds_bytes_per_wg", C.c_longlong),
                ("hbm_bytes", C.c_longlong), ("arch", C.c_char * 32), ("name", C.c_char * 96)]


VP = C.c_void_p
SZ = C.c_size_t
I = C.c_int
U32 = C.c_uint32
U64 = C.c_uint64
I64 = C.c_int64
D = C.c_double

# name -> (restype, argtypes). Kept in the order of include/xdom.h.
SIGNATURES: dict[str, tuple] = {
    "xd_version": (C.c_char_p, []),
    "xd_last_error": (C.c_char_p, []),
    "xd_timing_enable": (I, [I]),
    "xd_timing_query": (I, [I, C.c_char_p, I, C.POINTER(D), C.POINTER(C.c_longlong)]),
    "xd_topology_query": (I, [I, C.POINTER(Topology)]),
    "xd_domain_scan": (I, [I, VP, VP]),
    "xd_xcd_offset": (I, [VP]),
    "xd_home_mask": (U64, []),
    "xd_set_home_mask": (I, [U64]),
    "xd_home_map_pages": (SZ, [VP, SZ]),
    "xd_home_map_workspace_size": (SZ, [VP, SZ]),
    "xd_home_map": (I, [VP, SZ, VP, VP, SZ, VP]),
    "xd_cache_flush_bytes": (SZ, []),
    "xd_cache_flush": (I, [VP, SZ, VP]),
    "xd_read_stream": (I, [VP, SZ, I, VP, I, I, VP]),
    "xd_xdom_pchase": (I, [I, I, VP, SZ, I, I, VP, SZ, VP, VP]),
    "xd_mask_probe": (I, [VP, SZ, I, I, I, VP, VP]),
    "xd_domain_scan_latency": (I, [VP, SZ, I, I, I, C.c_uint32, VP, SZ, VP, VP]),
    "xd_memchannel_time": (I, [VP, SZ, C.POINTER(C.c_uint64), I, C.POINTER(C.c_float), VP]),
    "xd_memchannel_probe": (I, [VP, SZ, I, I, I, I, C.POINTER(C.c_float), C.POINTER(C.c_uint64),
                                C.POINTER(C.c_uint64), C.POINTER(C.c_int), VP]),
    "xd_channel_time": (I, [VP, SZ, I, C.POINTER(C.c_uint64), I, C.POINTER(C.c_float), VP]),
    "xd_channel_probe": (I, [VP, SZ, I, I, I, I, I, C.POINTER(C.c_float), C.POINTER(C.c_float),
                             C.POINTER(C.c_uint64), C.POINTER(C.c_float), C.POINTER(C.c_int), VP]),
    "xd_gemv_workspace_size": (SZ, [I, I, I]),
    "xd_gemv_f32": (I, [VP, VP, VP, I, I, I, VP, VP, SZ, VP]),
    "xd_gemv_f16f32": (I, [VP, VP, VP, I, I, I, VP, VP, SZ, VP]),
    "xd_hist_workspace_size": (SZ, [SZ, U32]),
    "xd_hist_u32": (I, [VP, SZ, VP, U32, I, VP, VP, SZ, VP]),
    "xd_hist256_workspace_size": (SZ, []),
    "xd_hist256_u32bytes": (I, [VP, SZ, VP, I, VP, VP, SZ, VP]),
    "xd_hist256_u32bytes_noalloc": (I, [VP, SZ, VP, I, VP, VP]),
    "xd_hash_table_bytes": (SZ, [U64]),
    "xd_hash_init": (I, [VP, U64, VP]),
    "xd_hash_insert_u64": (I, [VP, U64, VP, VP, U64, I, VP, VP, VP]),
    "xd_hash_lookup_u64": (I, [VP, U64, VP, U64, VP, VP, I, VP, VP]),
    "xd_hash_build_workspace_size": (SZ, [U64, U64]),
    "xd_hash_build_u64": (I, [VP, U64, VP, VP, U64, I, VP, VP, SZ, VP, VP]),
    "xd_gen_hash_kv": (I, [VP, VP, U64, U64, VP]),
    "xd_gen_hash_queries": (I, [VP, U64, U64, U64, U64, VP]),
    "xd_dep_make_keys": (I, [U64, U64, VP, C.c_int32, C.c_int32, VP, VP]),
    "xd_dep_build": (I, [VP, U64, VP, VP, C.c_int32, U64]),
    "xd_dep_queries": (I, [VP, C.c_int32, VP, C.c_int32, C.c_int32, C.c_int32, U64]),
    "xd_dep_probe": (I, [VP, U64, VP, U64, I, VP, I, VP, VP]),
    "xd_dep_route_bytes": (SZ, [U64]),
    "xd_dep_route": (I, [VP, U64, VP, U64, VP, VP, SZ, VP]),
    "xd_dep_probe_routed": (I, [VP, U64, VP, U64, I, VP, I, VP]),
    "xd_bfs_workspace_size": (SZ, [C.c_int32, I64]),
    "xd_bfs_route_bytes": (SZ, [C.c_int32]),
    "xd_bfs_route": (I, [VP, VP, C.c_int32, I64, VP, VP, SZ, VP]),
    "xd_bfs_csr": (I, [VP, VP, C.c_int32, I64, C.c_int32, VP, I, VP, VP, SZ, VP, C.POINTER(BfsStats)]),
    "xd_bfs_ref_graph": (I, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, U64, U64, VP, U64, VP, VP, VP, VP,
                             VP]),
    "xd_bfs_multi_workspace_size": (SZ, [C.c_int32]),
    "xd_bfs_multi": (I, [VP, VP, C.c_int32, I64, VP, C.c_int32, C.c_int32, VP, VP, I, VP, SZ, VP]),
    "xd_rand64": (U64, [U64, U64]),
    "xd_gen_uniform_f32": (I, [VP, SZ, U64]),
    "xd_gen_normal_f16": (I, [VP, SZ, D, D, U64]),
    "xd_gen_mix32_words": (I, [VP, SZ, U32]),
    "xd_gen_mix32_f32": (I, [VP, SZ, U32, U32, C.c_int32]),
    "xd_zipf_thresholds": (I, [VP, U32, D]),
    "xd_gen_zipf_keys": (I, [VP, SZ, VP, U32, U64, I, VP]),
    "xd_rmat_edge": (I, [I, D, D, D, U64, U64, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "xd_rmat_csr": (I, [I, I, D, D, D, U64, VP, VP, I64, C.POINTER(I64)]),
}


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"libxdom.so not found at {LIB_PATH}; build it first with `python -m l2domain_amd.build` "
            "(there is no CPU fallback for the XCD-domain kernels)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError here means the .so is stale
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(code: int, fn: str) -> None:
    if code != XD_OK:
        raise XdomError(code, fn, lib.xd_last_error().decode(errors="replace"))


def call(name: str, *args):
    """Calls an int-returning entry point and raises XdomError on a non-zero status."""
    rc = getattr(lib, name)(*args)
    check(rc, name)
    return rc


def timing_enable(on: bool = True) -> None:
    call("xd_timing_enable", 1 if on else 0)


def timing_read() -> dict:
    """{kernel name: (total_ms, launches)} for the library's launches since timing_enable()."""
    out = {}
    i = 0
    buf = C.create_string_buffer(128)
    while True:
        ms = C.c_double()
        n = C.c_longlong()
        if lib.xd_timing_query(i, buf, 128, C.byref(ms), C.byref(n)) != XD_OK:
            break
        out[buf.value.decode()] = (ms.value, n.value)
        i += 1
    return out
