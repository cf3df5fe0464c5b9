"""The C-ABI library loads, exports every entry point include/xdom.h declares, and rejects
bad arguments with an error code before touching the GPU (runs on CPU)."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "xdom.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xd_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "xd_gemv_f32" in names and "xd_topology_query" in names
    assert len(names) >= 10


def test_library_exports_every_declared_symbol():
    from l2domain_amd import _lib
    lib_path = _lib.LIB_PATH
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], capture_output=True, text=True,
                         check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_python_binding_covers_header():
    from l2domain_amd import _lib
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_version_and_error_string():
    from l2domain_amd import _lib
    assert _lib.lib.xd_version().startswith(b"xdom")


@pytest.mark.parametrize("M,K,mode", [(0, 4, 1), (4, 3, 1), (4, 4, 7), (-1, 4, 0)])
def test_gemv_rejects_bad_shapes(M, K, mode):
    from l2domain_amd import _lib
    buf = (C.c_float * 64)()
    p = C.cast(buf, C.c_void_p)
    rc = _lib.lib.xd_gemv_f32(p, p, p, M, K, mode, None, None, 0, None)
    assert rc == _lib.XD_ERR_INVALID_ARG
    assert _lib.lib.xd_last_error()


def test_gemv_rejects_null_and_misaligned():
    from l2domain_amd import _lib
    buf = (C.c_float * 64)()
    p = C.addressof(buf)
    assert _lib.lib.xd_gemv_f32(None, p, p, 4, 4, 1, None, None, 0, None) == _lib.XD_ERR_INVALID_ARG
    assert _lib.lib.xd_gemv_f16f32(p + 2, p, p, 4, 8, 1, None, None, 0, None) == _lib.XD_ERR_INVALID_ARG
    assert _lib.lib.xd_gemv_f16f32(p, p, p, 4, 12, 1, None, None, 0, None) == _lib.XD_ERR_INVALID_ARG


def test_gemv_rejects_k_beyond_lds():
    from l2domain_amd import _lib
    buf = (C.c_float * 64)()
    p = C.addressof(buf)
    assert _lib.lib.xd_gemv_f32(p, p, p, 4, 4 * 4097 * 4, 1, None, None, 0, None) == _lib.XD_ERR_UNSUPPORTED


def test_probes_reject_bad_arguments():
    """The channel probe and the DomainScan latency curves validate before any HIP call."""
    from l2domain_amd import _lib
    p = 1 << 21  # a 2 MiB-aligned stand-in address: never dereferenced on these paths
    us = C.c_float(0.0)
    vecs = (C.c_uint64 * 6)(*([128] * 6))
    bad = (C.c_uint64 * 6)(*([128] * 5 + [100]))  # not a multiple of 128
    E = _lib.XD_ERR_INVALID_ARG
    assert _lib.lib.xd_channel_time(p, 1 << 22, 0, None, 256, C.byref(us), None) == E
    assert _lib.lib.xd_channel_time(p, 1 << 22, 0, bad, 256, C.byref(us), None) == E
    assert _lib.lib.xd_channel_time(p, 1 << 22, 8, vecs, 256, C.byref(us), None) == E     # no XCD 8
    assert _lib.lib.xd_channel_time(p, 1 << 22, 0, vecs, 6, C.byref(us), None) == E       # iters % 4
    assert _lib.lib.xd_channel_time(p, 64, 0, vecs, 256, C.byref(us), None) == E          # span > bytes
    win = (C.c_float * 16)()
    fast = C.c_float(0.0)
    masks = (C.c_uint64 * 4)()
    curves = (C.c_float * 64)()
    nm = C.c_int(0)
    args = (win, C.byref(fast), masks, curves, C.byref(nm), None)
    assert _lib.lib.xd_channel_probe(p, 1 << 23, 0, 6, 20, 256, 64, *args) == E           # bit0 < 7
    assert _lib.lib.xd_channel_probe(p, 1 << 23, 0, 7, 12, 256, 64, *args) == E           # fewer than 7 bits
    assert _lib.lib.xd_channel_probe(p, 1 << 23, 0, 7, 20, 256, 0, *args) == E            # max_sets
    assert _lib.lib.xd_channel_probe(p, 1 << 20, 0, 7, 20, 256, 64, *args) == E           # buffer too small
    out = (C.c_uint32 * 32)()
    assert _lib.lib.xd_domain_scan_latency(p, 1 << 10, 7, 31, 0, 0, None, 0, out, None) == E  # 2^31 > bytes
    assert _lib.lib.xd_domain_scan_latency(p, 1 << 20, 9, 8, 0, 0, None, 0, out, None) == E   # empty range
    assert _lib.lib.xd_domain_scan_latency(p, 1 << 20, 7, 19, 8, 0, None, 0, out, None) == E  # leader XCD 8
    assert _lib.lib.xd_domain_scan_latency(p, 1 << 20, 7, 19, 0, 9 << 16, None, 0, out, None) == E  # XCD 9
    assert _lib.lib.xd_domain_scan_latency(p + 4, 1 << 20, 7, 19, 0, 0, None, 0, out, None) == E    # alignment
    ratio = (C.c_float * 196)()
    inactive = C.c_uint64(0)
    assert _lib.lib.xd_memchannel_time(p, 1 << 22, None, 64, C.byref(us), None) == E
    assert _lib.lib.xd_memchannel_time(p, 1 << 22, bad, 64, C.byref(us), None) == E
    assert _lib.lib.xd_memchannel_time(p, 1 << 22, vecs, 0, C.byref(us), None) == E          # iters
    assert _lib.lib.xd_memchannel_time(p, 64, vecs, 64, C.byref(us), None) == E              # span > bytes
    margs = (ratio, C.byref(inactive), masks, C.byref(nm), None)
    assert _lib.lib.xd_memchannel_probe(p, 1 << 23, 6, 20, 64, 6, *margs) == E              # bit0 < 7
    assert _lib.lib.xd_memchannel_probe(p, 1 << 23, 7, 20, 64, 0, *margs) == E              # nsets
    assert _lib.lib.xd_memchannel_probe(p, 1 << 20, 7, 20, 64, 6, *margs) == E              # too small


def test_hash_build_workspace_and_argument_checks():
    """The build's workspace query: 0 where the call clears and inserts (no pairs, tables
    outside 2^15 .. 2^30 slots, fewer than slots / 64 pairs), about 3.3 x 16 n bytes at load
    factor 0.5, at most 7 x 16 n bytes, and growing with n; bad arguments are refused before
    any HIP call."""
    from l2domain_amd import _lib
    lib = _lib.lib
    assert lib.xd_hash_build_workspace_size(0, 1 << 27) == 0
    assert lib.xd_hash_build_workspace_size(1500, 1 << 12) == 0
    assert lib.xd_hash_build_workspace_size(1 << 20, 1 << 31) == 0
    big = lib.xd_hash_build_workspace_size(1 << 26, 1 << 27)
    assert 3.0 * 16 * (1 << 26) < big < 3.4 * 16 * (1 << 26)
    assert lib.xd_hash_build_workspace_size(1, 1 << 30) == 0  # (the ranges' floor no longer sizes it)
    assert lib.xd_hash_build_workspace_size((1 << 14) - 1, 1 << 20) == 0
    ns = (1 << 14, 100000, 500000)
    sizes = [lib.xd_hash_build_workspace_size(n, 1 << 20) for n in ns]
    assert all(a < b for a, b in zip(sizes, sizes[1:])) and sizes[0] > 0
    for n, slots in [(n, 1 << 20) for n in ns] + [(1 << 24, 1 << 30), (1 << 26, 1 << 27)]:
        assert lib.xd_hash_build_workspace_size(n, slots) <= 7 * 16 * n, (n, slots)
    ws = (C.c_uint8 * 64)()
    fake = C.c_void_p(4096)  # never dereferenced: every call below fails its checks first
    keys = C.c_void_p(8192)
    n = 2000  # >= slots / 64: the bulk path, whose workspace checks come before any HIP call
    cases = [
        (None, 1 << 16, keys, keys, n, 0, None, ws, 64),      # NULL table
        (fake, 3 << 15, keys, keys, n, 0, None, ws, 64),      # slots not a power of two
        (fake, 1 << 16, None, keys, n, 0, None, ws, 64),      # NULL keys
        (fake, 1 << 16, keys, keys, n, 7, None, ws, 64),      # bad mode
        (fake, 1 << 16, C.c_void_p(8196), keys, n, 0, None, ws, 64),  # keys not 8-byte aligned
        (fake, 1 << 16, keys, keys, n, 0, None, ws, 64),      # workspace smaller than the query
        (fake, 1 << 16, keys, keys, n, 0, None, None, 0),     # no workspace
    ]
    assert lib.xd_hash_build_workspace_size(n, 1 << 16) > 64
    for table, slots, k, v, n, mode, home, w, wb in cases:
        rc = lib.xd_hash_build_u64(table, slots, k, v, n, mode, home, w, wb, None, None)
        assert rc in (_lib.XD_ERR_INVALID_ARG, _lib.XD_ERR_WORKSPACE), (slots, n, mode, rc)
