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
