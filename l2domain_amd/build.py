"""Builds libxdom.so (HIP, gfx950) and the per-application runner executables in-tree.

Usage:  python -m l2domain_amd.build [--jobs N]

Every .hip file under csrc/ is compiled by hipcc for gfx950 only; host-only .cpp files
by g++. The shared library lands at l2domain_amd/libxdom.so, runners in
l2domain_amd/bin/. Objects go to l2domain_amd/_build/ (ignored by git).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
RUNNERS = PKG / "runners"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB = PKG / "libxdom.so"
BIN = PKG / "bin"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Wno-unused-command-line-argument",
    # Packed FP32 (v_pk_*_f32) is disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]
CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-pthread", f"-I{INCLUDE}", f"-I{CSRC}"]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature; keep real diagnostics.
    err = "\n".join(l for l in res.stderr.splitlines()
                    if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{err}")
    if err.strip() and os.environ.get("XD_BUILD_VERBOSE"):
        print(err, file=sys.stderr)


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [CXX, *CXX_FLAGS, "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def build_library(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", str(tmp),
          *map(str, objs), "-Wl,-soname,libxdom.so"])
    os.replace(tmp, LIB)
    return LIB


def build_runners(jobs: int = 8) -> list[Path]:
    srcs = sorted(RUNNERS.glob("*.cpp"))
    if not srcs:
        return []
    BIN.mkdir(exist_ok=True)

    # the vendor-library comparison runner also links rocBLAS (timed for comparison only)
    extra_libs = {"xd_gemv_vendor_run": ["-L/opt/rocm/lib", "-lrocblas"]}

    def one(src: Path) -> Path:
        exe = BIN / src.stem
        _run([HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-pthread", f"-I{INCLUDE}", f"-I{RUNNERS}", str(src),
              "-o", str(exe), f"-L{PKG}", "-lxdom", *extra_libs.get(src.stem, []), f"-Wl,-rpath,$ORIGIN/.."])
        return exe

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        return list(ex.map(one, srcs))


def build_oracle() -> None:
    """The CPU oracle is test infrastructure; it is built beside the product, never linked."""
    oracle = ROOT / "oracle"
    if (oracle / "Makefile").exists() and shutil.which("make"):
        _run(["make", "-s", "-C", str(oracle)])


def build_all(jobs: int = 8) -> None:
    build_library(jobs)
    build_runners(jobs)
    build_oracle()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    args = ap.parse_args()
    build_all(args.jobs)
    print(f"built {LIB}")


if __name__ == "__main__":
    main()
