"""Resource guard for the built gfx950 kernels (CPU only: reads the code objects that
`build()` embedded in the library's objects, through the ROCm LLVM tools).

Two workgroups of 1024 threads share a CU only while a wave holds at most 80 scalar
registers in all: the histogram's routed partition at 82 ran with half its workgroups
resident although the compiler still reported 8 waves per SIMD. Every 1024-thread kernel
whose LDS and vector registers would allow two workgroups per CU must stay within that, and
no kernel may spill to scratch memory."""
import shutil
import subprocess
from pathlib import Path

import pytest
import yaml

ROOT = Path(__file__).resolve().parent.parent
BUILD = ROOT / "l2domain_amd" / "_build"
LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
MAX_SGPRS_TWO_WORKGROUPS = 80
LDS_PER_CU = 160 * 1024


def _tools_ok() -> bool:
    return all((LLVM / t).exists() for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf"))


def kernels_of(obj: Path, tmp: Path) -> list[dict]:
    """The AMDGPU metadata of every kernel in one host object's embedded gfx950 code object."""
    fat, dev = tmp / (obj.name + ".fatbin"), tmp / (obj.name + ".gfx950.o")
    subprocess.run([str(LLVM / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", str(obj), str(tmp / "copy.o")],
                   check=True, capture_output=True)
    subprocess.run([str(LLVM / "clang-offload-bundler"), "--type=o", f"--targets={TARGET}", f"--input={fat}",
                    f"--output={dev}", "--unbundle"], check=True, capture_output=True)
    notes = subprocess.run([str(LLVM / "llvm-readelf"), "--notes", str(dev)], check=True, capture_output=True,
                           text=True).stdout
    text = notes[notes.index("---"):]
    text = text[: text.index("\n...") + 4] if "\n..." in text else text
    return yaml.safe_load(text)["amdhsa.kernels"]


@pytest.fixture(scope="module")
def all_kernels(tmp_path_factory):
    if not _tools_ok():
        pytest.skip("ROCm LLVM tools not found")
    objs = sorted(BUILD.glob("*.hip.o"))
    if not objs:
        pytest.skip("library not built (run __graft_entry__.build())")
    tmp = tmp_path_factory.mktemp("codeobj")
    out = []
    for o in objs:
        for k in kernels_of(o, tmp):
            out.append((o.name, k))
    return out


def test_every_object_holds_kernels(all_kernels):
    files = {f for f, _ in all_kernels}
    assert {"xd_hist.hip.o", "xd_gemv.hip.o", "xd_hash.hip.o", "xd_hash_build.hip.o", "xd_bfs.hip.o"} <= files
    names = " ".join(k[".name"] for _, k in all_kernels)
    assert "hist_partition_packed_kernel" in names and "hist_hot_kernel" in names


def test_no_scratch_spills(all_kernels):
    spilled = [(f, k[".name"], k[".private_segment_fixed_size"]) for f, k in all_kernels
               if k.get(".private_segment_fixed_size", 0) != 0]
    assert not spilled, spilled


def test_two_workgroup_kernels_within_the_scalar_register_limit(all_kernels):
    checked, over = 0, []
    for f, k in all_kernels:
        if k[".max_flat_workgroup_size"] != 1024:
            continue
        if 2 * k[".group_segment_fixed_size"] > LDS_PER_CU or k[".vgpr_count"] > 64:
            continue  # one workgroup per CU anyway
        checked += 1
        if k[".sgpr_count"] > MAX_SGPRS_TWO_WORKGROUPS:
            over.append((f, k[".name"], k[".sgpr_count"]))
    assert checked >= 4  # the histogram partition kinds at least
    assert not over, over
