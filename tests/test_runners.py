"""Runner executables (CPU side): they are built, print their usage, and reject bad
arguments before touching the GPU. The GPU runs are in test_gpu_runners.py."""
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parents[1] / "l2domain_amd" / "bin"
RUNNERS = ["xd_gemv_run", "xd_gemv_vendor_run", "xd_hist_run", "xd_hash_run", "xd_bfs_run", "xd_arch_probe"]


@pytest.mark.parametrize("name", RUNNERS)
def test_runner_usage(name):
    exe = BIN / name
    assert exe.exists(), f"{exe} not built"
    r = subprocess.run([str(exe), "--help"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0
    assert "usage" in (r.stdout + r.stderr).lower()


def test_hash_runner_argc_rule():
    # the reference accepts no arguments or all seven (hash_probe_dep.cu:119-122)
    r = subprocess.run([str(BIN / "xd_hash_run"), "1", "2", "3"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "Usage" in r.stderr


def test_runner_argument_checks():
    r = subprocess.run([str(BIN / "xd_gemv_run"), "1024", "1", "1", "0", "6", "f32"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 2
    r = subprocess.run([str(BIN / "xd_hist_run"), "--workload=zipf", "1", "1", "256", "1", "1", str(1 << 25)],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    r = subprocess.run([str(BIN / "xd_hist_run"), "--workload=other"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    r = subprocess.run([str(BIN / "xd_hist_run"), "4096"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2  # 4096 MiB of words would overflow the u32 byte counts


def test_bfs_runner_rejects_unknown_workload():
    r = subprocess.run([str(BIN / "xd_bfs_run"), "--workload=grid"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
