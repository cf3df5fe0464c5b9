"""The preset driver (python -m l2domain_amd.run) on the CPU: option checks, dry runs of
every application's presets (the reference's case lists), the stdout parsers against
canned runner output in the reference's line formats, and the ROCm metadata file."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

from l2domain_amd import run as drv

ROOT = Path(__file__).resolve().parents[1]


def call(*args):
    r = subprocess.run([sys.executable, "-m", "l2domain_amd.run", *args], capture_output=True, text=True, cwd=ROOT,
                       timeout=300)
    return r.returncode, r.stdout, r.stderr


@pytest.mark.parametrize("bad", [["gemv", "--preset", "huge"], ["bfs", "--arch", "sm_90a"],
                                 ["architecture", "--figure", "5"], ["architecture", "--peer", "0,9"],
                                 ["hash", "--wait-timeout", "-1"], ["histogram", "--output-dir", ""]])
def test_option_errors_exit_2(bad):
    rc, out, err = call(*bad)
    assert rc == 2, out + err


def test_unknown_application():
    rc, out, err = call("relu")
    assert rc == 2


@pytest.mark.parametrize("app,preset,expect", [
    ("gemv", "quick", ["xd_gemv_run 2048 5 4242 1", "xd_gemv_vendor_run 2048 1024 5 1 1"]),
    ("gemv", "paper", ["xd_gemv_run 10240 50 4242 1", "xd_gemv_vendor_run 3072 1024 20 5 1"]),
    ("histogram", "quick", ["xd_hist_run 32 1 128 1 0"]),
    ("histogram", "paper", ["xd_hist_run 512 10 128 1 0"]),
    ("hash", "quick", ["xd_hash_run 1048576 524288 2097152 4 80 16384 1"]),
    ("hash", "paper", ["xd_hash_run 32000000 8000000 67108864 16 80 100000 7",
                       "xd_hash_run 32000000 8000000 33554432 4 80 100000 7"]),
    ("bfs", "quick", ["xd_bfs_run 65536 8 128 2 95 4096 1 8201"]),
    ("bfs", "paper", ["xd_bfs_run 2000000 128 4096 4 95 200000 5 8201", "xd_bfs_run 2000000 64 16384 4 95 200000 5 8201",
                      "xd_bfs_run 2000000 64 4096 8 95 200000 5 8201"]),
    ("architecture", "quick", ["xd_arch_probe pchase 0 4 2048 128", "xd_arch_probe domainscan 4096"]),
])
def test_dry_run_prints_the_reference_cases(tmp_path, app, preset, expect):
    out_dir = tmp_path / "o"
    rc, out, err = call(app, "--preset", preset, "--dry-run", "--output-dir", str(out_dir))
    assert rc == 0, out + err
    for e in expect:
        assert e in out, (e, out)
    assert "dry-run: would write metadata" in out
    assert not out_dir.exists()  # a dry run writes nothing


def test_paper_case_counts():
    assert len(drv.gemv_cases("paper")["M"]) == 9
    assert len(drv.hash_cases("paper")[1]) == 7
    assert [c[0] for c in drv.bfs_cases("paper")].count("degree") == 4 and len(drv.bfs_cases("paper")) == 8


class FakeRun:
    """Stands in for the runner executables with canned stdout in their formats."""

    def __init__(self, outputs):
        self.outputs = outputs
        self.ctx = type("Ctx", (), {"index": 0})()
        self.calls = []

    def __call__(self, name, *args, log=None):
        self.calls.append((name, args))
        return self.outputs[name]


def _args(**kw):
    import argparse
    d = dict(preset="quick", dry_run=False, figure=2, peer="auto")
    d.update(kw)
    return argparse.Namespace(**d)


def test_gemv_csv_rules(tmp_path):
    ours = ("baseline_ms 0.010000 ms 1.0 GFLOP/s\naware_ms 0.008000 ms aware_speedup=1.250x 2.0 GFLOP/s\n"
            "swapped_ms 0.020000 ms swapped_speedup=0.500x 1.0 GFLOP/s\n"
            "correctness max_abs_error baseline=1e-06 aware=2e-06 swapped=5e-07\n"
            "gbps baseline=1000.0 aware=1250.0 swapped=500.0\nroofline=hbm roofline_frac=0.1562 peak_gbps=8000\n"
            "cpu_ms=1.500 cpu_threads=1\n")
    fake = FakeRun({"xd_gemv_run": (0, ours), "xd_gemv_vendor_run": (0, "cublas_ms 0.012000 ms 3.0 GFLOP/s\n")})
    assert drv.run_gemv(_args(), fake, tmp_path) == 0
    rows = (tmp_path / "final_gemv_MI355X.csv").read_text().splitlines()
    assert rows[0].startswith("M,K,lanes_per_row,warps_per_block,baseline_ms,aware_ms,swapped_ms,cublas_ms,"
                              "max_abs_error,aware_speedup,swapped_speedup,aware_vs_cublas,pass")
    f = rows[1].split(",")
    assert f[:8] == ["2048", "1024", "64", "4", "0.010000", "0.008000", "0.020000", "0.012000"]
    assert float(f[8]) == 2e-06 and float(f[9]) == pytest.approx(1.25) and float(f[11]) == pytest.approx(1.5)
    assert f[12] == "PASS" and f[13] == "1250.0" and f[15] == "hbm"
    # the reference's pass rule: max error above 1e-3 fails the case
    fake.outputs["xd_gemv_run"] = (0, ours.replace("aware=2e-06", "aware=0.002"))
    assert drv.run_gemv(_args(), fake, tmp_path) == 1


def test_histogram_hash_bfs_csv_rules(tmp_path):
    hist = ("data=32MB words=8388608 runs=1 threads=128 blocks_per_sm=1 cache_mode=cold baseline_blocks=512 "
            "persistent_blocks=512 side_blocks[256,256]\n"
            "correct baseline=PASS green_aware=PASS green_swapped=PASS persistent_aware=PASS persistent_swapped=PASS\n"
            "baseline_kernel_ms 0.020000 ms\ngreen_aware_kernel_ms 0.010000 ms kernel_speedup_vs_baseline=2.000x\n"
            "green_swapped_kernel_ms 0.040000 ms kernel_speedup_vs_baseline=0.500x\n"
            "persistent_aware_kernel_ms 0.010000 ms kernel_speedup_vs_baseline=2.000x\n"
            "persistent_swapped_kernel_ms 0.040000 ms kernel_speedup_vs_baseline=0.500x\n")
    fake = FakeRun({"xd_hist_run": (0, hist)})
    assert drv.run_histogram(_args(), fake, tmp_path) == 0
    f = (tmp_path / "histogram_mi355x_quick.csv").read_text().splitlines()[1].split(",")
    assert f[5:7] == ["512", "512"] and f[9] == "0.020000" and f[14] == "2.000000" and f[18] == "PASS"
    fake.outputs["xd_hist_run"] = (0, hist.replace("green_swapped=PASS", "green_swapped=FAIL"))
    assert drv.run_histogram(_args(), fake, tmp_path) == 1

    res = ("RESULT baseline_ms=1.000000 aware_ms=0.800000 swapped_ms=2.000000 aware_speedup=1.250000 "
           "swapped_speedup=0.500000 pass=PASS\n")
    fake = FakeRun({"xd_hash_run": (0, res)})
    assert drv.run_hash(_args(), fake, tmp_path) == 0
    f = (tmp_path / "hash_mi355x_quick.csv").read_text().splitlines()[1].split(",")
    assert f[3] == "50.000000" and f[7:13] == ["1.000000", "0.800000", "2.000000", "1.250000", "0.500000", "PASS"]

    bfs = ("visited=1000 aware_bad=0 swapped_bad=0 overflow=0 groups=4/4 baseline_bad=0\n"
           "| mode | median_ms | speedup_vs_baseline |\n|---|---:|---:|\n| baseline | 2.000000 | 1.000000 |\n"
           "| aware | 1.000000 | 2.000000 |\n| swapped | 4.000000 | 0.500000 |\n")
    fake = FakeRun({"xd_bfs_run": (0, bfs)})
    assert drv.run_bfs(_args(), fake, tmp_path) == 0
    f = (tmp_path / "bfs_mi355x_quick.csv").read_text().splitlines()[1].split(",")
    assert f[:2] == ["quick", "default"] and f[12:16] == ["1000", "0", "0", "0"]
    assert f[16:22] == ["2.000000", "1.000000", "4.000000", "2.000000", "0.500000", "PASS"]
    fake.outputs["xd_bfs_run"] = (0, bfs.replace("aware_bad=0", "aware_bad=3"))
    assert drv.run_bfs(_args(), fake, tmp_path) == 1


def test_metadata_has_rocm_fields(tmp_path):
    import argparse
    a = argparse.Namespace(dry_run=False, device="0", arch="auto", wait_timeout=5, poll_interval=1)
    ctx = drv.GpuContext(a)
    p = tmp_path / "metadata.json"
    ctx.write_metadata(p, "python -m l2domain_amd.run gemv", application="gemv", preset="quick")
    md = json.loads(p.read_text())
    for key in ("timestamp_utc", "command", "cwd", "repo_root", "git_commit", "git_dirty", "rocm_version",
                "hipcc_version", "amdgpu_driver_version", "gpu", "idle_check", "application", "preset"):
        assert key in md
    assert md["gpu"]["arch"] == "gfx950" and md["gpu"]["physical_index"] == 0
    assert md["idle_check"]["lock_held"] is True and md["application"] == "gemv"
