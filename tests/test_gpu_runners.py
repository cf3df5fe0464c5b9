"""Runner executables on the GPU: small cases, stdout parsed with the field rules of the
reference's run.sh scripts (applications/gemv/run.sh:66-97,
applications/histogram/run.sh:72-84, applications/hash/run.sh:62-86,
applications/bfs/run.sh:84-92), exit status 0 and PASS everywhere."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
BIN = Path(__file__).resolve().parents[1] / "l2domain_amd" / "bin"


def run(name, *args, csv=None):
    cmd = [str(BIN / name), *map(str, args)]
    if csv:
        cmd.append(f"--csv={csv}")
    print("runner:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    return r.returncode, r.stdout, r.stderr


def first_field(out, key):
    # awk '$1 == key {print $2; exit}'
    for line in out.splitlines():
        f = line.split()
        if f and f[0] == key:
            return f[1]
    return None


@pytest.mark.parametrize("K,dtype", [(1024, "f32"), (4096, "f32"), (4096, "f16"), (14336, "f16")])
def test_gemv_runner(tmp_path, K, dtype):
    rc, out, err = run("xd_gemv_run", 1024, 5, 4242, 1, K, dtype, csv=tmp_path / "g.csv")
    assert rc == 0, out + err
    for key in ("baseline_ms", "aware_ms", "swapped_ms"):
        assert float(first_field(out, key)) > 0
    line = next(l for l in out.splitlines() if l.startswith("correctness max_abs_error"))
    errs = [float(t.split("=")[1]) for t in line.split() if "=" in t]
    assert len(errs) == 3
    if dtype == "f32":
        assert max(errs) <= 1e-3  # applications/gemv/run.sh:94-97
    rows = (tmp_path / "g.csv").read_text().splitlines()
    assert rows[0].startswith("M,K,lanes_per_row,warps_per_block,baseline_ms,aware_ms,swapped_ms,cublas_ms")
    assert rows[1].split(",")[12] == "PASS"


@pytest.mark.parametrize("init", ["mix32", "mix32int"])
def test_gemv_runner_reference_inputs(init):
    """The reference's own inputs (init_data) at its K = 1024 with M = 2048 (the quick preset)."""
    rc, out, err = run("xd_gemv_run", 2048, 5, 4242, 1, 1024, "f32", init)
    assert rc == 0, out + err
    line = next(l for l in out.splitlines() if l.startswith("correctness max_abs_error"))
    errs = [float(t.split("=")[1]) for t in line.split() if "=" in t]
    assert max(errs) <= 1e-3
    if init == "mix32int":
        assert max(errs) == 0.0  # integer-valued inputs: every summation order is exact


@pytest.mark.parametrize("inputs,shape", [("mix32", (2048, 1024)), ("f32", (4096, 4096)), ("f16", (14336, 4096)),
                                          ("f16", (4096, 14336))])
def test_gemv_vendor_runner(inputs, shape):
    """rocBLAS sgemv on the reference's inputs and on the fp32 configuration, and its
    mixed-precision gemv (fp16 in, fp32 accumulate and out) on both fp16 shapes; the runner
    checks the result itself (exit 3 on a mismatch)."""
    rc, out, err = run("xd_gemv_vendor_run", *shape, 5, 1, 1, inputs)
    assert rc == 0, out + err
    assert float(first_field(out, "cublas_ms")) > 0 and "vendor=rocblas" in out
    assert f"inputs={inputs}" in out


@pytest.mark.parametrize("args", [("--workload=zipf", 16, 2, 256, 1, 0, 1 << 20, 1.1, 1373), (32, 2, 128, 1, 0)])
def test_hist_runner(tmp_path, args):
    """(32, 2, 128, 1, 0): the reference's quick preset (data_mb 32, THREADS=128, BLOCKS_PER_SM=1,
    CACHE_MODE=0) on its own byte-histogram workload."""
    rc, out, err = run("xd_hist_run", *args, csv=tmp_path / "h.csv")
    assert rc == 0, out + err
    line = next(l for l in out.splitlines() if l.startswith("correct "))
    assert line.split()[1:] == ["baseline=PASS", "green_aware=PASS", "green_swapped=PASS", "persistent_aware=PASS",
                                "persistent_swapped=PASS"]
    for key in ("baseline_kernel_ms", "persistent_aware_kernel_ms", "persistent_swapped_kernel_ms"):
        assert float(first_field(out, key)) > 0
    assert "baseline_blocks=" in out and "persistent_blocks=" in out
    assert (tmp_path / "h.csv").read_text().splitlines()[1].split(",")[18] == "PASS"


@pytest.mark.parametrize("workload", ["dep", "insert_lookup"])
def test_hash_runner(tmp_path, workload):
    args = [1 << 20, 1 << 20, 1 << 21, 4, 80, 10000, 2]
    if workload == "insert_lookup":
        args = ["--workload=insert_lookup", 1 << 20, 1 << 20, 1 << 21, 1, 50, 0, 2]
    rc, out, err = run("xd_hash_run", *args, csv=tmp_path / "x.csv")
    assert rc == 0, out + err
    assert "Correctness: PASS" in out
    res = next(l for l in out.splitlines() if l.startswith("RESULT "))
    kv = dict(t.split("=") for t in res.split()[1:])  # applications/hash/run.sh:62-66
    assert kv["pass"] == "PASS"
    for key in ("baseline_ms", "aware_ms", "swapped_ms", "aware_speedup", "swapped_speedup"):
        assert float(kv[key]) > 0
    assert (tmp_path / "x.csv").read_text().splitlines()[0].startswith("K,Q,C,effective_load,L,h,H,baseline_ms")
    if workload == "insert_lookup":  # the bulk build checked and timed beside the insert
        assert "Build correctness: PASS" in out
        assert float(first_field(out, "build_ms").split("=")[1]) > 0


@pytest.mark.parametrize("args", [(65536, 8, 128, 2, 95, 4096, 1, 8201),  # the reference's quick preset
                                  ("--workload=rmat", 1 << 16, 32, 2, 0, 100, 0, 2, 8201)])
def test_bfs_runner(tmp_path, args):
    rc, out, err = run("xd_bfs_run", *args, csv=tmp_path / "b.csv")
    assert rc == 0, out + err
    line = next(l for l in out.splitlines() if l.startswith("visited="))
    f = line.replace("=", " ").split()  # awk -F'[ =]' ... $2, $4, $6, $8
    visited, aware_bad, swapped_bad, overflow = int(f[1]), int(f[3]), int(f[5]), int(f[7])
    assert visited > 1 and aware_bad == 0 and swapped_bad == 0 and overflow == 0
    rows = {l.split("|")[1].strip(): l.split("|")[2].strip() for l in out.splitlines() if l.startswith("| ")
            and not l.startswith("| mode")}
    assert float(rows["baseline"]) > 0 and float(rows["aware"]) > 0 and float(rows["swapped"]) > 0
    assert (tmp_path / "b.csv").read_text().splitlines()[1].split(",")[21] == "PASS"


def test_arch_probe_runner(tmp_path):
    rc, out, err = run("xd_arch_probe", "domainscan", 4096, csv=tmp_path / "d.csv")
    assert rc == 0 and "round_robin_matches=4096" in out, out + err
    rc, out, err = run("xd_arch_probe", "pchase", 0, 4, 2048, 128, csv=tmp_path / "p.csv")
    assert rc == 0, out + err
    rows = (tmp_path / "p.csv").read_text().splitlines()
    assert rows[0].startswith("device_index,device_name,leader_sm,follower_sm,index,offset_bytes") and len(rows) == 2049
    rc, out, err = run("xd_arch_probe", "maskprobe", 5, 29, 8, csv=tmp_path / "m.csv")
    assert rc == 0 and "active_mask=0x2000" in out, out + err
