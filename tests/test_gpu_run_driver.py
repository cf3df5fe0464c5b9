"""The preset driver on the GPU: every application's quick preset (the reference's smoke
point) runs end to end through the runners and writes its CSV with every case PASS, plus a
metadata file with the device's ROCm fields."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]
CSVS = {"gemv": "final_gemv_MI355X.csv", "histogram": "histogram_mi355x_quick.csv", "hash": "hash_mi355x_quick.csv",
        "bfs": "bfs_mi355x_quick.csv"}


@pytest.mark.parametrize("app", ["gemv", "histogram", "hash", "bfs"])
def test_quick_preset(tmp_path, app):
    print("driver:", app, flush=True)
    r = subprocess.run([sys.executable, "-m", "l2domain_amd.run", app, "--preset", "quick", "--device", "0",
                        "--output-dir", str(tmp_path)], capture_output=True, text=True, cwd=ROOT, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    rows = (tmp_path / CSVS[app]).read_text().splitlines()
    assert len(rows) == 2
    header, row = rows[0].split(","), rows[1].split(",")
    assert row[header.index("pass")] == "PASS"
    md = json.loads((tmp_path / "metadata.json").read_text())
    assert md["application"] == app and md["preset"] == "quick" and md["gpu"]["arch"] == "gfx950"
    assert md["rocm_version"] and md["hipcc_version"]


def test_architecture_figure_2(tmp_path):
    r = subprocess.run([sys.executable, "-m", "l2domain_amd.run", "architecture", "--figure", "2", "--device", "0",
                        "--output-dir", str(tmp_path)], capture_output=True, text=True, cwd=ROOT, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    rows = (tmp_path / "data" / "figure_02.csv").read_text().splitlines()
    assert rows[0].startswith("device_index,device_name,leader_sm,follower_sm,index,offset_bytes") and len(rows) == 2049
    assert json.loads((tmp_path / "metadata" / "figure_02.json").read_text())["figure"] == "02"


def test_architecture_figures_3_and_4(tmp_path):
    """Figure 3: the reference's DomainScan schema, one curve of 25 bits per compute unit;
    figure 4: MaskProbe rows plus the L2 channel functions and the memory-side unit classes."""
    for fig in ("3", "4"):
        r = subprocess.run([sys.executable, "-m", "l2domain_amd.run", "architecture", "--figure", fig, "--device", "0",
                            "--output-dir", str(tmp_path)], capture_output=True, text=True, cwd=ROOT, timeout=600)
        assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    rows = (tmp_path / "data" / "figure_03.csv").read_text().splitlines()
    assert rows[0] == ("device_index,device_name,leader_sm,tpc_id,resource_id,tpc_sm0,tpc_sm1,follower_sm,"
                       "address_bit,latency_cycles")
    assert len(rows) == 1 + 256 * 25
    chan = (tmp_path / "data" / "figure_04_channels.csv").read_text().splitlines()
    assert chan[0].startswith("device_index,device_name,xcd,function,mask,address_bit")
    assert len(chan) == 1 + 9 + 4 * 14   # 9 windows over bits 7..20, 4 functions of 14 bits
    mem = (tmp_path / "data" / "figure_04_memchannels.csv").read_text().splitlines()
    assert mem[0].startswith("device_index,device_name,bit_a,bit_b,min_slowdown") and len(mem) == 1 + 14 * 15 // 2
