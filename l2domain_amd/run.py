"""Preset driver: the reference's per-application run.sh layer on MI355X.

    python -m l2domain_amd.run APP [--preset quick|paper] [--device auto|INDEX|UUID]
                               [--build-only] [--dry-run] [--arch auto|gfx950]
                               [--wait-timeout SEC] [--poll-interval SEC] [--output-dir PATH]
                               [--figure 2|3|4] [--peer A,B]

APP is gemv, histogram, hash, bfs (applications/*/run.sh) or architecture (the probe
figures of architecture/run_figure_0N.sh). Options, presets, case lists, CSV file names,
CSV headers and the pass rules follow the reference (scripts/app_runner.sh:15-141,
applications/{gemv,histogram,hash,bfs}/run.sh, scripts/common.sh:183-305,
scripts/_support.py:247-285); each CSV gains this build's columns after the reference's.
The runners are the executables in l2domain_amd/bin (built by l2domain_amd.build); the
driver parses their stdout the way the reference's awk rules parse its binaries'.

ROCm stands in for CUDA in the metadata: the ROCm and hipcc versions, the amdgpu driver
version, and the GPU's name, gfx architecture, unique id, memory use and utilisation as
rocm-smi reports them (nvidia-smi / nvcc in the reference). The GPU is held with an
exclusive lock file while the cases run, and selected through HIP_VISIBLE_DEVICES.
"""
from __future__ import annotations

import argparse
import datetime as dt
import fcntl
import json
import os
import re
import shlex
import shutil
import subprocess
import sys
import time
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
BIN = PKG / "bin"
APPS = ("gemv", "histogram", "hash", "bfs", "architecture")
GPU_LABEL = "mi355x"        # the reference's a100 / h100 / b200 / custom (app_runner.sh:118-123)
GPU_CSV_NAME = "MI355X"     # applications/gemv/run.sh:22-28
IDLE_MAX_MEMORY_MIB = 1024  # idle thresholds in the spirit of common.sh's idle check
IDLE_MAX_UTIL = 10
IDLE_SAMPLES = 3


class UsageError(Exception):
    pass


# ---------------------------------------------------------------------------------------
# Presets and cases (the reference's run.sh case lists)
# ---------------------------------------------------------------------------------------
def gemv_cases(preset):
    # applications/gemv/run.sh:15-19: M values, our runs, cuBLAS runs, warm-ups
    if preset == "quick":
        return {"M": [2048], "runs": 5, "vendor_runs": 5, "warmups": 1}
    return {"M": [2048, 3072, 4096, 5120, 6144, 7168, 8192, 9216, 10240], "runs": 50, "vendor_runs": 20,
            "warmups": 5}


def histogram_cases(preset):
    # applications/histogram/run.sh:15-22
    data_mbs = [32] if preset == "quick" else [32, 64, 128, 512]
    return {"data_mb": data_mbs, "runs": 1 if preset == "quick" else 10, "threads": 128, "blocks_per_sm": 1,
            "cache_mode": 0}


def hash_cases(preset):
    # applications/hash/run.sh:15-45 (Table 8: default plus one-factor variations)
    runs = 1 if preset == "quick" else 7
    if preset == "quick":
        return runs, [(1048576, 524288, 2097152, 4, 80, 16384)]
    return runs, [(32000000, 8000000, 67108864, 1, 80, 100000), (32000000, 8000000, 67108864, 2, 80, 100000),
                  (32000000, 8000000, 67108864, 4, 80, 100000), (32000000, 8000000, 67108864, 16, 80, 100000),
                  (32000000, 8000000, 33554432, 4, 80, 100000), (32000000, 8000000, 67108864, 4, 70, 100000),
                  (32000000, 8000000, 67108864, 4, 99, 100000)]


def bfs_cases(preset):
    # applications/bfs/run.sh:15-63 (Table 10 sweeps)
    if preset == "quick":
        p = dict(vertices=65536, degree=8, sources=128, depth=2, dst_local=95, hot=4096, runs=1, seed=8201)
        return [("quick", "default", p)]
    p = dict(vertices=2000000, degree=64, sources=4096, depth=4, dst_local=95, hot=200000, runs=5, seed=8201)
    cases = [("degree", str(d), dict(p, degree=d)) for d in (16, 32, 64, 128)]
    cases += [("sources", str(s), dict(p, sources=s)) for s in (512, 16384)]
    cases += [("depth", str(d), dict(p, depth=d)) for d in (2, 8)]
    return cases


# ---------------------------------------------------------------------------------------
# stdout parsing (the reference's awk rules)
# ---------------------------------------------------------------------------------------
def first_field(text, key):
    """awk '$1 == key {print $2; exit}'"""
    for line in text.splitlines():
        f = line.split()
        if f and f[0] == key:
            return f[1] if len(f) > 1 else ""
    return ""


def kv_tokens(text, prefix):
    """key=value tokens of the first line starting with `prefix`."""
    for line in text.splitlines():
        if line.startswith(prefix):
            return dict(t.split("=", 1) for t in line.split() if "=" in t)
    return {}


def fnum(x):
    try:
        return float(x)
    except (TypeError, ValueError):
        return None


def ratio(a, b, fmt="%.9f"):
    a, b = fnum(a), fnum(b)
    return fmt % (a / b) if a is not None and b else ""


# ---------------------------------------------------------------------------------------
# GPU context: selection, lock, idle check, metadata
# ---------------------------------------------------------------------------------------
def _cmd_out(cmd, timeout=30):
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
        return r.returncode, r.stdout
    except (OSError, subprocess.TimeoutExpired):
        return 1, ""


def smi_query(index):
    """rocm-smi view of one GPU (empty fields where the tool or a field is unavailable)."""
    info = {"name": "", "uuid": "", "memory_used_mib": "", "util_percent": "", "driver_version": ""}
    smi = shutil.which("rocm-smi") or ("/opt/rocm/bin/rocm-smi" if Path("/opt/rocm/bin/rocm-smi").exists() else None)
    if smi:
        rc, out = _cmd_out([smi, "-d", str(index), "--showproductname", "--showuniqueid", "--showmemuse",
                            "--showuse", "--showmeminfo", "vram", "--json"])
        if rc == 0 and out.strip():
            try:
                card = next(iter(json.loads(out).values()))
            except (ValueError, StopIteration, AttributeError):
                card = {}
            for k, v in card.items():
                kl = k.lower()
                if "card series" in kl or ("product name" in kl and not info["name"]):
                    info["name"] = str(v)
                elif "unique id" in kl:
                    info["uuid"] = str(v)
                elif "gpu use" in kl:
                    info["util_percent"] = str(v)
                elif "vram total used memory" in kl:
                    try:
                        info["memory_used_mib"] = str(int(v) // (1024 * 1024))
                    except ValueError:
                        pass
        rc, out = _cmd_out([smi, "--showdriverversion", "--json"])
        if rc == 0:
            m = re.search(r'"Driver version":\s*"([^"]+)"', out)
            if m:
                info["driver_version"] = m.group(1)
    if not info["driver_version"] and Path("/sys/module/amdgpu/version").exists():
        info["driver_version"] = Path("/sys/module/amdgpu/version").read_text().strip()
    return info


def rocm_versions():
    rocm = ""
    for p in ("/opt/rocm/.info/version", "/opt/rocm/.info/version-dev"):
        if Path(p).exists():
            rocm = Path(p).read_text().strip()
            break
    rc, out = _cmd_out([os.environ.get("HIPCC", "/opt/rocm/bin/hipcc"), "--version"])
    return rocm, out.strip() if rc == 0 else ""


def git_metadata(root):
    rc, commit = _cmd_out(["git", "-C", str(root), "rev-parse", "HEAD"])
    if rc != 0:
        return "", None
    rc, status = _cmd_out(["git", "-C", str(root), "status", "--porcelain"])
    return commit.strip(), (bool(status.strip()) if rc == 0 else None)


def resolve_device(selector):
    """auto -> the first GPU that looks idle (else 0); INDEX; or a unique id."""
    if selector == "auto":
        for i in range(8):
            q = smi_query(i)
            if not q["name"] and not q["uuid"] and i > 0:
                break
            mem, util = fnum(q["memory_used_mib"]), fnum(q["util_percent"])
            if (mem is None or mem <= IDLE_MAX_MEMORY_MIB) and (util is None or util <= IDLE_MAX_UTIL):
                return i
        return 0
    if re.fullmatch(r"\d+", selector):
        return int(selector)
    for i in range(64):
        q = smi_query(i)
        if not q["uuid"] and not q["name"]:
            break
        if q["uuid"].lower() == selector.lower():
            return i
    raise UsageError(f"no GPU with unique id {selector}")


class GpuContext:
    """Selects the device, holds an exclusive lock on it and records the idle check."""

    def __init__(self, args):
        self.dry = args.dry_run
        self.index = None
        self.lock = None
        self.idle = {}
        self.info = {}
        self.arch = "gfx950" if args.arch == "auto" else args.arch
        if self.dry:
            self.index = args.device if args.device != "auto" else "<auto-selected-physical-index>"
            return
        self.index = resolve_device(args.device)
        self.lock_path = Path(f"/tmp/l2domain-amd-gpu-{self.index}.lock")
        deadline = time.monotonic() + args.wait_timeout
        self.lock = open(self.lock_path, "w")
        while True:
            try:
                fcntl.flock(self.lock, fcntl.LOCK_EX | fcntl.LOCK_NB)
                break
            except OSError:
                if time.monotonic() >= deadline:
                    raise UsageError(f"GPU {self.index} stayed locked for {args.wait_timeout} s ({self.lock_path})")
                time.sleep(max(args.poll_interval, 1))
        samples = []
        for _ in range(IDLE_SAMPLES):
            samples.append(smi_query(self.index))
            time.sleep(0.2)
        self.info = samples[-1]
        mems = [fnum(s["memory_used_mib"]) for s in samples if fnum(s["memory_used_mib"]) is not None]
        utils = [fnum(s["util_percent"]) for s in samples if fnum(s["util_percent"]) is not None]
        self.idle = {"samples": IDLE_SAMPLES, "max_memory_threshold_mib": IDLE_MAX_MEMORY_MIB,
                     "max_util_threshold_percent": IDLE_MAX_UTIL,
                     "max_memory_used_mib": int(max(mems)) if mems else None,
                     "max_util_percent": int(max(utils)) if utils else None,
                     "lock_path": str(self.lock_path), "lock_held": True}

    def env(self):
        e = dict(os.environ)
        if not self.dry:
            e["HIP_VISIBLE_DEVICES"] = str(self.index)
        return e

    def write_metadata(self, path: Path, command: str, **extra):
        if self.dry:
            print(f"dry-run: would write metadata to {path}")
            return
        commit, dirty = git_metadata(ROOT)
        rocm, hipcc = rocm_versions()
        md = {
            "timestamp_utc": dt.datetime.now(dt.timezone.utc).isoformat(),
            "command": command,
            "cwd": os.getcwd(),
            "repo_root": str(ROOT),
            "git_commit": commit,
            "git_dirty": dirty,
            "rocm_version": rocm,
            "hipcc_version": hipcc,
            "amdgpu_driver_version": self.info.get("driver_version", ""),
            "gpu": {"physical_index": self.index, "uuid": self.info.get("uuid", ""),
                    "name": self.info.get("name", ""), "arch": self.arch,
                    "memory_used_mib": self.info.get("memory_used_mib", ""),
                    "max_util_percent": self.info.get("util_percent", "")},
            "idle_check": self.idle,
        }
        md.update({k: str(v) for k, v in extra.items()})
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(json.dumps(md, indent=2, sort_keys=True) + "\n", encoding="utf-8")


# ---------------------------------------------------------------------------------------
# Running the runners
# ---------------------------------------------------------------------------------------
class Runner:
    def __init__(self, ctx: GpuContext, dry: bool):
        self.ctx, self.dry = ctx, dry

    def __call__(self, name, *args, log: Path | None = None):
        cmd = [str(BIN / name), *map(str, args)]
        print("+ " + " ".join(shlex.quote(c) for c in cmd), flush=True)
        if self.dry:
            return 0, ""
        r = subprocess.run(cmd, capture_output=True, text=True, env=self.ctx.env())
        out = r.stdout + r.stderr
        sys.stdout.write(out)
        sys.stdout.flush()
        if log is not None:
            log.write_text(out)
        return r.returncode, out


def run_gemv(args, run, out_dir: Path):
    c = gemv_cases(args.preset)
    if args.dry_run:
        for m in c["M"]:
            run("xd_gemv_run", m, c["runs"], 4242, 1)
            run("xd_gemv_vendor_run", m, 1024, c["vendor_runs"], c["warmups"], 1)
        return 0
    csv = out_dir / f"final_gemv_{GPU_CSV_NAME}.csv"
    header = ("M,K,lanes_per_row,warps_per_block,baseline_ms,aware_ms,swapped_ms,cublas_ms,max_abs_error,"
              "aware_speedup,swapped_speedup,aware_vs_cublas,pass,aware_gbps,roofline_frac,roofline,cpu_ms")
    rows, failures = [header], 0
    for m in c["M"]:
        print(f"===== M={m} K=1024 =====", flush=True)
        st, ours = run("xd_gemv_run", m, c["runs"], 4242, 1)
        cst, vend = run("xd_gemv_vendor_run", m, 1024, c["vendor_runs"], c["warmups"], 1)
        base, aware, swap = (first_field(ours, k) for k in ("baseline_ms", "aware_ms", "swapped_ms"))
        vms = first_field(vend, "cublas_ms")
        errs = [fnum(v) for v in kv_tokens(ours, "correctness max_abs_error").values()]
        err = max([e for e in errs if e is not None], default=None)
        ok = (st == 0 and cst == 0 and all((fnum(x) or 0) > 0 for x in (base, aware, swap, vms))
              and err is not None and err <= 0.001)  # applications/gemv/run.sh:94-97
        g, rl = kv_tokens(ours, "gbps "), kv_tokens(ours, "roofline=")
        rows.append(",".join([str(m), "1024", "64", "4", base, aware, swap, vms, "" if err is None else repr(err),
                              ratio(base, aware), ratio(base, swap), ratio(vms, aware), "PASS" if ok else "FAIL",
                              g.get("aware", ""), rl.get("roofline_frac", ""), rl.get("roofline", ""),
                              kv_tokens(ours, "cpu_ms=").get("cpu_ms", "")]))
        failures += 0 if ok else 1
    csv.write_text("\n".join(rows) + "\n")
    print(f"CSV: {csv}")
    return failures


def run_histogram(args, run, out_dir: Path):
    c = histogram_cases(args.preset)
    argv = lambda mb: (mb, c["runs"], c["threads"], c["blocks_per_sm"], c["cache_mode"])  # noqa: E731
    if args.dry_run:
        for mb in c["data_mb"]:
            run("xd_hist_run", *argv(mb))
        return 0
    csv = out_dir / f"histogram_{GPU_LABEL}_{args.preset}.csv"
    header = ("gpu_label,gpu_index,data_mb,threads,blocks_per_sm,total_blocks,persistent_blocks,runs,cache_mode,"
              "baseline_kernel_ms,green_aware_kernel_ms,green_swapped_kernel_ms,persistent_aware_kernel_ms,"
              "persistent_swapped_kernel_ms,green_aware_kernel_speedup,green_swapped_kernel_speedup,"
              "persistent_aware_kernel_speedup,persistent_swapped_kernel_speedup,pass,aware_gbps,roofline_frac,cpu_ms")
    rows, failures = [header], 0
    for mb in c["data_mb"]:
        print(f"===== data_mb={mb} threads={c['threads']} blocks_per_sm={c['blocks_per_sm']} "
              f"cache_mode={c['cache_mode']} =====", flush=True)
        st, out = run("xd_hist_run", *argv(mb))
        tb = re.search(r"baseline_blocks=(\d+)", out)
        pb = re.search(r"persistent_blocks=(\d+)", out)
        ms = {k: first_field(out, k) for k in ("baseline_kernel_ms", "green_aware_kernel_ms", "green_swapped_kernel_ms",
                                                "persistent_aware_kernel_ms", "persistent_swapped_kernel_ms")}
        corr = next((l.split()[1:6] for l in out.splitlines() if l.startswith("correct")), [])
        want = ["baseline=PASS", "green_aware=PASS", "green_swapped=PASS", "persistent_aware=PASS",
                "persistent_swapped=PASS"]
        ok = st == 0 and corr == want  # applications/histogram/run.sh:80
        b = ms["baseline_kernel_ms"]
        rows.append(",".join([GPU_LABEL, str(run.ctx.index), str(mb), str(c["threads"]), str(c["blocks_per_sm"]),
                              tb.group(1) if tb else "", pb.group(1) if pb else "", str(c["runs"]),
                              str(c["cache_mode"]), b, ms["green_aware_kernel_ms"], ms["green_swapped_kernel_ms"],
                              ms["persistent_aware_kernel_ms"], ms["persistent_swapped_kernel_ms"],
                              ratio(b, ms["green_aware_kernel_ms"], "%.6f"),
                              ratio(b, ms["green_swapped_kernel_ms"], "%.6f"),
                              ratio(b, ms["persistent_aware_kernel_ms"], "%.6f"),
                              ratio(b, ms["persistent_swapped_kernel_ms"], "%.6f"), "PASS" if ok else "FAIL",
                              kv_tokens(out, "gbps ").get("aware", ""),
                              kv_tokens(out, "roofline=").get("roofline_frac", ""),
                              kv_tokens(out, "cpu_ms=").get("cpu_ms", "")]))
        failures += 0 if ok else 1
    csv.write_text("\n".join(rows) + "\n")
    print(f"CSV: {csv}")
    return failures


def run_hash(args, run, out_dir: Path):
    runs, cases = hash_cases(args.preset)
    if args.dry_run:
        for case in cases:
            run("xd_hash_run", *case, runs)
        return 0
    csv = out_dir / f"hash_{GPU_LABEL}_{args.preset}.csv"
    header = ("K,Q,C,effective_load,L,h,H,baseline_ms,aware_ms,swapped_ms,aware_speedup,swapped_speedup,pass,"
              "aware_mprobes_per_s")
    rows, failures = [header], 0
    for K, Q, C, L, h, H in cases:
        print(f"===== K={K} Q={Q} C={C} L={L} h={h} H={H} =====", flush=True)
        st, out = run("xd_hash_run", K, Q, C, L, h, H, runs)
        res = kv_tokens(out, "RESULT ")  # applications/hash/run.sh:62-66
        ok = st == 0 and res.get("pass") == "PASS"
        rows.append(",".join([str(K), str(Q), str(C), "%.6f" % (100.0 * K / C), str(L), str(h), str(H),
                              res.get("baseline_ms", ""), res.get("aware_ms", ""), res.get("swapped_ms", ""),
                              res.get("aware_speedup", ""), res.get("swapped_speedup", ""), "PASS" if ok else "FAIL",
                              kv_tokens(out, "mprobes_per_s ").get("aware", "")]))
        failures += 0 if ok else 1
    csv.write_text("\n".join(rows) + "\n")
    print(f"CSV: {csv}")
    return failures


def run_bfs(args, run, out_dir: Path):
    cases = bfs_cases(args.preset)
    argv = lambda p: (p["vertices"], p["degree"], p["sources"], p["depth"], p["dst_local"], p["hot"],  # noqa: E731
                      p["runs"], p["seed"])
    if args.dry_run:
        for _, _, p in cases:
            run("xd_bfs_run", *argv(p))
        return 0
    csv = out_dir / f"bfs_{GPU_LABEL}_{args.preset}.csv"
    header = ("sweep,value,gpu_label,gpu_index,vertices,degree,sources,depth,dst_local_pct,hot_per_side,runs,seed,"
              "visited,aware_bad,swapped_bad,overflow,baseline_med_ms,aware_med_ms,swapped_med_ms,aware_speedup,"
              "swapped_speedup,pass,aware_gteps,baseline_bad")
    rows, failures = [header], 0
    for sweep, value, p in cases:
        print(f"===== {sweep}={value} degree={p['degree']} sources={p['sources']} depth={p['depth']} "
              f"dst_local={p['dst_local']} =====", flush=True)
        st, out = run("xd_bfs_run", *argv(p))
        vis = kv_tokens(out, "visited=")  # applications/bfs/run.sh:84
        table = {}
        for line in out.splitlines():
            if line.startswith("| ") and not line.startswith("| mode"):
                cells = [c.strip() for c in line.split("|")]
                if len(cells) > 2:
                    table[cells[1]] = cells[2]
        base, aware, swap = table.get("baseline", ""), table.get("aware", ""), table.get("swapped", "")
        ok = (st == 0 and vis.get("aware_bad") == "0" and vis.get("swapped_bad") == "0"
              and vis.get("overflow") == "0")  # applications/bfs/run.sh:92
        rows.append(",".join([sweep, value, GPU_LABEL, str(run.ctx.index), str(p["vertices"]), str(p["degree"]),
                              str(p["sources"]), str(p["depth"]), str(p["dst_local"]), str(p["hot"]), str(p["runs"]),
                              str(p["seed"]), vis.get("visited", ""), vis.get("aware_bad", ""),
                              vis.get("swapped_bad", ""), vis.get("overflow", ""), base, aware, swap,
                              ratio(base, aware, "%.6f"), ratio(base, swap, "%.6f"), "PASS" if ok else "FAIL",
                              kv_tokens(out, "gteps ").get("aware", ""), vis.get("baseline_bad", "")]))
        failures += 0 if ok else 1
    csv.write_text("\n".join(rows) + "\n")
    print(f"CSV: {csv}")
    return failures


def run_architecture(args, run, out_dir: Path):
    """architecture/_run_figure.sh for the figures this build measures: 2 (XDom-PChase, the
    leader/follower chase), 3 (DomainScan latency curves of every compute unit after a leader
    on XCD 0) and 4 (MaskProbe, with the L2 channel functions beside it in
    figure_04_channels.csv and the memory-side unit classes in figure_04_memchannels.csv);
    DomainScan's workgroup -> XCD map goes beside every figure."""
    tag = "%02d" % args.figure
    data = out_dir / "data"
    csv = data / f"figure_{tag}.csv"
    if not args.dry_run:
        data.mkdir(parents=True, exist_ok=True)
        csv.unlink(missing_ok=True)
    st1 = 0
    if args.figure == 2:
        leader, follower = (0, 4) if args.peer == "auto" else map(int, args.peer.split(","))
        st, _ = run("xd_arch_probe", "pchase", leader, follower, 2048, 128, f"--csv={csv}")
    elif args.figure == 3:
        st, _ = run("xd_arch_probe", "scanlat", 7, 31, 0, f"--csv={csv}")
    else:
        st, _ = run("xd_arch_probe", "maskprobe", 5, 29, 8, f"--csv={csv}")
        chan = data / "figure_04_channels.csv"
        if not args.dry_run:
            chan.unlink(missing_ok=True)
        st1, _ = run("xd_arch_probe", "chanprobe", 0, 7, 20, f"--csv={chan}")
        mem = data / "figure_04_memchannels.csv"
        if not args.dry_run:
            mem.unlink(missing_ok=True)
        st3, _ = run("xd_arch_probe", "memprobe", 7, 20, 6, f"--csv={mem}")
        st1 = st1 or st3
    st2, _ = run("xd_arch_probe", "domainscan", 4096, f"--csv={data / 'domainscan.csv'}")
    if not args.dry_run:
        print(f"Figure {tag} CSV: {csv}")
    return (1 if st else 0) + (1 if st1 else 0) + (1 if st2 else 0)


APP_FUNCS = {"gemv": run_gemv, "histogram": run_histogram, "hash": run_hash, "bfs": run_bfs,
             "architecture": run_architecture}


def parse(argv):
    ap = argparse.ArgumentParser(prog="python -m l2domain_amd.run",
                                 description="Run an application's preset on MI355X (the reference's run.sh layer).")
    ap.add_argument("app", choices=APPS)
    ap.add_argument("--device", default="auto", help="GPU selection: auto, physical index or unique id (default: auto)")
    ap.add_argument("--preset", default="quick", help="quick (smoke point) or paper (sweep); default quick")
    ap.add_argument("--build-only", action="store_true", help="compile without running")
    ap.add_argument("--dry-run", action="store_true", help="print commands without executing them")
    ap.add_argument("--arch", default="auto", help="auto or gfx950")
    ap.add_argument("--wait-timeout", type=int, default=1800, help="wait for a free GPU (seconds, default 1800)")
    ap.add_argument("--poll-interval", type=int, default=10, help="GPU polling interval (seconds, default 10)")
    ap.add_argument("--output-dir", default=None, help="runtime output directory (default: out/APP)")
    ap.add_argument("--figure", type=int, default=2, help="architecture: figure 2, 3 or 4")
    ap.add_argument("--peer", default="auto", help="architecture figure 2: leader,follower XCD pair")
    args = ap.parse_args(argv)
    if args.preset not in ("quick", "paper"):
        raise UsageError("--preset must be quick or paper")
    if args.wait_timeout < 0 or args.poll_interval < 0:
        raise UsageError("--wait-timeout and --poll-interval must be non-negative integers")
    if args.arch not in ("auto", "gfx950"):
        raise UsageError("--arch must be auto or gfx950 (this build targets MI355X only)")
    if args.device != "auto" and not re.fullmatch(r"\d+|[0-9A-Za-z_-]{8,}", args.device):
        raise UsageError("--device must be auto, a physical index or a unique id")
    if args.figure not in (2, 3, 4):
        raise UsageError("--figure must be 2, 3 or 4")
    if args.peer != "auto" and (args.figure != 2 or not re.fullmatch(r"[0-7],[0-7]", args.peer)):
        raise UsageError("--peer must be A,B with XCD ids in [0, 8), and only for figure 2")
    if args.output_dir == "":
        raise UsageError("--output-dir must not be empty")
    return args


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    try:
        args = parse(argv)
    except UsageError as e:
        print(str(e), file=sys.stderr)
        return 2
    out_dir = Path(args.output_dir or (Path("out") / args.app)).resolve()
    # the reference compiles on every run; here the library and runners are built when one
    # is missing, or always with --build-only
    runners = ["xd_gemv_run", "xd_gemv_vendor_run", "xd_hist_run", "xd_hash_run", "xd_bfs_run", "xd_arch_probe"]
    built = (PKG / "libxdom.so").exists() and all((BIN / r).exists() for r in runners)
    if args.build_only or not built:
        if args.dry_run:
            print(f"+ {sys.executable} -m l2domain_amd.build")
        else:
            from . import build
            build.build_library()
            build.build_runners()
    if args.build_only:
        return 0
    try:
        ctx = GpuContext(args)
    except UsageError as e:
        print(str(e), file=sys.stderr)
        return 2
    if not args.dry_run:
        out_dir.mkdir(parents=True, exist_ok=True)
    command = " ".join(shlex.quote(a) for a in ["python", "-m", "l2domain_amd.run", *argv])
    if args.app == "architecture":
        ctx.write_metadata(out_dir / "metadata" / ("figure_%02d.json" % args.figure), command, figure="%02d" % args.figure,
                           peer_request=args.peer, gpu_arch=ctx.arch)
    else:
        ctx.write_metadata(out_dir / "metadata.json", command, application=args.app, preset=args.preset)
    failures = APP_FUNCS[args.app](args, Runner(ctx, args.dry_run), out_dir)
    if failures > 0:
        print(f"{failures} benchmark case(s) failed", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
