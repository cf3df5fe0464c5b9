#!/usr/bin/env python3
"""Benchmark of the XCD-domain kernels on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--cold] [--only] [--no-cpu]

A step is one pass of the hot path over one batch of synthetic input already resident in
HBM: one GEMV call, one histogram of 2^28 keys, ... W untimed warm-up steps, then exactly K
steps timed with HIP events on the stream the kernels are launched on. Prints ONE JSON line.
`value` is the XCD-aware variant's throughput; the oblivious and rotated variants are
timed over the same K steps and reported beside it with the aware/oblivious speedup.
Unless --only is given, every other configuration (GEMV fp32 and fp16 warm and cold, hash,
the reference's dependent probe, byte histogram and fixed-depth BFS, BFS) is measured the same way, with at most 50 timed steps, under "extras".
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "GEMV GB/s (% HBM peak); hist Gkeys/s; XCD-aware vs oblivious speedup"
MODES = ("oblivious", "aware", "rotated")


def _cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


# ---------------------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------------------
class GemvF32:
    single_kernel = True  # a step is exactly one launch: the timed region gives its duration

    """configs[0]: fp32 y = A.x, A 4096x4096 and x from U[-1,1) (seed 4242)."""
    name = "gemv_f32_4096x4096"
    unit = "GB/s"
    dtype = "f32"
    dominant = "gemv_f32"

    def __init__(self, M=4096, K=4096):
        import numpy as np
        import torch
        from l2domain_amd import gen
        self.M, self.K = M, K
        from l2domain_amd.domain import home_map
        from l2domain_amd.gemv import workspace as gemv_workspace
        A, x = gen.gemv_f32_inputs(M, K)
        self.hA, self.hx = A, x
        self.A = torch.from_numpy(A).cuda()
        self.x = torch.from_numpy(x).cuda()
        self.y = torch.empty(M, dtype=torch.float32, device="cuda")
        self.home = home_map(self.A)
        self.ws = gemv_workspace(M, K, self.A.dtype)
        self.bytes = 4 * M * K + 4 * K + 4 * M
        self.np = np

    def step(self, mode):
        from l2domain_amd.gemv import gemv
        gemv(self.A, self.x, self.y, mode=mode, home_attr=self.home, workspace=self.ws)

    def throughput(self, sec_per_step):
        return self.bytes / sec_per_step / 1e9

    def verify(self):
        import oracle as ora
        ref, yabs = ora.gemv_f64(self.hA, self.hx, nthreads=_cpu_threads())
        ok = True
        for mode in MODES:
            self.step(mode)
            y = self.y.cpu().numpy()
            rel = float(self.np.max(self.np.abs(y - ref)) / self.np.max(self.np.abs(ref)))
            ok = ok and rel <= 1e-3
        return ok

    def roofline(self, sec_per_launch):
        achieved = self.bytes / sec_per_launch / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": self.kernel_name(), "algorithmic_bytes_per_launch": self.bytes}

    def kernel_name(self):
        # the aware launch routes rows by home die when a row divides an 8 KiB interleave chunk
        row_bytes = self.A.element_size() * self.K
        f16 = "true" if self.A.element_size() == 2 else "false"
        if 8192 % row_bytes == 0:
            return f"gemv_rowhome_kernel<{f16},*>"
        if self.ws is not None and self.A.data_ptr() % 8192 == 0:
            return f"gemv_seghome_kernel<{f16}>"
        return f"gemv_exact_kernel<{f16},*>"

    def config(self):
        return {"workload": self.name, "M": self.M, "K": self.K, "dtype": "fp32", "seed": 4242}

    def cpu_baseline(self):
        import oracle as ora
        nt = _cpu_threads()
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 2.0:
            ora.gemv_f32_seq(self.hA, self.hx, nthreads=nt)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        return {"value": round(self.bytes / dt / 1e9, 3), "unit": "GB/s", "cores": nt, "kind": "port",
                "sample": f"{reps} full 4096x4096 fp32 GEMVs (oracle fp32 row loop, GEMV.cu:383-390)"}


class GemvF16(GemvF32):
    """fp16 W (N(0,0.02), seed 4243), x (N(0,1), seed 4244), fp32 accumulate."""
    dtype = "f16->f32"
    dominant = "gemv_f16f32"

    def __init__(self, M=14336, K=4096):
        import numpy as np
        import torch
        from l2domain_amd import gen
        self.M, self.K = M, K
        self.name = f"gemv_f16_{M}x{K}"
        from l2domain_amd.domain import home_map
        from l2domain_amd.gemv import workspace as gemv_workspace
        W, x = gen.gemv_f16_inputs(M, K)
        self.hA, self.hx = W, x
        self.A = torch.from_numpy(W).cuda()
        self.x = torch.from_numpy(x).cuda()
        self.y = torch.empty(M, dtype=torch.float32, device="cuda")
        self.home = home_map(self.A)
        self.ws = gemv_workspace(M, K, self.A.dtype)
        self.bytes = 2 * M * K + 2 * K + 4 * M
        self.np = np

    def verify(self):
        import oracle as ora
        ref, _ = ora.gemv_f64(self.hA, self.hx, nthreads=_cpu_threads())
        ok = True
        for mode in MODES:
            self.step(mode)
            y = self.y.cpu().numpy()
            ok = ok and float(self.np.max(self.np.abs(y - ref)) / self.np.max(self.np.abs(ref))) <= 2e-2
        return ok

    def config(self):
        return {"workload": self.name, "M": self.M, "K": self.K, "dtype": "fp16 in, fp32 accumulate",
                "seeds": [4243, 4244]}

    def cpu_baseline(self):
        import oracle as ora
        nt = _cpu_threads()
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 2.0:
            ora.gemv_f64(self.hA, self.hx, nthreads=nt)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        return {"value": round(self.bytes / dt / 1e9, 3), "unit": "GB/s", "cores": nt, "kind": "port",
                "sample": f"{reps} full {self.M}x{self.K} fp16 GEMVs (oracle row loop)"}


class Hist:
    """2^28 u32 keys ~ Zipf(1.1) over 2^20 bins (seed 1373), bit-exact counts."""
    name = "hist_2p28_zipf1.1_2p20bins"
    unit = "Gkeys/s"
    dtype = "u32"
    dominant = "hist_partition"

    def __init__(self, n=1 << 28, num_bins=1 << 20):
        import torch
        from l2domain_amd import gen
        from l2domain_amd.domain import home_map
        from l2domain_amd.histogram import HIST_SEED, ZIPF_S, Histogram
        self.n, self.num_bins = n, num_bins
        self.keys = gen.zipf_keys_device(n, num_bins, HIST_SEED, ZIPF_S)
        self.home = home_map(self.keys.view(torch.uint8))  # the aware mode reads near chunks
        self.h = Histogram(n, num_bins)
        self.counts = torch.empty(num_bins, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        # algorithmic bytes: 4 B per key read + 4 B per counter written
        self.bytes = 4 * n + 4 * num_bins

    def step(self, mode):
        self.h(self.keys, self.counts, mode=mode, home_attr=self.home)

    def throughput(self, sec_per_step):
        return self.n / sec_per_step / 1e9

    def verify(self):
        import numpy as np
        import oracle as ora
        host = self.keys.cpu().numpy().view(np.uint32)
        ref, _ = ora.histogram(host, self.num_bins, nthreads=_cpu_threads())
        self._host = host
        ok = True
        for mode in MODES:
            self.step(mode)
            got = self.counts.cpu().numpy().view(np.uint32)
            ok = ok and bool(np.array_equal(got, ref))
        return ok

    def roofline(self, sec_per_launch):
        # dominant kernel: the partition pass; its algorithmic traffic is the 4 B/key read.
        # traffic: rocprofv3 --pmc FETCH_SIZE (x2.000, copy-kernel calibration) + WRITE_SIZE of
        # the aware (routed) launch at this configuration: 1,073,954,202 B read + 540,019,405 B
        # written.
        achieved = 4 * self.n / sec_per_launch / 1e9
        traffic = 1613854300 if (self.n, self.num_bins) == (1 << 28, 1 << 20) else None
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": "hist_partition_kernel",
                "algorithmic_bytes_per_launch": 4 * self.n}

    def op_roofline(self, sec_per_step):
        achieved = self.bytes / sec_per_step / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": self.bytes}

    def config(self):
        return {"workload": self.name, "keys": self.n, "bins": self.num_bins, "zipf_s": 1.1, "seed": 1373,
                "bin_map": "scrambled rank ((r+1)*0x9E3779B1 mod 2^20)"}

    def cpu_baseline(self):
        import numpy as np
        import oracle as ora
        nt = _cpu_threads()
        sample = self._host[: 1 << 26] if hasattr(self, "_host") else self.keys[: 1 << 26].cpu().numpy().view(np.uint32)
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 10.0:
            ora.histogram(sample, self.num_bins, nthreads=nt)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        return {"value": round(sample.size / dt / 1e9, 4), "unit": "Gkeys/s", "cores": nt, "kind": "port",
                "sample": f"{reps} x 2^26 keys of the same Zipf stream (oracle counting loop, HIST.cu:279-288, "
                          f"{nt} threads with private histograms)"}


class Hash:
    """2^26 distinct u64 keys + values inserted at load factor 0.5 (2^27 slots),
    then 2^26 lookups at 50% hits. A step = clear + insert + lookup."""
    name = "hash_2p26_lf0.5_u64"
    unit = "Mops/s"
    dtype = "u64"
    dominant = "hash_lookup"

    def __init__(self):
        import torch
        from l2domain_amd.hashtable import HASH_KEYS, HASH_SEED, HASH_QSEED, HASH_SLOTS, HashTable, gen_kv, gen_queries
        self.n, self.slots = HASH_KEYS, HASH_SLOTS
        self.keys, self.vals = gen_kv(self.n, HASH_SEED)
        self.q = gen_queries(self.n, self.n, HASH_SEED, HASH_QSEED)
        self.t = HashTable(self.slots)
        self.v = torch.empty(self.n, dtype=torch.int64, device="cuda")
        self.f = torch.empty(self.n, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()

    def step(self, mode):
        self.t.clear()
        self.t.insert(self.keys, self.vals, mode=mode)
        self.t.lookup(self.q, mode=mode, vals_out=self.v, found_out=self.f)

    def throughput(self, sec_per_step):
        return 2 * self.n / sec_per_step / 1e6

    def verify(self):
        import numpy as np
        import oracle as ora
        hk = self.keys.cpu().numpy().view(np.uint64)
        hv = self.vals.cpu().numpy().view(np.uint64)
        hq = self.q.cpu().numpy().view(np.uint64)
        ref = ora.HashTable(self.slots)
        ref.build(hk, hv)
        rv, rf = ref.lookup(hq, nthreads=_cpu_threads())
        self._ref = (hk, hv, hq)
        ok = True
        for mode in MODES:
            self.step(mode)
            ok = ok and self.t.failures() == 0
            ok = ok and bool(np.array_equal(self.f.cpu().numpy(), rf))
            ok = ok and bool(np.array_equal(self.v.cpu().numpy().view(np.uint64), rv))
        return ok

    def roofline(self, sec_per_launch):
        # algorithmic bytes: lookup = 8 B key + 16 B slot + 8 B value + 1 B found per query
        achieved = 33 * self.n / sec_per_launch / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "hash_lookup_kernel",
                "algorithmic_bytes_per_launch": 33 * self.n}

    def config(self):
        return {"workload": self.name, "keys": self.n, "slots": self.slots, "lookups": self.n, "hit_rate": 0.5,
                "seed": 42}

    def cpu_baseline(self):
        import numpy as np
        import oracle as ora
        hk, hv, hq = self._ref
        m = 1 << 23
        t0 = time.perf_counter()
        ref = ora.HashTable(1 << 24)
        ref.build(hk[:m], hv[:m])
        ref.lookup(hq[:m], nthreads=1)
        dt = time.perf_counter() - t0
        return {"value": round(2 * m / dt / 1e6, 3), "unit": "Mops/s", "cores": 1, "kind": "port",
                "sample": "2^23 serial inserts into 2^24 slots + 2^23 lookups (oracle, HASH.cu:46-64,226-241)"}


class Hist256:
    """The reference's own histogram workload (histogram256_sideaware.cu): data_mb = 512 (the
    paper preset's largest, applications/histogram/run.sh:16) of words[i] = mix32(i), every
    byte counted into 256 bins. A step = one xd_hist256_u32bytes call (count + fused merge)."""
    name = "hist256_bytes_512MiB_mix32"
    unit = "GB/s"
    dtype = "u8"
    dominant = "hist256"
    single_kernel = True

    def __init__(self, data_mb=512):
        import numpy as np
        import torch
        from l2domain_amd import gen
        from l2domain_amd.domain import home_map
        from l2domain_amd.histogram import ByteHistogram
        self.n = data_mb * (1 << 20) // 4
        self.data_mb = data_mb
        self.host = gen.mix32_words(self.n)
        self.words = torch.from_numpy(self.host.view(np.int32)).cuda()
        self.home = home_map(self.words.view(torch.uint8))
        self.bh = ByteHistogram()
        self.counts = torch.empty(256, dtype=torch.int32, device="cuda")
        self.bytes = 4 * self.n + 4 * 256

    def step(self, mode):
        self.bh(self.words, self.counts, mode=mode, home_attr=self.home)

    def throughput(self, sec_per_step):
        return self.bytes / sec_per_step / 1e9

    def verify(self):
        import numpy as np
        import oracle as ora
        ref = ora.hist256_bytes(self.host, nthreads=_cpu_threads())
        ok = True
        for mode in MODES:
            self.step(mode)
            ok = ok and bool(np.array_equal(self.counts.cpu().numpy().view(np.uint32), ref))
        return ok

    def roofline(self, sec_per_launch):
        achieved = self.bytes / sec_per_launch / 1e9
        # traffic: rocprofv3 --pmc FETCH_SIZE (x2.000, copy-kernel calibration) + WRITE_SIZE of
        # this kernel at this configuration: 537,088,000 B read + 550,912 B written.
        traffic = 537638912 if self.data_mb == 512 else None
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": "hist256_kernel",
                "algorithmic_bytes_per_launch": self.bytes}

    def config(self):
        return {"workload": self.name, "data_mb": self.data_mb, "words": self.n, "bins": 256,
                "data": "words[i] = mix32(i) (HIST.cu:331-340)"}

    def cpu_baseline(self):
        import oracle as ora
        nt = _cpu_threads()
        sample = self.host[: 1 << 26]
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 5.0:
            ora.hist256_bytes(sample, nthreads=nt)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        return {"value": round(4 * sample.size / dt / 1e9, 3), "unit": "GB/s", "cores": nt, "kind": "port",
                "sample": f"{reps} x 2^26 words of the same data (oracle byte-counting loop, HIST.cu:279-288, "
                          f"{nt} threads with private histograms)"}


class BfsRef:
    """The reference's own BFS workload at its paper preset (applications/bfs/run.sh:24-27):
    2,000,000 vertices of degree 64 in its directed hot-pool graph (hot_per_side 200,000,
    dst_local 95 %, seed 8201; sides from the measured homes of this run's buffers), 4096
    sources, 4 top-down levels. A step = one whole search, initialisation included."""
    name = "bfs_ref_V2M_deg64_src4096_depth4"
    unit = "GTEPS"
    dtype = "int32"
    dominant = "bfs_multi"

    def __init__(self):
        import numpy as np
        from l2domain_amd.bfs import REF_PAPER, RefGraph, ref_clamp
        p = REF_PAPER
        self.V, self.deg, self.nsrc, self.depth, self.dl, self.H = ref_clamp(
            p["vertices"], p["degree"], p["sources"], p["depth"], p["dst_local_pct"], p["hot_per_side"])
        self.g = RefGraph(self.V, self.deg, self.nsrc, self.dl, self.H, p["seed"])
        import oracle as ora
        self.ref, self.reached = ora.bfs_multi(self.g.h_rowptr, self.g.h_col, self.g.h_sources, self.depth)
        expanded = (self.ref != 0xFFFFFFFF) & (self.ref < self.depth)
        self.edges = int(np.diff(self.g.h_rowptr.astype(np.int64))[expanded].sum())
        self.nexp = int(expanded.sum())
        self.np = np

    def step(self, mode):
        self.g.bfs(self.depth, mode=mode)

    def throughput(self, sec_per_step):
        return self.edges / sec_per_step / 1e9

    def verify(self):
        ok = True
        for mode in MODES:
            self.step(mode)
            got = self.g.level.cpu().numpy().view(self.np.uint32)
            ok = ok and bool(self.np.array_equal(got, self.ref))
        return ok

    def roofline(self, sec_per_launch):
        # adjacency lists of the expanded vertices, their two rowptr entries, and the level
        # array written once (initialisation)
        nbytes = 4 * self.edges + 8 * self.nexp + 4 * self.V
        achieved = nbytes / sec_per_launch / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "bfs search (multi_init/seed/level kernels)", "algorithmic_bytes_per_bfs": nbytes}

    def config(self):
        return {"workload": self.name, "vertices": self.V, "degree": self.deg, "sources": self.nsrc,
                "depth": self.depth, "dst_local_pct": self.dl, "hot_per_side": self.H, "seed": 8201,
                "edges_walked": self.edges, "reached": self.reached}

    def cpu_baseline(self):
        import oracle as ora
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 5.0:
            ora.bfs_multi(self.g.h_rowptr, self.g.h_col, self.g.h_sources, self.depth)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        return {"value": round(self.edges / dt / 1e9, 4), "unit": "GTEPS", "cores": 1, "kind": "port",
                "sample": f"{reps} full serial multi-source searches of the same graph (oracle, bfs.cu:215-252)"}


class HashDep:
    """The reference's own hash workload (hash_probe_dep.cu, defaults :124-130): K = 32000000
    int32 keys with successors in 2^26 8-byte entries, two hot pools of 100000 keys homed on
    opposite I/O dies, 8000000 queries (80 % hot) following their chains for 4 dependent
    probes. A step = one probe pass."""
    name = "hash_dep_K32M_Q8M_C2p26_L4"
    unit = "Mprobes/s"
    dtype = "int32"
    dominant = "dep_probe"
    single_kernel = True

    def __init__(self, K=32000000, Q=8000000, slots=1 << 26, L=4, hot=80, H=100000):
        import torch
        from l2domain_amd.hashdep import DepTable
        self.K, self.Q, self.slots, self.L, self.hot, self.H = K, Q, slots, L, hot, H
        t0 = time.perf_counter()
        self.t = DepTable(K, slots, H)
        self.hq = self.t.queries(Q, hot)
        self.build_s = time.perf_counter() - t0
        self.q = torch.from_numpy(self.hq).cuda()
        self.out = torch.empty(Q, dtype=torch.int32, device="cuda")

    def step(self, mode):
        self.t.probe(self.q, self.L, mode=mode, out=self.out)

    def throughput(self, sec_per_step):
        return self.Q * self.L / sec_per_step / 1e6

    def verify(self):
        import numpy as np
        import oracle as ora
        ref = ora.dep_probe(self.t.host_table, self.slots, self.hq, self.L)
        ok = True
        for mode in MODES:
            self.step(mode)
            ok = ok and bool(np.array_equal(self.out.cpu().numpy(), ref))
        return ok

    def roofline(self, sec_per_launch):
        # latency-bound dependent chains: algorithmic bytes = 8 B entry per probe + 4 B query
        # in + 4 B out per query
        nbytes = 8 * self.Q * self.L + 8 * self.Q
        achieved = nbytes / sec_per_launch / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "dep_probe_kernel",
                "algorithmic_bytes_per_launch": nbytes}

    def config(self):
        return {"workload": self.name, "K": self.K, "Q": self.Q, "C": self.slots, "L": self.L, "hot_pct": self.hot,
                "H": self.H, "seed": 42, "host_build_s": round(self.build_s, 2)}

    def cpu_baseline(self):
        import oracle as ora
        n = 1 << 20
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 5.0:
            ora.dep_probe(self.t.host_table, self.slots, self.hq[:n], self.L)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        return {"value": round(n * self.L / dt / 1e6, 3), "unit": "Mprobes/s", "cores": 1, "kind": "port",
                "sample": f"{reps} x 2^20 queries of the same stream (oracle probe_dep_base loop, HASH.cu:66-83)"}


class Bfs:
    """undirected R-MAT scale 22, edge factor 16, a/b/c/d = .57/.19/.19/.05 (seed
    8201), CSR int32, source 0. A step = one BFS to completion."""
    name = "bfs_rmat22_ef16"
    unit = "GTEPS"
    dtype = "int32"
    dominant = "bfs_level"
    single_kernel = True  # roofline over the whole search (init, levels, control, conversion)

    def __init__(self):
        from l2domain_amd.bfs import RMAT_EDGE_FACTOR, RMAT_SCALE, RMAT_SEED, Graph, rmat_csr
        t0 = time.perf_counter()
        self.rowptr, self.col = rmat_csr(RMAT_SCALE, RMAT_EDGE_FACTOR, RMAT_SEED)
        self.gen_s = time.perf_counter() - t0
        self.g = Graph(self.rowptr, self.col)
        self.stats = None

    def step(self, mode):
        _, self.stats = self.g.bfs(0, mode=mode)

    def throughput(self, sec_per_step):
        return self.stats["reached_edges"] / 2 / sec_per_step / 1e9

    def verify(self):
        import numpy as np
        import oracle as ora
        ref, _ = ora.bfs(self.rowptr, self.col, 0)
        ok = True
        for mode in MODES:
            self.step(mode)
            ok = ok and bool(np.array_equal(self.g.level.cpu().numpy().view(np.uint32), ref))
        return ok

    def roofline(self, sec_per_launch):
        # algorithmic bytes per search: CSR read once + level written once, 4(V+1) + 4 nnz + 4V,
        # over the time of the whole search (sec_per_launch is the per-step time here)
        V = self.g.V
        nbytes = 4 * (V + 1) + 4 * self.stats["reached_edges"] + 4 * V
        achieved = nbytes / sec_per_launch / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "bfs search (bfs_level/hubs/control/b2q kernels)", "algorithmic_bytes_per_bfs": nbytes}

    def config(self):
        return {"workload": self.name, "vertices": self.g.V, "nnz": self.g.nnz, "source": 0, "seed": 8201,
                "levels": self.stats["levels"] if self.stats else None,
                "reached_edges": self.stats["reached_edges"] if self.stats else None,
                "host_generation_s": round(self.gen_s, 2)}

    def cpu_baseline(self):
        import oracle as ora
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 3.0:
            ora.bfs(self.rowptr, self.col, 0)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        return {"value": round(self.stats["reached_edges"] / 2 / dt / 1e9, 4), "unit": "GTEPS", "cores": 1,
                "kind": "port", "sample": f"{reps} full serial queue BFS runs of the same graph (oracle)"}


WORKLOADS = {
    "hist": Hist,
    "bfs": Bfs,
    "hash": Hash,
    "hash_dep": HashDep,
    "hist256": Hist256,
    "bfs_ref": BfsRef,
    "gemv_f32": GemvF32,
    "gemv_f16_up": lambda: GemvF16(14336, 4096),
    "gemv_f16_down": lambda: GemvF16(4096, 14336),
}
DEFAULT_WORKLOAD = "hist"
# every other BASELINE config, reported under "extras" of the same JSON line
EXTRAS = (("gemv_f32", False), ("gemv_f32", True), ("gemv_f16_up", False), ("gemv_f16_up", True),
          ("gemv_f16_down", False), ("gemv_f16_down", True), ("hash", False), ("hash_dep", False),
          ("bfs", False), ("hist256", True), ("hist256", False), ("bfs_ref", False))


# ---------------------------------------------------------------------------------------
# Timing
# ---------------------------------------------------------------------------------------
def time_steps(wl, mode, steps, warmup, flusher=None):
    """Returns seconds per step over exactly `steps` steps (HIP events on the launch stream)."""
    import torch
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        wl.step(mode)
    torch.cuda.synchronize()
    if flusher is None:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            wl.step(mode)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / steps
    # cold: flush before each step, time each step separately
    total = 0.0
    for _ in range(steps):
        flusher.flush()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        wl.step(mode)
        e1.record(stream)
        torch.cuda.synchronize()
        total += e0.elapsed_time(e1) / 1e3
    return total / steps


def kernel_times(wl, mode, steps, flusher=None):
    """Per-kernel average launch duration (s) from the library's HIP events, over `steps` steps."""
    import torch
    from l2domain_amd import _lib
    torch.cuda.synchronize()
    _lib.timing_enable(True)
    for _ in range(steps):
        if flusher is not None:
            flusher.flush()
        wl.step(mode)
    torch.cuda.synchronize()
    t = _lib.timing_read()
    _lib.timing_enable(False)
    return {k: (ms / 1e3 / max(n, 1), n) for k, (ms, n) in t.items()}


def launch_seconds(wl, r):
    """Average duration of the dominant kernel in the aware mode. A one-kernel step is timed by
    the back-to-back timed region (per-launch events would add their own overhead to a ~10 us
    kernel); otherwise by the library's HIP events around that kernel."""
    if getattr(wl, "single_kernel", False):
        return r["sec"]["aware"]
    return r["kernels"][wl.dominant][0]


def run_workload(name, steps, warmup, cold=False, with_cpu=True):
    import torch
    from l2domain_amd.domain import CacheFlusher
    wl = WORKLOADS[name]()
    ok = wl.verify()
    flusher = CacheFlusher() if cold else None
    res = {}
    for mode in MODES:
        res[mode] = time_steps(wl, mode, steps, warmup, flusher)
    torch.cuda.synchronize()
    kt = kernel_times(wl, "aware", steps, flusher)
    kt_modes = {m: (kt if m == "aware" else kernel_times(wl, m, min(steps, 5), flusher)) for m in MODES}
    out = {
        "workload": wl,
        "verified": ok,
        "sec": res,
        "tput": {m: wl.throughput(s) for m, s in res.items()},
        "kernels": kt,
        "kernels_by_mode": kt_modes,
    }
    if with_cpu:
        out["cpu"] = wl.cpu_baseline()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    ap.add_argument("--cold", action="store_true", help="flush L2 + Infinity Cache before every step")
    ap.add_argument("--only", action="store_true", help="measure the selected workload only (no extras)")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one MI355X only (one-GPU tier); "
              f"--gpus {args.gpus} / WORLD_SIZE={world} is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        sys.exit(1)
    from l2domain_amd.domain import topology

    r = run_workload(args.workload, args.steps, args.warmup, cold=args.cold, with_cpu=not args.no_cpu)
    wl = r["workload"]
    sec = r["sec"]["aware"]
    line = {
        "metric": METRIC,
        "value": round(r["tput"]["aware"], 3),
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype,
        "data": "synthetic (seeded generators, inputs resident in HBM)",
        "config": dict(wl.config(), cache="cold" if args.cold else "warm", mode="xcd_aware"),
        "verified": r["verified"],
        "modes": {m: {"ms_per_step": round(r["sec"][m] * 1e3, 6), "value": round(r["tput"][m], 3)}
                  for m in MODES},
        "speedup_aware_vs_oblivious": round(r["sec"]["oblivious"] / r["sec"]["aware"], 4),
        "speedup_rotated_vs_oblivious": round(r["sec"]["oblivious"] / r["sec"]["rotated"], 4),
        "roofline": wl.roofline(launch_seconds(wl, r)),
        "kernels_us": {k: round(v[0] * 1e6, 3) for k, v in r["kernels"].items()},
        "kernels_us_by_mode": {m: {k: round(v[0] * 1e6, 3) for k, v in kk.items()}
                               for m, kk in r["kernels_by_mode"].items()},
        "cpu_baseline": r.get("cpu"),
        "device": topology(0)["name"],
    }
    if hasattr(wl, "op_roofline"):
        line["roofline_op"] = wl.op_roofline(sec)
    if not args.only:
        extras = {}
        esteps = min(args.steps, 50)
        for name, cold in EXTRAS:
            if name == args.workload and cold == args.cold:
                continue
            print(f"bench.py: extra {name} ({'cold' if cold else 'warm'})", file=sys.stderr, flush=True)
            e = run_workload(name, esteps, min(args.warmup, 5), cold=cold, with_cpu=not args.no_cpu and not cold)
            ew = e["workload"]
            entry = {"verified": e["verified"], "unit": ew.unit, "steps": esteps,
                     "cache": "cold" if cold else "warm", "config": ew.config(),
                     "value_aware": round(e["tput"]["aware"], 3),
                     "value_oblivious": round(e["tput"]["oblivious"], 3),
                     "value_rotated": round(e["tput"]["rotated"], 3),
                     "speedup_aware_vs_oblivious": round(e["sec"]["oblivious"] / e["sec"]["aware"], 4),
                     "speedup_rotated_vs_oblivious": round(e["sec"]["oblivious"] / e["sec"]["rotated"], 4),
                     "roofline": ew.roofline(launch_seconds(ew, e)),
                     "kernels_us": {k: round(v[0] * 1e6, 3) for k, v in e["kernels"].items()},
                     "kernels_us_by_mode": {m: {k: round(v[0] * 1e6, 3) for k, v in kk.items()}
                                            for m, kk in e["kernels_by_mode"].items()}}
            if "cpu" in e:
                entry["cpu_baseline"] = e["cpu"]
            extras[f"{name}_{'cold' if cold else 'warm'}"] = entry
            del e, ew
            torch.cuda.empty_cache()
        line["extras"] = extras
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
