#!/usr/bin/env python3
"""Benchmark of the XCD-domain kernels on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--cold] [--only]
                [--modes aware,oblivious,rotated] [--no-cpu] [--no-verify] [--detail FILE]

A step is one pass of the hot path over one batch of synthetic input already resident in
HBM: one GEMV call, one histogram of 2^28 keys, one hash build + lookup, one BFS.
W untimed warm-up steps, then exactly K steps timed with HIP events on the stream the
kernels are launched on. Prints ONE JSON line: the headline (the
histogram, XCD-aware) first, then one short entry per other configuration under "configs".
`value` is the XCD-aware variant's throughput; the oblivious and rotated variants are timed
over the same K steps and reported beside it with the aware/oblivious speedup.

Rooflines use each kernel's own execution time: the library stamps a start/stop event pair
on every dispatch (hipExtLaunchKernel) while timing is on, so a duration here is what a
rocprofv3 kernel trace reports for that kernel. Warm configurations whose data fits the
Infinity Cache are priced against a read stream of the same footprint measured in the same
run (bound "infinity_cache"); the rest against the 8 TB/s HBM peak. A cold step flushes
the L2s and the Infinity Cache first and its throughput is taken from the kernels' own
durations (the flush and the dispatch gaps are not part of the step).

--detail FILE writes every per-kernel, per-mode duration and the CPU baseline samples as
JSON; --modes restricts the timed modes (one mode per rocprofv3 run gives one row per
configuration and mode).
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

# Bytes per step that the roofline kernel(s) move between the L2s and memory (HBM or the
# Infinity Cache), XCD-aware mode: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (KiB per
# dispatch) under `bench.py --only --no-cpu --no-verify --steps 10 --warmup 2 --workload W
# --modes aware [--cold]`, FETCH_SIZE scaled by the copy-kernel calibration factor (a 256 MiB
# copy reads 2.000x what FETCH_SIZE counts, WRITE_SIZE 1.000x), summed over a step's
# launches. Atomic and random-access kernels move whole requests (a 16-byte CAS or probe
# costs a request each way).
TRAFFIC_SRC = "profiles/traffic_by_config.md (FETCH_SIZE/WRITE_SIZE runs of the commit named there)"
TRAFFIC = {
    ("hist_2p28_zipf1.1_2p20bins", "warm", "aware"): 1305528162,
    ("hash_2p26_lf0.5_u64", "warm", "aware"): 19910025236,
    ("hist256_bytes_512MiB_mix32", "warm", "aware"): 543800710,
    ("hist256_bytes_512MiB_mix32", "cold", "aware"): 544154466,
    ("bfs_ref_V2M_deg64_src4096_depth4", "warm", "aware"): 245717927,
    ("hash_dep_K32M_Q8M_C2p26_L4", "warm", "aware"): 3927067605,
    ("bfs_rmat22_ef16", "warm", "aware"): 239020958,
    ("gemv_f32_4096x4096", "warm", "aware"): 67730532,
    ("gemv_f32_4096x4096", "cold", "aware"): 67736254,
    ("gemv_f16_14336x4096", "warm", "aware"): 117648613,
    ("gemv_f16_14336x4096", "cold", "aware"): 117649957,
    ("gemv_f16_4096x14336", "warm", "aware"): 117821674,
    ("gemv_f16_4096x14336", "cold", "aware"): 117821669,
}


def cpu_threads() -> int:
    """The host threads a CPU baseline may use: the process's CPU affinity, capped by
    OMP_NUM_THREADS where the box sets its CPU share there."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS")
    if share and share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(1, n)


def timed_loop(fn, min_s: float, max_reps: int = 1 << 30) -> tuple[float, int]:
    """Seconds per call of fn() over at least one call and about min_s seconds."""
    t0 = time.perf_counter()
    reps = 0
    while reps < max_reps:
        fn()
        reps += 1
        if time.perf_counter() - t0 >= min_s:
            break
    return (time.perf_counter() - t0) / reps, reps


# ---------------------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------------------
class Workload:
    single_kernel = False  # a step is exactly one launch
    min_steps = 1          # timed steps at least (configs[0]: "single call plus 100 timed repeats")
    ic_resident = False    # warm data fits the 256 MB Infinity Cache
    cpu_parallel = True    # the CPU restatement has a multi-threaded form
    roof_bytes = 0         # algorithmic bytes per launch of the roofline kernel(s)

    def roof_kernels(self, mode: str) -> tuple[str, ...]:
        """Kernels whose summed duration per step is the roofline launch."""
        raise NotImplementedError

    def roof_footprint(self):
        """Device tensor streamed to measure the Infinity-Cache peak of a warm run."""
        return None


class GemvF32(Workload):
    """fp32 y = A.x, A 4096x4096 and x from U[-1,1) (seed 4242)."""
    unit = "GB/s"
    dtype = "f32"
    ic_resident = True
    min_steps = 100  # a single call (the verification) plus 100 timed repeats, whatever --steps is

    def __init__(self, M=4096, K=4096):
        import numpy as np
        import torch
        from l2domain_amd import gen
        from l2domain_amd.domain import home_map
        from l2domain_amd.gemv import workspace as gemv_workspace
        self.M, self.K = M, K
        self.name = f"gemv_f32_{M}x{K}"
        A, x = gen.gemv_f32_inputs(M, K)
        self.hA, self.hx = A, x
        self.A = torch.from_numpy(A).cuda()
        self.x = torch.from_numpy(x).cuda()
        self.y = torch.empty(M, dtype=torch.float32, device="cuda")
        self.home = home_map(self.A)
        self.ws = gemv_workspace(M, K, self.A.dtype)
        self.bytes = 4 * M * K + 4 * K + 4 * M
        self.roof_bytes = self.bytes
        self.np = np

    def step(self, mode):
        from l2domain_amd.gemv import gemv
        gemv(self.A, self.x, self.y, mode=mode, home_attr=self.home, workspace=self.ws)

    def throughput(self, sec_per_step):
        return self.bytes / sec_per_step / 1e9

    def tol(self):
        return 1e-3

    def verify(self):
        import oracle as ora
        ref, _ = ora.gemv_f64(self.hA, self.hx, nthreads=cpu_threads())
        ok = True
        for mode in MODES:
            self.step(mode)
            y = self.y.cpu().numpy()
            rel = float(self.np.max(self.np.abs(y - ref)) / self.np.max(self.np.abs(ref)))
            ok = ok and rel <= self.tol()
        return ok

    def roof_kernels(self, mode):
        return ("gemv_kernel", "gemv_exact_kernel", "gemv_rowhome_kernel", "gemv_seghome_kernel")

    def roof_footprint(self):
        return self.A

    def config(self):
        return {"workload": self.name, "M": self.M, "K": self.K, "dtype": "fp32", "seed": 4242}

    def cpu_baseline(self, nt, budget_s):
        import oracle as ora
        dt, reps = timed_loop(lambda: ora.gemv_f32_seq(self.hA, self.hx, nthreads=nt), budget_s)
        return self.bytes / dt / 1e9, f"{reps} x {self.M}x{self.K} fp32 GEMV (oracle fp32 row loop, GEMV.cu:383-390)"


class GemvF16(GemvF32):
    """fp16 W (N(0,0.02), seed 4243), x (N(0,1), seed 4244), fp32 accumulate."""
    dtype = "f16->f32"

    def __init__(self, M=14336, K=4096):
        import numpy as np
        import torch
        from l2domain_amd import gen
        from l2domain_amd.domain import home_map
        from l2domain_amd.gemv import workspace as gemv_workspace
        self.M, self.K = M, K
        self.name = f"gemv_f16_{M}x{K}"
        W, x = gen.gemv_f16_inputs(M, K)
        self.hA, self.hx = W, x
        self.A = torch.from_numpy(W).cuda()
        self.x = torch.from_numpy(x).cuda()
        self.y = torch.empty(M, dtype=torch.float32, device="cuda")
        self.home = home_map(self.A)
        self.ws = gemv_workspace(M, K, self.A.dtype)
        self.bytes = 2 * M * K + 2 * K + 4 * M
        self.roof_bytes = self.bytes
        self.np = np

    def tol(self):
        return 2e-2

    def config(self):
        return {"workload": self.name, "M": self.M, "K": self.K, "dtype": "fp16 in, fp32 accumulate",
                "seeds": [4243, 4244]}

    def cpu_baseline(self, nt, budget_s):
        import oracle as ora
        dt, reps = timed_loop(lambda: ora.gemv_f64(self.hA, self.hx, nthreads=nt), budget_s)
        return self.bytes / dt / 1e9, f"{reps} x {self.M}x{self.K} fp16 GEMV (oracle row loop)"


class Hist(Workload):
    """2^28 u32 keys ~ Zipf(1.1) over 2^20 bins (seed 1373), bit-exact counts."""
    name = "hist_2p28_zipf1.1_2p20bins"
    unit = "Gkeys/s"
    dtype = "u32"

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
        # algorithmic bytes of the step: 4 B per key read + 4 B per counter written
        # (1,077,936,128 at the config); the roofline kernel, the partition pass, reads the keys
        # (4 B per key) and never touches the counters, which the merge writes
        self.bytes = 4 * n + 4 * num_bins
        self.roof_bytes = 4 * n
        self.roof_basis = "keys read by the partition pass (4 B per key); the counters are written by the merge"

    def step(self, mode):
        self.h(self.keys, self.counts, mode=mode, home_attr=self.home)

    def throughput(self, sec_per_step):
        return self.n / sec_per_step / 1e9

    def verify(self):
        import numpy as np
        import oracle as ora
        host = self.keys.cpu().numpy().view(np.uint32)
        ref, _ = ora.histogram(host, self.num_bins, nthreads=cpu_threads())
        self._host = host
        ok = True
        for mode in MODES:
            self.step(mode)
            got = self.counts.cpu().numpy().view(np.uint32)
            ok = ok and bool(np.array_equal(got, ref))
        return ok

    def roof_kernels(self, mode):
        return ("hist_partition_kernel",)

    def config(self):
        return {"workload": self.name, "keys": self.n, "bins": self.num_bins, "zipf_s": 1.1, "seed": 1373,
                "bin_map": "scrambled rank ((r+1)*0x9E3779B1 mod 2^20)"}

    def cpu_baseline(self, nt, budget_s):
        import numpy as np
        import oracle as ora
        sample = self._host[: 1 << 26] if hasattr(self, "_host") else self.keys[: 1 << 26].cpu().numpy().view(np.uint32)
        dt, reps = timed_loop(lambda: ora.histogram(sample, self.num_bins, nthreads=nt), budget_s)
        return sample.size / dt / 1e9, (f"{reps} x 2^26 keys of the same Zipf stream (oracle counting loop, "
                                         f"HIST.cu:279-288; threads keep private histograms)")


class Hash(Workload):
    """2^26 distinct u64 keys + values inserted at load factor 0.5 (2^27 slots),
    then 2^26 lookups at 50% hits. A step = the table built from the pairs (xd_hash_build_u64:
    every slot written, so it also clears) + the lookups."""
    name = "hash_2p26_lf0.5_u64"
    unit = "Mops/s"
    dtype = "u64"

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
        # the whole step: build (16 B pair in per key, every 16 B slot written) + lookups
        # (8 B query + one 16 B slot + 8 B value + 1 B found per query)
        self.roof_bytes = 16 * self.n + 16 * self.slots + 33 * self.n

    def step(self, mode):
        self.t.build(self.keys, self.vals, mode=mode)
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
        rv, rf = ref.lookup(hq, nthreads=cpu_threads())
        self._ref = (hk, hv, hq)
        del ref
        ok = True
        for mode in MODES:
            self.step(mode)
            ok = ok and self.t.failures() == 0
            ok = ok and bool(np.array_equal(self.f.cpu().numpy(), rf))
            ok = ok and bool(np.array_equal(self.v.cpu().numpy().view(np.uint64), rv))
        return ok

    def roof_kernels(self, mode):
        return ("hb_clear_kernel", "hb_split_kernel", "hb_build_kernel", "hb_fixup_kernel", "hash_lookup_kernel")

    def config(self):
        return {"workload": self.name, "keys": self.n, "slots": self.slots, "lookups": self.n, "hit_rate": 0.5,
                "seed": 42}

    def cpu_baseline(self, nt, budget_s):
        import oracle as ora
        hk, hv, hq = self._ref
        t0 = time.perf_counter()
        ref = ora.HashTable(self.slots)
        ref.build(hk, hv)
        t1 = time.perf_counter()
        ref.lookup(hq, nthreads=nt)
        t2 = time.perf_counter()
        del ref
        return 2 * self.n / (t2 - t0) / 1e6, (f"the whole config once: 2^26 serial inserts into 2^27 slots "
                                               f"({t1 - t0:.2f} s, HASH.cu:226-241) + 2^26 lookups ({t2 - t1:.2f} s, "
                                               f"HASH.cu:46-64)")


class Hist256(Workload):
    """The reference's own histogram workload (histogram256_sideaware.cu): data_mb = 512 (the
    paper preset's largest, applications/histogram/run.sh:16) of words[i] = mix32(i), every
    byte counted into 256 bins. A step = one xd_hist256_u32bytes call (count + fused merge)."""
    name = "hist256_bytes_512MiB_mix32"
    unit = "GB/s"
    dtype = "u8"
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
        self.roof_bytes = self.bytes

    def step(self, mode):
        self.bh(self.words, self.counts, mode=mode, home_attr=self.home)

    def throughput(self, sec_per_step):
        return self.bytes / sec_per_step / 1e9

    def verify(self):
        import numpy as np
        import oracle as ora
        ref = ora.hist256_bytes(self.host, nthreads=cpu_threads())
        ok = True
        for mode in MODES:
            self.step(mode)
            ok = ok and bool(np.array_equal(self.counts.cpu().numpy().view(np.uint32), ref))
        return ok

    def roof_kernels(self, mode):
        return ("hist256_kernel",)

    def config(self):
        return {"workload": self.name, "data_mb": self.data_mb, "words": self.n, "bins": 256,
                "data": "words[i] = mix32(i) (HIST.cu:331-340)"}

    def cpu_baseline(self, nt, budget_s):
        import oracle as ora
        sample = self.host[: 1 << 26]
        dt, reps = timed_loop(lambda: ora.hist256_bytes(sample, nthreads=nt), budget_s)
        return 4 * sample.size / dt / 1e9, (f"{reps} x 2^26 words of the same data (oracle byte-counting loop, "
                                             f"HIST.cu:279-288)")


class BfsRef(Workload):
    """The reference's own BFS workload at its paper preset (applications/bfs/run.sh:24-27):
    2,000,000 vertices of degree 64 in its directed hot-pool graph (hot_per_side 200,000,
    dst_local 95 %, seed 8201; sides from the measured homes of this run's buffers), 4096
    sources, 4 top-down levels. A step = one whole search, initialisation included."""
    name = "bfs_ref_V2M_deg64_src4096_depth4"
    unit = "GTEPS"
    dtype = "int32"
    cpu_parallel = False

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
        # adjacency lists of the expanded vertices, their two rowptr entries, and the level
        # array written once (initialisation)
        self.roof_bytes = 4 * self.edges + 8 * self.nexp + 4 * self.V
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

    def roof_kernels(self, mode):
        return ("multi_init_kernel", "multi_seed_kernel", "multi_level_kernel")

    def config(self):
        return {"workload": self.name, "vertices": self.V, "degree": self.deg, "sources": self.nsrc,
                "depth": self.depth, "dst_local_pct": self.dl, "hot_per_side": self.H, "seed": 8201,
                "edges_walked": self.edges, "reached": self.reached}

    def cpu_baseline(self, nt, budget_s):
        import oracle as ora
        dt, reps = timed_loop(lambda: ora.bfs_multi(self.g.h_rowptr, self.g.h_col, self.g.h_sources, self.depth),
                              budget_s)
        return self.edges / dt / 1e9, f"{reps} serial multi-source searches of the same graph (oracle, BFS.cu:215-252)"


class HashDep(Workload):
    """The reference's own hash workload (hash_probe_dep.cu, defaults :124-130): K = 32000000
    int32 keys with successors in 2^26 8-byte entries, two hot pools of 100000 keys homed on
    opposite I/O dies, 8000000 queries (80 % hot) following their chains for 4 dependent
    probes. A step = one probe pass."""
    name = "hash_dep_K32M_Q8M_C2p26_L4"
    unit = "Mprobes/s"
    dtype = "int32"
    single_kernel = True
    cpu_parallel = False

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
        # latency-bound dependent chains: 8 B entry per probe + 4 B query in + 4 B out
        self.roof_bytes = 8 * Q * L + 8 * Q

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

    def roof_kernels(self, mode):
        return ("dep_probe_kernel",)

    def config(self):
        return {"workload": self.name, "K": self.K, "Q": self.Q, "C": self.slots, "L": self.L, "hot_pct": self.hot,
                "H": self.H, "seed": 42, "host_build_s": round(self.build_s, 2)}

    def cpu_baseline(self, nt, budget_s):
        import oracle as ora
        n = 1 << 20
        dt, reps = timed_loop(lambda: ora.dep_probe(self.t.host_table, self.slots, self.hq[:n], self.L), budget_s)
        return n * self.L / dt / 1e6, f"{reps} x 2^20 queries of the same stream (oracle probe_dep_base loop, HASH.cu:66-83)"


class Bfs(Workload):
    """undirected R-MAT scale 22, edge factor 16, a/b/c/d = .57/.19/.19/.05 (seed
    8201), CSR int32, source 0. A step = one BFS to completion."""
    name = "bfs_rmat22_ef16"
    unit = "GTEPS"
    dtype = "int32"
    cpu_parallel = False

    def __init__(self):
        from l2domain_amd.bfs import RMAT_EDGE_FACTOR, RMAT_SCALE, RMAT_SEED, Graph, rmat_csr
        t0 = time.perf_counter()
        self.rowptr, self.col = rmat_csr(RMAT_SCALE, RMAT_EDGE_FACTOR, RMAT_SEED)
        self.gen_s = time.perf_counter() - t0
        self.g = Graph(self.rowptr, self.col)
        self.stats = None
        self.step("aware")
        V = self.g.V
        # CSR read once + level written once per search: 4(V+1) + 4 nnz_reached + 4V
        self.roof_bytes = 4 * (V + 1) + 4 * self.stats["reached_edges"] + 4 * V

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

    def roof_kernels(self, mode):
        return ("bfs_init_kernel", "bfs_level_kernel", "bfs_hubs_kernel")

    def config(self):
        return {"workload": self.name, "vertices": self.g.V, "nnz": self.g.nnz, "source": 0, "seed": 8201,
                "levels": self.stats["levels"] if self.stats else None,
                "reached_edges": self.stats["reached_edges"] if self.stats else None,
                "host_generation_s": round(self.gen_s, 2)}

    def cpu_baseline(self, nt, budget_s):
        import oracle as ora
        dt, reps = timed_loop(lambda: ora.bfs(self.rowptr, self.col, 0), budget_s)
        return self.stats["reached_edges"] / 2 / dt / 1e9, f"{reps} serial queue BFS runs of the same graph (oracle)"


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
# every other configuration, reported under "configs" of the same JSON line: (name, cold)
EXTRAS = (("gemv_f32", False), ("gemv_f32", True), ("gemv_f16_up", False), ("gemv_f16_up", True),
          ("gemv_f16_down", False), ("gemv_f16_down", True), ("hash", False), ("bfs", False),
          ("hash_dep", False), ("hist256", True), ("hist256", False), ("bfs_ref", False))


# ---------------------------------------------------------------------------------------
# Timing
# ---------------------------------------------------------------------------------------
def time_steps(wl, mode, steps, warmup, flusher=None):
    """Seconds per step over exactly `steps` steps, HIP events on the launch stream. Cold:
    a flush before every step, each step timed by its own event pair."""
    import torch
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        if flusher is not None:
            flusher.flush()
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
    """{kernel: (seconds per step, launches per step)} from the dispatch-stamped events."""
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
    t.pop("cache_flush_kernel", None)
    return {k: (ms / 1e3 / steps, n / steps) for k, (ms, n) in t.items()}


def stream_sweep(wl, steps, flusher=None):
    """Read-stream throughput (GB/s) over the workload's own footprint, {"mode/workgroups/
    depth": GB/s}: a sweep of chunk order (oblivious: contiguous; aware: each die's workgroups
    read only the 8 KiB chunks homed on their die), workgroups and loads in flight, each point
    from the read kernel's own dispatch-stamped durations (as the roofline kernels are timed).
    With a flusher, the L2s and the Infinity Cache are flushed before every timed read (cold,
    from HBM); without, one untimed pass first (warm)."""
    import torch
    from l2domain_amd import _lib
    from l2domain_amd.domain import home_map, read_stream
    buf = wl.roof_footprint()
    home = getattr(wl, "home", None)
    if home is None:
        home = home_map(buf.view(torch.uint8))
    nbytes = buf.numel() * buf.element_size()
    res = {}
    for mode in ("oblivious", "aware"):
        for wgs in (512, 1024, 2048, 4096, 8192):
            for depth in (1, 2, 4, 8):
                if flusher is not None:
                    flusher.flush()
                read_stream(buf, mode, home, wgs, depth)
                torch.cuda.synchronize()
                _lib.timing_enable(True)
                for _ in range(steps):
                    if flusher is not None:
                        flusher.flush()
                    read_stream(buf, mode, home, wgs, depth)
                torch.cuda.synchronize()
                t = _lib.timing_read()
                _lib.timing_enable(False)
                ms, n = t["read_stream_kernel"]
                res[f"{mode}/{wgs}/{depth}"] = nbytes / (ms / 1e3 / n) / 1e9
    return res


def ic_peak(wl, steps):
    """Best warm read-stream throughput (GB/s) over the workload's own footprint: the
    Infinity-Cache roofline of a warm run of that footprint."""
    res = stream_sweep(wl, steps)
    best = max(res, key=res.get)
    return res[best], {"best": best, **{k: round(v, 1) for k, v in res.items()}}


def run_workload(name, steps, warmup, cold=False, modes=MODES, cpu=True, cpu_budget=2.0, verify=True):
    import torch
    from l2domain_amd.domain import CacheFlusher
    wl = WORKLOADS[name]()
    steps = max(steps, wl.min_steps)
    ok = wl.verify() if verify else None
    flusher = CacheFlusher() if cold else None
    # The first ~30 steps of a process run up to 20 % slower than the steady state, and so do
    # the first milliseconds after the GPU idled (the CPU check above runs for seconds): every
    # mode is warmed up together, for at least 0.3 s of steps, so that the mode timed first
    # (oblivious) is out of that phase. (With 10 rounds only, the 90 us byte-histogram step
    # timed 97.8 us by events against 87.6 us of kernel for the first mode, and agreed within
    # 2 % for the others.)
    t_warm = time.perf_counter()
    rounds = 0
    while rounds < max(warmup, 10) or time.perf_counter() - t_warm < 0.3:
        for m in modes:
            if flusher is not None:
                flusher.flush()
            wl.step(m)
        rounds += 1
        if rounds % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    sec = {m: time_steps(wl, m, steps, warmup, flusher) for m in modes}
    torch.cuda.synchronize()
    kt = {m: kernel_times(wl, m, steps, flusher) for m in modes}
    roof_s = {m: sum(v[0] for k, v in kt[m].items() if k in wl.roof_kernels(m)) for m in modes}
    # Throughput from the event pair around each step, cold ones included: after the flush, an
    # event, the step's launches, an event (as the reference times a cold call,
    # gemv_cublas_benchmark.cu:84-90), so a step of two launches pays the gap between them.
    # The kernels' own summed durations stay in the detail (ms_per_step_kernels).
    tput_s = sec
    out = {"workload": wl, "verified": ok, "sec": sec, "tput_s": tput_s, "roof_s": roof_s, "kernels": kt,
           "tput": {m: wl.throughput(tput_s[m]) for m in modes}, "steps": steps}
    if not cold and wl.ic_resident:
        out["ic_peak"] = ic_peak(wl, steps)
    if cpu:
        nt = cpu_threads()
        v1, s1 = wl.cpu_baseline(1, cpu_budget)
        cb = {"value_1thread": round(v1, 4), "sample": s1, "kind": "port"}
        if wl.cpu_parallel and nt > 1:
            vn, _ = wl.cpu_baseline(nt, cpu_budget)
            cb.update(value=round(vn, 4), cores=nt)
        else:
            cb.update(value=round(v1, 4), cores=1)
        cb["unit"] = wl.unit
        out["cpu"] = cb
    return out


def roofline(r, mode="aware", cold=False):
    wl = r["workload"]
    sec = r["roof_s"][mode]
    achieved = wl.roof_bytes / sec / 1e9 if sec > 0 else 0.0
    if "ic_peak" in r:
        bound, peak = "infinity_cache", r["ic_peak"][0]
    else:
        bound, peak = "hbm", HBM_PEAK_GBS
    name = getattr(wl, "name", "")
    traffic = TRAFFIC.get((name, "cold" if cold else "warm", mode))
    out = {"bound": bound, "achieved": round(achieved, 1), "peak": round(peak, 1), "unit": "GB/s",
           "frac": round(achieved / peak, 4), "traffic": traffic,
           "traffic_src": TRAFFIC_SRC if traffic is not None else None,
           "kernel": "+".join(k for k in r["kernels"][mode] if k in wl.roof_kernels(mode)),
           "kernel_us": round(sec * 1e6, 3), "bytes": wl.roof_bytes}
    if getattr(wl, "roof_basis", None):
        out["bytes_basis"] = wl.roof_basis
    return out


def compact(r, cold):
    """One short entry per configuration (the driver keeps only the tail of the line)."""
    t = r["tput"]
    e = {"ok": r["verified"], "unit": r["workload"].unit, "steps": r["steps"]}
    for m, k in (("aware", "aware"), ("oblivious", "obl"), ("rotated", "rot")):
        if m in t:
            e[k] = round(t[m], 2)
    if "oblivious" in t and "aware" in t:
        e["sp"] = round(r["tput_s"]["oblivious"] / r["tput_s"]["aware"], 4)
    if "oblivious" in t and "rotated" in t:
        e["sp_rot"] = round(r["tput_s"]["oblivious"] / r["tput_s"]["rotated"], 4)
    if "aware" in t:
        ro = roofline(r, "aware", cold)
        e["roof"] = {k: ro[k] for k in ("bound", "achieved", "peak", "frac", "traffic", "kernel_us")}
    if "cpu" in r:
        c = r["cpu"]
        e["cpu"] = {"v": c["value"], "v1": c["value_1thread"], "cores": c["cores"]}
    return e


def detail(r, cold):
    d = {"verified": r["verified"], "cache": "cold" if cold else "warm", "config": r["workload"].config(),
         "ms_per_step_events": {m: round(s * 1e3, 6) for m, s in r["sec"].items()},
         "ms_per_step_kernels": {m: round(sum(v[0] for v in kk.values()) * 1e3, 6) for m, kk in r["kernels"].items()},
         "kernels_us_per_step": {m: {k: [round(v[0] * 1e6, 3), v[1]] for k, v in kk.items()}
                                 for m, kk in r["kernels"].items()},
         "roofline_by_mode": {m: roofline(r, m, cold) for m in r["kernels"]}}
    if "ic_peak" in r:
        d["ic_peak_gbs"] = r["ic_peak"][1]
    if "cpu" in r:
        d["cpu_baseline"] = r["cpu"]
    return d


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    ap.add_argument("--cold", action="store_true", help="flush L2 + Infinity Cache before every step")
    ap.add_argument("--only", action="store_true", help="measure the selected workload only (no other configs)")
    ap.add_argument("--modes", default=",".join(MODES), help="comma list of modes to time (default: all three)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--detail", default=None, help="write per-kernel, per-mode detail to this JSON file")
    ap.add_argument("--no-verify", action="store_true",
                    help="skip the oracle check (profiling runs only; the line then says verified: null)")
    ap.add_argument("--stream-sweep", action="store_true",
                    help="print the read-stream sweep over the workload's footprint (GEMV workloads; "
                         "--cold: from HBM) instead of a bench line")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one MI355X only (one-GPU tier); "
              f"--gpus {args.gpus} / WORLD_SIZE={world} is not supported", file=sys.stderr)
        sys.exit(2)
    modes = tuple(m for m in MODES if m in args.modes.split(","))
    if not modes:
        print("bench.py: --modes names none of oblivious, aware, rotated", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        sys.exit(1)
    from l2domain_amd.domain import topology

    if args.stream_sweep:
        from l2domain_amd.domain import CacheFlusher
        wl = WORKLOADS[args.workload]()
        if wl.roof_footprint() is None:
            print(f"bench.py: {args.workload} has no read-stream footprint", file=sys.stderr)
            sys.exit(2)
        res = stream_sweep(wl, args.steps, CacheFlusher() if args.cold else None)
        best = {m: max((k for k in res if k.startswith(m + "/")), key=res.get) for m in ("oblivious", "aware")}
        print(json.dumps({"workload": wl.name, "cache": "cold" if args.cold else "warm", "steps": args.steps,
                          "best": {m: [k, round(res[k], 1)] for m, k in best.items()},
                          "points": {k: round(v, 1) for k, v in res.items()}}))
        return

    r = run_workload(args.workload, args.steps, args.warmup, cold=args.cold, modes=modes, cpu=not args.no_cpu,
                     cpu_budget=10.0, verify=not args.no_verify)
    wl = r["workload"]
    head = "aware" if "aware" in modes else modes[0]
    sec = r["tput_s"][head]
    line = {
        "metric": METRIC,
        "value": round(r["tput"][head], 3),
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype,
        "data": "synthetic (seeded generators, inputs resident in HBM)",
        "config": dict(wl.config(), cache="cold" if args.cold else "warm", mode=head),
        "verified": r["verified"],
    }
    if "oblivious" in modes and "aware" in modes:
        line["speedup_aware_vs_oblivious"] = round(r["tput_s"]["oblivious"] / r["tput_s"]["aware"], 4)
    if "oblivious" in modes and "rotated" in modes:
        line["speedup_rotated_vs_oblivious"] = round(r["tput_s"]["oblivious"] / r["tput_s"]["rotated"], 4)
    line["modes"] = {m: round(v, 3) for m, v in r["tput"].items()}
    line["roofline"] = roofline(r, head, args.cold)
    if getattr(wl, "bytes", 0) and wl.bytes != wl.roof_bytes:
        # the whole step against the same peak: every algorithmic byte over the step's time
        st = wl.bytes / sec / 1e9
        line["roofline"]["step"] = {"bytes": wl.bytes, "achieved": round(st, 1),
                                    "frac": round(st / line["roofline"]["peak"], 4)}
    line["cpu_baseline"] = r.get("cpu")
    details = {f"{args.workload}_{'cold' if args.cold else 'warm'}": detail(r, args.cold)}
    if not args.only:
        configs = {}
        esteps = min(args.steps, 50)
        for name, cold in EXTRAS:
            if name == args.workload and cold == args.cold:
                continue
            key = f"{name}_{'cold' if cold else 'warm'}"
            print(f"bench: {key}", file=sys.stderr, flush=True)
            e = run_workload(name, esteps, min(args.warmup, 5), cold=cold, modes=modes,
                             cpu=not args.no_cpu and not cold, verify=not args.no_verify)
            configs[key] = compact(e, cold)
            details[key] = detail(e, cold)
            del e
            torch.cuda.empty_cache()
        line["configs"] = configs
    line["device"] = topology(0)["name"]
    if args.detail:
        Path(args.detail).parent.mkdir(parents=True, exist_ok=True)
        Path(args.detail).write_text(json.dumps(details, indent=1))
    print(json.dumps(line, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
