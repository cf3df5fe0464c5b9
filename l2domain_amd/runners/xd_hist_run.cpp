// Histogram runner: the command line, stdout lines and exit status of the reference's
// histogram benchmark (applications/histogram/src/histogram256_sideaware.cu:309-560, parsed
// by applications/histogram/run.sh:54-90), on libxdom's large-bin histogram.
//
//   xd_hist_run [data_mb=256] [runs=10] [threads=256] [blocks_per_sm=1] [cache_mode=1]
//               [bins=1048576] [zipf_s=1.1] [seed=1373] [--csv=FILE]
//
// data_mb MiB of uint32 keys, Zipf(zipf_s) ranks over `bins` bins through the scrambled
// rank -> bin map (xd_gen_zipf_keys); cache_mode 1 = warm, 0 = cold (L2 + Infinity Cache
// evicted before each timed run). threads and blocks_per_sm are accepted and echoed: the
// launch shapes here are fixed by the kernels (1024-thread partition and count workgroups).
// "baseline" = XD_MODE_OBLIVIOUS; "persistent_aware" / "persistent_swapped" =
// XD_MODE_AWARE / XD_MODE_ROTATED. ROCm has no Green Contexts (the reference's green_*
// variants partition SMs into sides); the XCD dispatch is already partitioned, so the
// green_* lines report the same aware / rotated launches so that run.sh-style parsers keep
// working. Correctness: every mode's counts equal the runner's serial CPU count
// (HIST.cu:279-299) bit for bit; exit 3 otherwise.
#include "runner_common.hpp"

using namespace runner;

int main(int argc, char **argv) {
    Options o(argc, argv);
    if (o.help) {
        printf("usage: %s [data_mb=256] [runs=10] [threads=256] [blocks_per_sm=1] [cache_mode=1] [bins=1048576] "
               "[zipf_s=1.1] [seed=1373] [--csv=FILE]\n",
               argv[0]);
        return 0;
    }
    const int data_mb = (int)std::max<long long>(o.geti(0, 256), 1);
    const int runs = (int)std::max<long long>(o.geti(1, 10), 1);
    const int threads = (int)o.geti(2, 256);
    const int blocks_per_sm = (int)o.geti(3, 1);
    const int cache_mode = o.geti(4, 1) ? 1 : 0;
    const uint32_t bins = (uint32_t)o.geti(5, 1 << 20);
    const double zs = o.getd(6, 1.1);
    const uint64_t seed = (uint64_t)o.geti(7, 1373);
    const size_t n = (size_t)data_mb * (1u << 20) / 4;
    if (bins < 1 || bins > (1u << 24) || n >= (1ull << 32)) {
        fprintf(stderr, "bins must be in [1, 2^24] and data_mb < 16384\n");
        return 2;
    }
    const xd_topology_t topo = topology();
    hipStream_t s;
    RUN_HIP(hipStreamCreate(&s));

    std::vector<uint64_t> thr(bins);
    RUN_XD(xd_zipf_thresholds(thr.data(), bins, zs));
    uint64_t *dthr = nullptr;
    uint32_t *keys = nullptr, *counts = nullptr;
    RUN_HIP(hipMalloc(&dthr, (size_t)bins * 8));
    RUN_HIP(hipMalloc(&keys, n * 4));
    RUN_HIP(hipMalloc(&counts, (size_t)bins * 4));
    RUN_HIP(hipMemcpy(dthr, thr.data(), (size_t)bins * 8, hipMemcpyHostToDevice));
    RUN_XD(xd_gen_zipf_keys(keys, n, dthr, bins, seed, 1, s));
    const size_t wsb = xd_hist_workspace_size(n, bins);
    void *ws = nullptr;
    RUN_HIP(hipMalloc(&ws, wsb));
    RUN_HIP(hipMemset(ws, 0, wsb));
    Flusher flush;

    // serial CPU count (the reference's compute_reference_hist)
    std::vector<uint32_t> hk(n), ref(bins, 0u), got(bins);
    RUN_HIP(hipMemcpy(hk.data(), keys, n * 4, hipMemcpyDeviceToHost));
    const auto t0 = std::chrono::steady_clock::now();
    for (size_t i = 0; i < n; ++i)
        if (hk[i] < bins) ++ref[hk[i]];
    const double cpu_ms = wall_ms(t0);

    bool ok[3];
    for (int mode = 0; mode < 3; ++mode) {
        RUN_HIP(hipMemset(counts, 0xff, (size_t)bins * 4));
        RUN_XD(xd_hist_u32(keys, n, counts, bins, mode, ws, wsb, s));
        RUN_HIP(hipMemcpy(got.data(), counts, (size_t)bins * 4, hipMemcpyDeviceToHost));
        ok[mode] = got == ref;
    }
    for (int mode = 0; mode < 3; ++mode)
        for (int w = 0; w < 3; ++w) RUN_XD(xd_hist_u32(keys, n, counts, bins, mode, ws, wsb, s));
    double ms[3] = {0, 0, 0};
    for (int r = 0; r < runs; ++r)
        for (int mode = 0; mode < 3; ++mode) {
            if (!cache_mode) flush(s);
            ms[mode] += time_ms(s, [&] { RUN_XD(xd_hist_u32(keys, n, counts, bins, mode, ws, wsb, s)); });
        }
    for (double &m : ms) m /= runs;
    const char *P[2] = {"FAIL", "PASS"};

    printf("=== Histogram, %u bins (XCD domains) ===\n", bins);
    printf("data=%dMB words=%zu runs=%d threads=%d blocks_per_sm=%d cache_mode=%s baseline_blocks=%d "
           "persistent_blocks=%d side_blocks[%d,%d]\n",
           data_mb, n, runs, threads, blocks_per_sm, cache_mode ? "warm" : "cold", (int)((n + 16383) / 16384),
           topo.num_cu, topo.num_cu / 2, topo.num_cu / 2);
    printf("device_cus=%d xcds=%d cu_per_xcd=%d zipf_s=%.3f seed=%llu bins=%u\n\n", topo.num_cu, topo.num_xcd,
           topo.cu_per_xcd, zs, (unsigned long long)seed, bins);
    printf("correct baseline=%s green_aware=%s green_swapped=%s persistent_aware=%s persistent_swapped=%s\n\n", P[ok[0]],
           P[ok[1]], P[ok[2]], P[ok[1]], P[ok[2]]);
    printf("baseline_kernel_ms %.6f ms\n", ms[0]);
    printf("green_aware_kernel_ms %.6f ms kernel_speedup_vs_baseline=%.3fx\n", ms[1], ms[0] / ms[1]);
    printf("green_swapped_kernel_ms %.6f ms kernel_speedup_vs_baseline=%.3fx\n", ms[2], ms[0] / ms[2]);
    printf("persistent_aware_kernel_ms %.6f ms kernel_speedup_vs_baseline=%.3fx\n", ms[1], ms[0] / ms[1]);
    printf("persistent_swapped_kernel_ms %.6f ms kernel_speedup_vs_baseline=%.3fx\n", ms[2], ms[0] / ms[2]);
    const double bytes = 4.0 * n + 4.0 * bins;
    printf("gkeys_per_s baseline=%.2f aware=%.2f swapped=%.2f\n", n / (ms[0] * 1e6), n / (ms[1] * 1e6),
           n / (ms[2] * 1e6));
    printf("roofline=hbm roofline_frac=%.4f peak_gbps=8000\n", bytes / (ms[1] * 1e6) / 8000.0);
    printf("cpu_ms=%.3f cpu_threads=1\n", cpu_ms);

    const bool pass = ok[0] && ok[1] && ok[2];
    char row[512];
    snprintf(row, sizeof row, "%s,0,%d,%d,%d,%d,%d,%d,%d,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%s,%u,%.3f,%.3f",
             topo.name, data_mb, threads, blocks_per_sm, (int)((n + 16383) / 16384), topo.num_cu, runs, cache_mode, ms[0],
             ms[1], ms[2], ms[1], ms[2], ms[0] / ms[1], ms[0] / ms[2], ms[0] / ms[1], ms[0] / ms[2], pass ? "PASS" : "FAIL",
             bins, n / (ms[1] * 1e6), cpu_ms);
    csv_append(o.csv,
               "gpu_label,gpu_index,data_mb,threads,blocks_per_sm,total_blocks,persistent_blocks,runs,cache_mode,"
               "baseline_kernel_ms,green_aware_kernel_ms,green_swapped_kernel_ms,persistent_aware_kernel_ms,"
               "persistent_swapped_kernel_ms,green_aware_kernel_speedup,green_swapped_kernel_speedup,"
               "persistent_aware_kernel_speedup,persistent_swapped_kernel_speedup,pass,bins,aware_gkeys_per_s,cpu_ms",
               row);
    (void)hipFree(dthr);
    (void)hipFree(keys);
    (void)hipFree(counts);
    (void)hipFree(ws);
    return pass ? 0 : 3;
}
