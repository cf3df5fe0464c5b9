// Histogram runner: the command line, stdout lines and exit status of the reference's
// histogram benchmark (applications/histogram/src/histogram256_sideaware.cu:309-560, parsed
// by applications/histogram/run.sh:54-90), on libxdom's histograms.
//
//   xd_hist_run [data_mb=256] [runs=10] [threads=256] [blocks_per_sm=1] [cache_mode=1] [--csv=FILE]
//   xd_hist_run --workload=zipf [data_mb runs threads blocks_per_sm cache_mode] [bins=1048576]
//               [zipf_s=1.1] [seed=1373] [--csv=FILE]
//
// Default workload: the reference's own -- data_mb MiB of words[i] = mix32(i) (:331-340),
// every byte counted into 256 bins (xd_hist256_u32bytes). --workload=zipf: data_mb MiB of
// uint32 keys, Zipf(zipf_s) ranks over `bins` bins through the scrambled rank -> bin map
// (xd_gen_zipf_keys), one bin per key (xd_hist_u32). cache_mode 1 = warm, 0 = cold (L2 and
// Infinity Cache evicted before each timed run). threads and blocks_per_sm are accepted and
// echoed: the launch shapes here are fixed by the kernels. "baseline" = XD_MODE_OBLIVIOUS;
// "persistent_aware" / "persistent_swapped" = XD_MODE_AWARE / XD_MODE_ROTATED. ROCm has no
// Green Contexts (the reference's green_* variants partition SMs into sides); the XCD
// dispatch is already partitioned, so the green_* lines report the same aware / rotated
// launches so that run.sh-style parsers keep working. Times cover the whole call (the
// merge included). Correctness: every mode's counts equal the runner's serial CPU count
// (HIST.cu:279-299) bit for bit; exit 3 otherwise.
#include "runner_common.hpp"

using namespace runner;

static const char *kCsvHeader =
    "gpu_label,gpu_index,data_mb,threads,blocks_per_sm,total_blocks,persistent_blocks,runs,cache_mode,"
    "baseline_kernel_ms,green_aware_kernel_ms,green_swapped_kernel_ms,persistent_aware_kernel_ms,"
    "persistent_swapped_kernel_ms,green_aware_kernel_speedup,green_swapped_kernel_speedup,"
    "persistent_aware_kernel_speedup,persistent_swapped_kernel_speedup,pass,bins,aware_gkeys_per_s,cpu_ms,"
    "workload,aware_gbps,roofline_frac";

// The reference's workload: 256 byte-bins of mix32(i) words.
static int run_bytes(const Options &o) {
    const int data_mb = (int)std::max<long long>(o.geti(0, 256), 1);
    const int runs = (int)std::max<long long>(o.geti(1, 10), 1);
    const int threads = (int)o.geti(2, 256);
    const int blocks_per_sm = (int)o.geti(3, 1);
    const int cache_mode = o.geti(4, 1) ? 1 : 0;
    const size_t n = (size_t)data_mb * (1u << 20) / 4;
    if (n >= (1ull << 30)) {
        fprintf(stderr, "data_mb must be < 4096\n");
        return 2;
    }
    const xd_topology_t topo = topology();
    hipStream_t s;
    RUN_HIP(hipStreamCreate(&s));
    std::vector<uint32_t> hw(n);
    RUN_XD(xd_gen_mix32_words(hw.data(), n, 0u));
    uint32_t *words = nullptr, *counts = nullptr;
    RUN_HIP(hipMalloc(&words, n * 4));
    RUN_HIP(hipMalloc(&counts, 256 * 4));
    RUN_HIP(hipMemcpy(words, hw.data(), n * 4, hipMemcpyHostToDevice));
    const size_t wsb = xd_hist256_workspace_size();
    void *ws = nullptr;
    RUN_HIP(hipMalloc(&ws, wsb));
    RUN_HIP(hipMemset(ws, 0, wsb));
    HomeMap home(words, n * 4, s);
    Flusher flush;

    // serial CPU count (the reference's compute_reference_hist, :279-288)
    std::vector<uint32_t> ref(256, 0u), got(256);
    const auto t0 = std::chrono::steady_clock::now();
    for (size_t i = 0; i < n; ++i) {
        const uint32_t w = hw[i];
        ++ref[w & 0xffu];
        ++ref[(w >> 8) & 0xffu];
        ++ref[(w >> 16) & 0xffu];
        ++ref[w >> 24];
    }
    const double cpu_ms = wall_ms(t0);
    auto launch = [&](int mode) { RUN_XD(xd_hist256_u32bytes(words, n, counts, mode, home.attr, ws, wsb, s)); };
    bool ok[3];
    for (int mode = 0; mode < 3; ++mode) {
        RUN_HIP(hipMemset(counts, 0xff, 256 * 4));
        launch(mode);
        RUN_HIP(hipMemcpy(got.data(), counts, 256 * 4, hipMemcpyDeviceToHost));
        ok[mode] = got == ref;
    }
    for (int w = 0; w < 5; ++w)
        for (int mode = 0; mode < 3; ++mode) launch(mode);
    double ms[3] = {0, 0, 0};
    for (int r = 0; r < runs; ++r)
        for (int mode = 0; mode < 3; ++mode) {
            if (!cache_mode) flush(s);
            ms[mode] += time_ms(s, [&] { launch(mode); });
        }
    for (double &m : ms) m /= runs;
    const char *P[2] = {"FAIL", "PASS"};
    const int pairs = (int)((n * 4 + 16383) / 16384);
    const int grid = std::min(512, std::max(8, (pairs + 7) / 8 * 8));

    printf("=== Histogram256 (XCD domains) ===\n");
    printf("data=%dMB words=%zu runs=%d threads=%d blocks_per_sm=%d cache_mode=%s baseline_blocks=%d "
           "persistent_blocks=%d side_blocks[%d,%d]\n",
           data_mb, n, runs, threads, blocks_per_sm, cache_mode ? "warm" : "cold", grid, grid, grid / 2, grid / 2);
    printf("device_cus=%d xcds=%d cu_per_xcd=%d chunk_bytes=8192 home=measured\n\n", topo.num_cu, topo.num_xcd,
           topo.cu_per_xcd);
    printf("correct baseline=%s green_aware=%s green_swapped=%s persistent_aware=%s persistent_swapped=%s\n\n", P[ok[0]],
           P[ok[1]], P[ok[2]], P[ok[1]], P[ok[2]]);
    printf("baseline_kernel_ms %.6f ms\n", ms[0]);
    printf("green_aware_kernel_ms %.6f ms kernel_speedup_vs_baseline=%.3fx\n", ms[1], ms[0] / ms[1]);
    printf("green_swapped_kernel_ms %.6f ms kernel_speedup_vs_baseline=%.3fx\n", ms[2], ms[0] / ms[2]);
    printf("persistent_aware_kernel_ms %.6f ms kernel_speedup_vs_baseline=%.3fx\n", ms[1], ms[0] / ms[1]);
    printf("persistent_swapped_kernel_ms %.6f ms kernel_speedup_vs_baseline=%.3fx\n", ms[2], ms[0] / ms[2]);
    const double bytes = 4.0 * n + 4.0 * 256;
    printf("gbps baseline=%.1f aware=%.1f swapped=%.1f\n", bytes / (ms[0] * 1e6), bytes / (ms[1] * 1e6),
           bytes / (ms[2] * 1e6));
    printf("roofline=hbm roofline_frac=%.4f peak_gbps=8000\n", bytes / (ms[1] * 1e6) / 8000.0);
    printf("cpu_ms=%.3f cpu_threads=1\n", cpu_ms);

    const bool pass = ok[0] && ok[1] && ok[2];
    char row[640];
    snprintf(row, sizeof row,
             "%s,0,%d,%d,%d,%d,%d,%d,%d,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%s,256,%.3f,%.3f,bytes256,%.1f,%.4f",
             topo.name, data_mb, threads, blocks_per_sm, grid, grid, runs, cache_mode, ms[0], ms[1], ms[2], ms[1], ms[2],
             ms[0] / ms[1], ms[0] / ms[2], ms[0] / ms[1], ms[0] / ms[2], pass ? "PASS" : "FAIL", n / (ms[1] * 1e6),
             cpu_ms, bytes / (ms[1] * 1e6), bytes / (ms[1] * 1e6) / 8000.0);
    csv_append(o.csv, kCsvHeader, row);
    (void)hipFree(words);
    (void)hipFree(counts);
    (void)hipFree(ws);
    return pass ? 0 : 3;
}

static int run_zipf(const Options &o) {
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
    HomeMap home(keys, n * 4, s);  // the aware mode reads the key chunks each die homes
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
        RUN_XD(xd_hist_u32(keys, n, counts, bins, mode, home.attr, ws, wsb, s));
        RUN_HIP(hipMemcpy(got.data(), counts, (size_t)bins * 4, hipMemcpyDeviceToHost));
        ok[mode] = got == ref;
    }
    for (int mode = 0; mode < 3; ++mode)
        for (int w = 0; w < 3; ++w) RUN_XD(xd_hist_u32(keys, n, counts, bins, mode, home.attr, ws, wsb, s));
    double ms[3] = {0, 0, 0};
    for (int r = 0; r < runs; ++r)
        for (int mode = 0; mode < 3; ++mode) {
            if (!cache_mode) flush(s);
            ms[mode] += time_ms(s, [&] { RUN_XD(xd_hist_u32(keys, n, counts, bins, mode, home.attr, ws, wsb, s)); });
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
    char row[640];
    snprintf(row, sizeof row,
             "%s,0,%d,%d,%d,%d,%d,%d,%d,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%.6f,%s,%u,%.3f,%.3f,zipf,%.1f,%.4f",
             topo.name, data_mb, threads, blocks_per_sm, (int)((n + 16383) / 16384), topo.num_cu, runs, cache_mode, ms[0],
             ms[1], ms[2], ms[1], ms[2], ms[0] / ms[1], ms[0] / ms[2], ms[0] / ms[1], ms[0] / ms[2], pass ? "PASS" : "FAIL",
             bins, n / (ms[1] * 1e6), cpu_ms, bytes / (ms[1] * 1e6), bytes / (ms[1] * 1e6) / 8000.0);
    csv_append(o.csv, kCsvHeader, row);
    (void)hipFree(dthr);
    (void)hipFree(keys);
    (void)hipFree(counts);
    (void)hipFree(ws);
    return pass ? 0 : 3;
}

int main(int argc, char **argv) {
    Options o(argc, argv);
    const std::string workload = o.opt("workload", "bytes");
    if (o.help || (workload != "bytes" && workload != "zipf")) {
        printf("usage: %s [--workload=bytes|zipf] [data_mb=256] [runs=10] [threads=256] [blocks_per_sm=1] "
               "[cache_mode=1] [bins=1048576 zipf_s=1.1 seed=1373 (zipf only)] [--csv=FILE]\n",
               argv[0]);
        return o.help ? 0 : 2;
    }
    return workload == "bytes" ? run_bytes(o) : run_zipf(o);
}
