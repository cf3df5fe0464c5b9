// Hash runner: the command line, stdout lines and exit status of the reference's hash
// benchmark (applications/hash/src/hash_probe_dep.cu:118-385, parsed by
// applications/hash/run.sh:55-90), on libxdom's uint64 linear-probing table.
//
//   xd_hash_run [K Q C L h H runs] [--csv=FILE]     (no positional arguments, or all seven)
//
// K keys (xd_gen_hash_kv, seed 42) are inserted into a table of C slots (C a power of
// two), then Q lookups run (xd_gen_hash_queries, qseed 4242: even queries hit, odd ones
// miss). Defaults are the build's benchmark configuration: K = 2^26, Q = 2^26, C = 2^27.
// L (dependent chain length), h (hot-query percent) and H (hot keys per side) shape the
// reference's dependent-probe workload and are accepted and echoed only. A timed run is
// clear + insert + lookup. "Persistent baseline" = XD_MODE_OBLIVIOUS, "Aware" =
// XD_MODE_AWARE (keys routed to the die homing their slot, with the table's measured home
// map), "Swapped" = XD_MODE_ROTATED. Correctness: every mode's found/value output equals
// the closed-form expectation of the generators (hit j: key index xd_rand64(qseed, j) mod K,
// value xd_rand64(42 ^ 0x5BD1E9955BD1E995, index); miss: 0/0) and the modes agree with each
// other (the reference checks GPU against GPU, :345-353); exit 1 otherwise, as the
// reference does (:384).
#include "runner_common.hpp"

using namespace runner;

int main(int argc, char **argv) {
    Options o(argc, argv);
    if (o.help || (o.pos.size() != 0 && o.pos.size() != 7)) {
        fprintf(stderr, "Usage: %s K Q C L h H runs [--csv=FILE]\n", argv[0]);
        return o.help ? 0 : 2;
    }
    const uint64_t K = (uint64_t)o.geti(0, 1ll << 26);
    const uint64_t Q = (uint64_t)o.geti(1, 1ll << 26);
    const uint64_t C = (uint64_t)o.geti(2, 1ll << 27);
    const int L = (int)o.geti(3, 1), h = (int)o.geti(4, 50), H = (int)o.geti(5, 0);
    const int runs = (int)std::max<long long>(o.geti(6, 7), 1);
    if (K == 0 || Q == 0 || K >= (1ull << 32) || Q >= (1ull << 32) || C < 2 || (C & (C - 1)) || K >= C) {
        fprintf(stderr, "need 0 < K < C, 0 < Q < 2^32, C a power of two\n");
        return 2;
    }
    const uint64_t seed = 42, qseed = 4242;
    const xd_topology_t topo = topology();
    hipStream_t s;
    RUN_HIP(hipStreamCreate(&s));
    uint64_t *keys, *vals, *q, *vout[3];
    uint8_t *fout[3];
    unsigned long long *failed;
    void *table;
    RUN_HIP(hipMalloc(&keys, K * 8));
    RUN_HIP(hipMalloc(&vals, K * 8));
    RUN_HIP(hipMalloc(&q, Q * 8));
    for (int m = 0; m < 3; ++m) {
        RUN_HIP(hipMalloc(&vout[m], Q * 8));
        RUN_HIP(hipMalloc(&fout[m], Q));
    }
    RUN_HIP(hipMalloc(&failed, 8));
    RUN_HIP(hipMalloc(&table, xd_hash_table_bytes(C)));
    RUN_XD(xd_gen_hash_kv(keys, vals, K, seed, s));
    RUN_XD(xd_gen_hash_queries(q, Q, K, seed, qseed, s));
    HomeMap home(table, xd_hash_table_bytes(C), s);

    auto step = [&](int mode, float *ins_ms, float *look_ms) {
        RUN_XD(xd_hash_init(table, C, s));
        const float a = time_ms(s, [&] { RUN_XD(xd_hash_insert_u64(table, C, keys, vals, K, mode, home.attr, failed, s)); });
        const float b = time_ms(s, [&] {
            RUN_XD(xd_hash_lookup_u64(table, C, q, Q, vout[mode], fout[mode], mode, home.attr, s));
        });
        if (ins_ms) *ins_ms += a;
        if (look_ms) *look_ms += b;
    };
    RUN_HIP(hipMemset(failed, 0, 8));
    for (int mode = 0; mode < 3; ++mode) step(mode, nullptr, nullptr);
    RUN_HIP(hipStreamSynchronize(s));
    unsigned long long hfail = 0;
    RUN_HIP(hipMemcpy(&hfail, failed, 8, hipMemcpyDeviceToHost));

    // closed-form expectation of the seeded inputs
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<uint64_t> ev(Q);
    std::vector<uint8_t> ef(Q);
    for (uint64_t j = 0; j < Q; ++j) {
        if (j & 1) {
            ev[j] = 0;
            ef[j] = 0;
        } else {
            const uint64_t idx = xd_rand64(qseed, j) % K;
            ev[j] = xd_rand64(seed ^ 0x5BD1E9955BD1E995ull, idx);
            ef[j] = 1;
        }
    }
    const double cpu_ms = wall_ms(t0);
    bool pass = hfail == 0;
    std::vector<uint64_t> gv(Q);
    std::vector<uint8_t> gf(Q);
    for (int mode = 0; mode < 3; ++mode) {
        RUN_HIP(hipMemcpy(gv.data(), vout[mode], Q * 8, hipMemcpyDeviceToHost));
        RUN_HIP(hipMemcpy(gf.data(), fout[mode], Q, hipMemcpyDeviceToHost));
        pass = pass && gv == ev && gf == ef;
    }
    printf("K=%llu Q=%llu C=%llu L=%d h=%d H=%d runs=%d gpu=%s xcds=%d load=%.4f insert_failures=%llu\n",
           (unsigned long long)K, (unsigned long long)Q, (unsigned long long)C, L, h, H, runs, topo.name, topo.num_xcd,
           (double)K / C, hfail);
    printf("Correctness: %s\n\n", pass ? "PASS" : "FAIL");

    float ins[3] = {0, 0, 0}, look[3] = {0, 0, 0};
    for (int r = 0; r < runs; ++r)
        for (int mode = 0; mode < 3; ++mode) step(mode, &ins[mode], &look[mode]);
    double ms[3];
    for (int m = 0; m < 3; ++m) {
        ins[m] /= runs;
        look[m] /= runs;
        ms[m] = (double)ins[m] + look[m];
    }
    printf("%-28s %8.3f ms\n", "Persistent baseline", ms[0]);
    printf("%-28s %8.3f ms  (speedup %.2fx)\n", "Aware", ms[1], ms[0] / ms[1]);
    printf("%-28s %8.3f ms  (speedup %.2fx)\n", "Swapped", ms[2], ms[0] / ms[2]);
    printf("insert_ms baseline=%.6f aware=%.6f swapped=%.6f\n", ins[0], ins[1], ins[2]);
    printf("lookup_ms baseline=%.6f aware=%.6f swapped=%.6f\n", look[0], look[1], look[2]);
    printf("mops baseline=%.1f aware=%.1f swapped=%.1f\n", (K + Q) / (ms[0] * 1e3), (K + Q) / (ms[1] * 1e3),
           (K + Q) / (ms[2] * 1e3));
    const double lbytes = 33.0 * Q;
    printf("roofline=hbm lookup_roofline_frac=%.4f peak_gbps=8000\n", lbytes / (look[1] * 1e6) / 8000.0);
    printf("cpu_ms=%.3f cpu_threads=1\n", cpu_ms);
    printf("RESULT baseline_ms=%.6f aware_ms=%.6f swapped_ms=%.6f aware_speedup=%.6f swapped_speedup=%.6f pass=%s\n",
           ms[0], ms[1], ms[2], ms[0] / ms[1], ms[0] / ms[2], pass ? "PASS" : "FAIL");
    char row[512];
    snprintf(row, sizeof row, "%llu,%llu,%llu,%.6f,%d,%d,%d,%.6f,%.6f,%.6f,%.6f,%.6f,%s,%.6f,%.6f,%.6f,%.6f",
             (unsigned long long)K, (unsigned long long)Q, (unsigned long long)C, 100.0 * K / C, L, h, H, ms[0], ms[1],
             ms[2], ms[0] / ms[1], ms[0] / ms[2], pass ? "PASS" : "FAIL", ins[0], ins[1], look[0], look[1]);
    csv_append(o.csv,
               "K,Q,C,effective_load,L,h,H,baseline_ms,aware_ms,swapped_ms,aware_speedup,swapped_speedup,pass,"
               "baseline_insert_ms,aware_insert_ms,baseline_lookup_ms,aware_lookup_ms",
               row);
    return pass ? 0 : 1;
}
