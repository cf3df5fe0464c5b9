// Hash runner: the command line, stdout lines and exit status of the reference's hash
// benchmark (applications/hash/src/hash_probe_dep.cu:118-385, parsed by
// applications/hash/run.sh:55-90).
//
//   xd_hash_run [K Q C L h H runs] [--csv=FILE]                          (reference workload)
//   xd_hash_run --workload=insert_lookup [K Q C L h H runs] [--csv=FILE] (uint64 table)
//
// No positional arguments, or all seven (:119-122). The default workload is the reference's
// own: K int32 keys with successors in a table of C 8-byte entries, two hot pools of H keys
// homed on opposite I/O dies and chained into cycles, Q queries of which h percent alternate
// the hot pools, each following its chain for L dependent probes (xd_dep_*; defaults K =
// 32000000, Q = 8000000, C = 2^26, L = 4, h = 80, H = 100000, runs = 7 as in :124-130).
// "Persistent baseline" = XD_MODE_OBLIVIOUS (probe_dep_base), "Aware" / "Swapped" = the routed
// probe (probe_dep_sa) over the per-die query lists, each die probing its own / the other
// die's list. As in the reference, the lists are built before the timed runs (the reference
// builds them on the host, :244-270); here xd_dep_route builds them on the device and its
// time is reported on its own line (route_ms), with the aware time including it and the
// single-call XD_MODE_AWARE of xd_dep_probe (routing inside the probe kernel).
// Correctness as in the reference: the outputs agree (:345-353); exit 1 otherwise.
//
// --workload=insert_lookup: the build's insert + lookup configuration on the uint64 table.
// K keys (xd_gen_hash_kv, seed 42) are inserted into a table of C slots (C a power of
// two), then Q lookups run (xd_gen_hash_queries, qseed 4242: even queries hit, odd ones
// miss). Defaults: K = 2^26, Q = 2^26, C = 2^27; L, h and H are echoed only. A timed run is
// clear + insert + lookup. "Persistent baseline" = XD_MODE_OBLIVIOUS, "Aware" =
// XD_MODE_AWARE (keys routed to the die homing their slot, with the table's measured home
// map), "Swapped" = XD_MODE_ROTATED. Correctness: every mode's found/value output equals
// the closed-form expectation of the generators (hit j: key index xd_rand64(qseed, j) mod K,
// value xd_rand64(42 ^ 0x5BD1E9955BD1E995, index); miss: 0/0) and the modes agree with each
// other (the reference checks GPU against GPU, :345-353); exit 1 otherwise, as the
// reference does (:384).
#include "runner_common.hpp"

using namespace runner;

static int dep_probe(const Options &o);
static int insert_lookup(const Options &o);

int main(int argc, char **argv) {
    Options o(argc, argv);
    const std::string workload = o.opt("workload", "dep");
    if (o.help || (o.pos.size() != 0 && o.pos.size() != 7) || (workload != "dep" && workload != "insert_lookup")) {
        fprintf(stderr, "Usage: %s [--workload=dep|insert_lookup] K Q C L h H runs [--csv=FILE]\n", argv[0]);
        return o.help ? 0 : 2;
    }
    return workload == "dep" ? dep_probe(o) : insert_lookup(o);
}

static int dep_probe(const Options &o) {
    const long long K = o.geti(0, 32000000), Q = o.geti(1, 8000000);
    const unsigned long long C = (unsigned long long)o.geti(2, 1ll << 26);
    const int L = (int)o.geti(3, 4), h = (int)o.geti(4, 80), H = (int)o.geti(5, 100000);
    const int runs = (int)o.geti(6, 7);
    if (K <= 0 || Q <= 0 || K > INT32_MAX || Q > INT32_MAX || C < 2 || (C & (C - 1)) || C > (1ull << 32) ||
        (unsigned long long)K >= C || L <= 0 || h < 0 || h > 100 || H <= 0 || 2LL * H > K || runs <= 0) {
        fprintf(stderr, "need 0 < K < C (a power of two), 0 < Q, L > 0, 0 <= h <= 100, 0 < 2H <= K, runs > 0\n");
        return 2;
    }
    const xd_topology_t topo = topology();
    hipStream_t s;
    RUN_HIP(hipStreamCreate(&s));
    const size_t tbytes = (size_t)C * 8;
    char *raw;
    RUN_HIP(hipMalloc(&raw, tbytes + (2u << 20)));
    int32_t *table = reinterpret_cast<int32_t *>(((uintptr_t)raw + (2u << 20) - 1) & ~(uintptr_t)((2u << 20) - 1));
    HomeMap home(table, tbytes, s);
    std::vector<uint8_t> attr(xd_home_map_pages(table, tbytes));
    RUN_HIP(hipMemcpy(attr.data(), home.attr, attr.size(), hipMemcpyDeviceToHost));
    std::vector<int32_t> keys((size_t)K), nexts((size_t)K), ht(2 * (size_t)C), q((size_t)Q);
    RUN_XD(xd_dep_make_keys(reinterpret_cast<uint64_t>(table), C, attr.data(), (int32_t)K, H, keys.data(), nexts.data()));
    RUN_XD(xd_dep_build(ht.data(), C, keys.data(), nexts.data(), (int32_t)K, 42));
    RUN_XD(xd_dep_queries(q.data(), (int32_t)Q, keys.data(), (int32_t)K, H, h, 4242));
    RUN_HIP(hipMemcpy(table, ht.data(), tbytes, hipMemcpyHostToDevice));
    // queries per home die of their first slot (the reference's aware_q0 / aware_q1)
    long long nq[2] = {0, 0};
    auto mix32 = [](uint32_t x) {
        x ^= x >> 16;
        x *= 0x7feb352du;
        x ^= x >> 15;
        x *= 0x846ca68bu;
        x ^= x >> 16;
        return x;
    };
    const uint64_t tb = reinterpret_cast<uint64_t>(table);
    for (long long i = 0; i < Q; ++i) {
        const uint64_t a = tb + (uint64_t)(mix32((uint32_t)q[i]) & (uint32_t)(C - 1)) * 8;
        nq[((a >> 13) & 1u) ^ attr[(a >> 21) - (tb >> 21)]]++;
    }
    int32_t *dq, *dout[3];
    RUN_HIP(hipMalloc(&dq, (size_t)Q * 4));
    for (auto &p : dout) RUN_HIP(hipMalloc(&p, (size_t)Q * 4));
    RUN_HIP(hipMemcpy(dq, q.data(), (size_t)Q * 4, hipMemcpyHostToDevice));

    printf("=== Dependent Hash Probe (XCD domains) ===\n");
    printf("CONFIG K=%lld Q=%lld C=%llu effective_load=%.6f L=%d h=%d H=%d runs=%d\n\n", K, Q, C, 100.0 * K / C, L, h, H,
           runs);
    printf("table=%.1f MiB chunks=%zu hot_chain_set_per_side=%.1f MiB aware_q0=%lld aware_q1=%lld gpu=%s\n\n",
           tbytes / 1048576.0, tbytes / 8192, H * 8.0 / 1048576.0, nq[0], nq[1], topo.name);
    const size_t rb = xd_dep_route_bytes((uint64_t)Q);
    void *route;
    RUN_HIP(hipMalloc(&route, rb));
    auto route_ms = [&] { return time_ms(s, [&] { RUN_XD(xd_dep_route(table, C, dq, (uint64_t)Q, home.attr, route, rb, s)); }); };
    route_ms();
    auto run = [&](int mode) {
        if (mode == 0)
            return time_ms(s, [&] { RUN_XD(xd_dep_probe(table, C, dq, (uint64_t)Q, L, dout[0], 0, home.attr, s)); });
        return time_ms(s, [&] { RUN_XD(xd_dep_probe_routed(table, C, route, (uint64_t)Q, L, dout[mode], mode, s)); });
    };
    auto run_fly = [&] {
        return time_ms(s, [&] { RUN_XD(xd_dep_probe(table, C, dq, (uint64_t)Q, L, dout[1], XD_MODE_AWARE, home.attr, s)); });
    };
    for (int mode = 0; mode < 3; ++mode) run(mode);
    std::vector<int32_t> r0((size_t)Q), r1((size_t)Q), r2((size_t)Q), r3((size_t)Q);
    RUN_HIP(hipMemcpy(r0.data(), dout[0], (size_t)Q * 4, hipMemcpyDeviceToHost));
    RUN_HIP(hipMemcpy(r1.data(), dout[1], (size_t)Q * 4, hipMemcpyDeviceToHost));
    RUN_HIP(hipMemcpy(r2.data(), dout[2], (size_t)Q * 4, hipMemcpyDeviceToHost));
    run_fly();
    RUN_HIP(hipMemcpy(r3.data(), dout[1], (size_t)Q * 4, hipMemcpyDeviceToHost));
    const bool pass = r0 == r1 && r0 == r2 && r0 == r3;
    printf("Correctness: %s\n\n", pass ? "PASS" : "FAIL");
    double tbm = 0, ta = 0, ts = 0, tr = 0, tf = 0;
    for (int r = 0; r < runs; ++r) {
        tbm += run(0);
        ta += run(1);
        ts += run(2);
        tr += route_ms();
        tf += run_fly();
    }
    const double b = tbm / runs, a = ta / runs, w = ts / runs, rt = tr / runs, fl = tf / runs;
    printf("%-28s %8.3f ms\n", "Persistent baseline", b);
    printf("%-28s %8.3f ms  (speedup %.2fx)\n", "Aware", a, b / a);
    printf("%-28s %8.3f ms  (speedup %.2fx)\n", "Swapped", w, b / w);
    printf("route_ms=%.6f aware_incl_route_ms=%.6f aware_incl_route_speedup=%.3f aware_single_call_ms=%.6f "
           "aware_single_call_speedup=%.3f\n",
           rt, a + rt, b / (a + rt), fl, b / fl);
    printf("mprobes_per_s baseline=%.1f aware=%.1f swapped=%.1f\n", (double)Q * L / (b * 1e3), (double)Q * L / (a * 1e3),
           (double)Q * L / (w * 1e3));
    printf("RESULT baseline_ms=%.6f aware_ms=%.6f swapped_ms=%.6f aware_speedup=%.6f swapped_speedup=%.6f pass=%s\n", b, a,
           w, b / a, b / w, pass ? "PASS" : "FAIL");
    char row[512];
    snprintf(row, sizeof row, "%lld,%lld,%llu,%.6f,%d,%d,%d,%.6f,%.6f,%.6f,%.6f,%.6f,%s", K, Q, C, 100.0 * K / C, L, h, H,
             b, a, w, b / a, b / w, pass ? "PASS" : "FAIL");
    csv_append(o.csv, "K,Q,C,effective_load,L,h,H,baseline_ms,aware_ms,swapped_ms,aware_speedup,swapped_speedup,pass",
               row);
    for (auto p : dout) (void)hipFree(p);
    (void)hipFree(route);
    (void)hipFree(dq);
    (void)hipFree(raw);
    return pass ? 0 : 1;
}

static int insert_lookup(const Options &o) {
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
    const size_t ws_bytes = xd_hash_build_workspace_size(K, C);
    void *ws = nullptr;
    if (ws_bytes) RUN_HIP(hipMalloc(&ws, ws_bytes));
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

    // the bulk build (xd_hash_build_u64) in place of init + insert: the same lookups
    auto build = [&](int mode) {
        return time_ms(s, [&] {
            RUN_XD(xd_hash_build_u64(table, C, keys, vals, K, mode, home.attr, ws, ws_bytes, failed, s));
        });
    };
    bool bpass = true;
    for (int mode = 0; mode < 3; ++mode) {
        build(mode);
        RUN_XD(xd_hash_lookup_u64(table, C, q, Q, vout[mode], fout[mode], mode, home.attr, s));
        RUN_HIP(hipStreamSynchronize(s));
        RUN_HIP(hipMemcpy(gv.data(), vout[mode], Q * 8, hipMemcpyDeviceToHost));
        RUN_HIP(hipMemcpy(gf.data(), fout[mode], Q, hipMemcpyDeviceToHost));
        bpass = bpass && gv == ev && gf == ef;
    }
    RUN_HIP(hipMemcpy(&hfail, failed, 8, hipMemcpyDeviceToHost));
    bpass = bpass && hfail == 0;
    pass = pass && bpass;
    printf("Build correctness: %s\n", bpass ? "PASS" : "FAIL");

    float ins[3] = {0, 0, 0}, look[3] = {0, 0, 0}, bld[3] = {0, 0, 0};
    for (int r = 0; r < runs; ++r)
        for (int mode = 0; mode < 3; ++mode) {
            step(mode, &ins[mode], &look[mode]);
            bld[mode] += build(mode);
        }
    double ms[3];
    for (int m = 0; m < 3; ++m) {
        ins[m] /= runs;
        look[m] /= runs;
        bld[m] /= runs;
        ms[m] = (double)ins[m] + look[m];
    }
    printf("%-28s %8.3f ms\n", "Persistent baseline", ms[0]);
    printf("%-28s %8.3f ms  (speedup %.2fx)\n", "Aware", ms[1], ms[0] / ms[1]);
    printf("%-28s %8.3f ms  (speedup %.2fx)\n", "Swapped", ms[2], ms[0] / ms[2]);
    printf("insert_ms baseline=%.6f aware=%.6f swapped=%.6f\n", ins[0], ins[1], ins[2]);
    printf("lookup_ms baseline=%.6f aware=%.6f swapped=%.6f\n", look[0], look[1], look[2]);
    printf("build_ms baseline=%.6f aware=%.6f swapped=%.6f\n", bld[0], bld[1], bld[2]);
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
