// BFS runner: the command line, stdout lines and exit status of the reference's BFS
// benchmark (applications/bfs/src/bfs.cu:324-560, parsed by applications/bfs/run.sh:60-100).
//
//   xd_bfs_run [vertices=2000000] [degree=64] [sources=4096] [depth=4] [dst_local_pct=100]
//              [hot_per_side=200000] [runs=5] [seed=8201] [--sweep=NAME --value=V] [--csv=FILE]
//   xd_bfs_run --workload=rmat [vertices=2^22] [degree=32] [sources=1] [depth] [dst_local_pct]
//              [hot_per_side] [runs=5] [seed=8201] [--csv=FILE]
//
// Default workload: the reference's own (the same argument defaults and clamps, :329-343) --
// its directed hot-pool graph (xd_bfs_ref_graph, sides from the measured homes of this
// run's col and level buffers) searched from `sources` sources for `depth` top-down levels
// (xd_bfs_multi). "baseline" = XD_MODE_OBLIVIOUS, "aware" = XD_MODE_AWARE (per-die
// frontiers by work side), "swapped" = XD_MODE_ROTATED. Times are medians over `runs` of the
// whole search, initialisation included, as the reference times it (:510-533). visited =
// vertices the baseline reached; aware_bad / swapped_bad count levels that differ from the
// baseline's (diff_dist_kernel, :310-320); baseline_bad counts the baseline's differences
// from the runner's serial multi-source BFS. Exit 3 on any difference (:558), 2 when a hot
// pool cannot be filled (:374-377).
//
// --workload=rmat: the build's undirected R-MAT graph with 2^ceil(log2(vertices)) vertices
// and edge factor degree / 2, searched to completion from vertices 0, 1, ... (sources of
// them) by the direction-optimizing xd_bfs_csr; depth, dst_local_pct and hot_per_side are
// echoed only. In both workloads overflow is 0: these queues hold every vertex.
#include <math.h>

#include <queue>

#include "runner_common.hpp"

using namespace runner;

static const char *kCsvHeader =
    "sweep,value,gpu_label,gpu_index,vertices,degree,sources,depth,dst_local_pct,hot_per_side,runs,seed,"
    "visited,aware_bad,swapped_bad,overflow,baseline_med_ms,aware_med_ms,swapped_med_ms,aware_speedup,"
    "swapped_speedup,pass,workload,nnz,aware_gteps,baseline_bad";

static int run_rmat(const Options &o) {
    const long long vertices = std::max<long long>(o.geti(0, 1 << 22), 4096);
    const int degree = (int)std::max<long long>(o.geti(1, 32), 2);
    const int sources = (int)std::max<long long>(o.geti(2, 1), 1);
    const int depth = (int)o.geti(3, 0);
    const int dst_local = (int)o.geti(4, 100);
    const int hot = (int)o.geti(5, 0);
    const int runs = (int)std::max<long long>(o.geti(6, 5), 1);
    const uint64_t seed = (uint64_t)o.geti(7, 8201);
    int scale = 0;
    while ((1ll << scale) < vertices) ++scale;
    if (scale > 26) {
        fprintf(stderr, "vertices must be <= 2^26\n");
        return 2;
    }
    const int ef = std::max(1, degree / 2);
    const int32_t V = 1 << scale;
    const int nsrc = std::min<int>(sources, V);
    const xd_topology_t topo = topology();
    hipStream_t s;
    RUN_HIP(hipStreamCreate(&s));

    std::vector<int32_t> rowptr((size_t)V + 1), col((size_t)2 * ef * V);
    int64_t nnz = 0;
    RUN_XD(xd_rmat_csr(scale, ef, 0.57, 0.19, 0.19, seed, rowptr.data(), col.data(), (int64_t)col.size(), &nnz));
    int32_t *drow, *dcol;
    uint32_t *lvl[3];
    RUN_HIP(hipMalloc(&drow, rowptr.size() * 4));
    RUN_HIP(hipMalloc(&dcol, std::max<int64_t>(nnz, 1) * 4));
    RUN_HIP(hipMemcpy(drow, rowptr.data(), rowptr.size() * 4, hipMemcpyHostToDevice));
    if (nnz) RUN_HIP(hipMemcpy(dcol, col.data(), (size_t)nnz * 4, hipMemcpyHostToDevice));
    for (auto &p : lvl) RUN_HIP(hipMalloc(&p, (size_t)V * 4));
    const size_t wsb = xd_bfs_workspace_size(V, nnz);
    void *ws;
    RUN_HIP(hipMalloc(&ws, wsb));
    HomeMap home(dcol, (size_t)std::max<int64_t>(nnz, 1) * 4, s);
    void *route;  // per-die block lists, built once per graph
    RUN_HIP(hipMalloc(&route, xd_bfs_route_bytes(V)));
    RUN_XD(xd_bfs_route(drow, dcol, V, nnz, home.attr, route, xd_bfs_route_bytes(V), s));

    // serial queue BFS of the first source
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<uint32_t> ref((size_t)V, XD_BFS_UNVISITED);
    {
        std::queue<int32_t> fq;
        ref[0] = 0;
        fq.push(0);
        while (!fq.empty()) {
            const int32_t u = fq.front();
            fq.pop();
            for (int64_t e = rowptr[u]; e < rowptr[u + 1]; ++e)
                if (ref[col[e]] == XD_BFS_UNVISITED) {
                    ref[col[e]] = ref[u] + 1;
                    fq.push(col[e]);
                }
        }
    }
    const double cpu_ms = wall_ms(t0);

    xd_bfs_stats_t st{};
    long long bad[3] = {0, 0, 0};
    std::vector<uint32_t> got[3];
    for (int mode = 0; mode < 3; ++mode) {
        RUN_XD(xd_bfs_csr(drow, dcol, V, nnz, 0, lvl[mode], mode, route, ws, wsb, s, &st));
        got[mode].resize(V);
        RUN_HIP(hipMemcpy(got[mode].data(), lvl[mode], (size_t)V * 4, hipMemcpyDeviceToHost));
    }
    for (int32_t v = 0; v < V; ++v) {
        bad[0] += got[0][v] != ref[v];
        bad[1] += got[1][v] != got[0][v];
        bad[2] += got[2][v] != got[0][v];
    }
    const long long visited = std::count_if(ref.begin(), ref.end(), [](uint32_t l) { return l != XD_BFS_UNVISITED; });

    std::vector<float> samples[3];
    double teps_edges = 0;
    for (int r = 0; r < runs; ++r)
        for (int mode = 0; mode < 3; ++mode) {
            double edges = 0;
            const float t = time_ms(s, [&] {
                for (int k = 0; k < nsrc; ++k) {
                    RUN_XD(xd_bfs_csr(drow, dcol, V, nnz, k, lvl[mode], mode, route, ws, wsb, s, &st));
                    edges += st.reached_edges / 2.0;
                }
            });
            samples[mode].push_back(t);
            teps_edges = edges;
        }
    const double med[3] = {median(samples[0]), median(samples[1]), median(samples[2])};

    printf("=== Locality-aware BFS, R-MAT (XCD domains) ===\n");
    printf("gpu=%s vertices=%d degree=%d sources=%d depth=%d dst_local=%d%% hot/side=%d runs=%d seed=%llu nnz=%lld\n",
           topo.name, V, degree, nsrc, depth, dst_local, hot, runs, (unsigned long long)seed, (long long)nnz);
    // overflow: the reference's fixed-size queues can overflow; these queues hold every vertex
    printf("visited=%lld aware_bad=%lld swapped_bad=%lld overflow=0 groups=%d/%d baseline_bad=%lld\n", visited, bad[1],
           bad[2], topo.num_xcd / 2, topo.num_xcd / 2, bad[0]);
    printf("| mode | median_ms | speedup_vs_baseline |\n");
    printf("|---|---:|---:|\n");
    printf("| baseline | %.6f | 1.000000 |\n", med[0]);
    printf("| aware | %.6f | %.6f |\n", med[1], med[0] / med[1]);
    printf("| swapped | %.6f | %.6f |\n", med[2], med[0] / med[2]);
    printf("gteps baseline=%.3f aware=%.3f swapped=%.3f levels=%d topdown_steps=%d bottomup_steps=%d\n",
           teps_edges / (med[0] * 1e6), teps_edges / (med[1] * 1e6), teps_edges / (med[2] * 1e6), st.levels,
           st.topdown_steps, st.bottomup_steps);
    printf("cpu_ms=%.3f cpu_threads=1\n", cpu_ms);
    const bool pass = bad[0] == 0 && bad[1] == 0 && bad[2] == 0;
    char row[512];
    snprintf(row, sizeof row,
             "%s,%s,%s,0,%d,%d,%d,%d,%d,%d,%d,%llu,%lld,%lld,%lld,0,%.6f,%.6f,%.6f,%.6f,%.6f,%s,rmat,%lld,%.3f,%lld",
             o.opt("sweep", "run").c_str(), o.opt("value", std::to_string(V).c_str()).c_str(), topo.name, V, degree, nsrc,
             depth, dst_local, hot, runs, (unsigned long long)seed, visited, bad[1], bad[2], med[0], med[1], med[2],
             med[0] / med[1], med[0] / med[2], pass ? "PASS" : "FAIL", (long long)nnz, teps_edges / (med[1] * 1e6),
             bad[0]);
    csv_append(o.csv, kCsvHeader, row);
    return pass ? 0 : 3;
}

// The reference's workload: its hot-pool graph, many sources, a fixed number of levels.
static int run_ref(const Options &o) {
    // the reference's defaults and clamps (bfs.cu:329-343)
    const int32_t V = (int32_t)std::max<long long>(o.geti(0, 2000000), 4096);
    const int32_t degree = (int32_t)std::max<long long>(o.geti(1, 64), 1);
    const int32_t nsrc = (int32_t)std::max<long long>(1, std::min<long long>(o.geti(2, 4096), V / 4));
    const int32_t depth = (int32_t)std::max<long long>(o.geti(3, 4), 1);
    const int32_t dst_local = (int32_t)std::max<long long>(0, std::min<long long>(o.geti(4, 100), 100));
    const int32_t hot = (int32_t)std::max<long long>(1024, std::min<long long>(o.geti(5, 200000), V / 3));
    const int runs = (int)std::max<long long>(o.geti(6, 5), 1);
    const uint64_t seed = (uint64_t)o.geti(7, 8201);
    if ((long long)V * degree >= (1ll << 31)) {
        fprintf(stderr, "vertices * degree must be < 2^31\n");
        return 2;
    }
    const xd_topology_t topo = topology();
    hipStream_t s;
    RUN_HIP(hipStreamCreate(&s));
    const int64_t nnz = (int64_t)V * degree;
    int32_t *drow, *dcol, *dsrc;
    uint8_t *dside;
    uint32_t *lvl_ref, *lvl;  // baseline, and aware / swapped (the buffer the sides are derived for)
    RUN_HIP(hipMalloc(&dcol, (size_t)nnz * 4));
    RUN_HIP(hipMalloc(&lvl_ref, (size_t)V * 4));
    RUN_HIP(hipMalloc(&lvl, (size_t)V * 4));
    std::vector<uint8_t> ch, lh;
    {
        HomeMap hc(dcol, (size_t)nnz * 4, s), hl(lvl, (size_t)V * 4, s);
        ch.resize(xd_home_map_pages(dcol, (size_t)nnz * 4));
        lh.resize(xd_home_map_pages(lvl, (size_t)V * 4));
        RUN_HIP(hipMemcpy(ch.data(), hc.attr, ch.size(), hipMemcpyDeviceToHost));
        RUN_HIP(hipMemcpy(lh.data(), hl.attr, lh.size(), hipMemcpyDeviceToHost));
    }
    std::vector<int32_t> rowptr((size_t)V + 1), col((size_t)nnz), src((size_t)nsrc);
    std::vector<uint8_t> side((size_t)V);
    const int rc = xd_bfs_ref_graph(V, degree, nsrc, dst_local, hot, seed, (uint64_t)(uintptr_t)dcol, ch.data(),
                                    (uint64_t)(uintptr_t)lvl, lh.data(), rowptr.data(), col.data(), side.data(),
                                    src.data());
    if (rc == XD_ERR_UNSUPPORTED) {
        fprintf(stderr, "failed hot pools: fewer than %d vertices per side whose row and level homes agree\n", hot);
        return 2;
    }
    RUN_XD(rc);
    RUN_HIP(hipMalloc(&drow, rowptr.size() * 4));
    RUN_HIP(hipMalloc(&dsrc, src.size() * 4));
    RUN_HIP(hipMalloc(&dside, side.size()));
    RUN_HIP(hipMemcpy(drow, rowptr.data(), rowptr.size() * 4, hipMemcpyHostToDevice));
    RUN_HIP(hipMemcpy(dcol, col.data(), (size_t)nnz * 4, hipMemcpyHostToDevice));
    RUN_HIP(hipMemcpy(dsrc, src.data(), src.size() * 4, hipMemcpyHostToDevice));
    RUN_HIP(hipMemcpy(dside, side.data(), side.size(), hipMemcpyHostToDevice));
    const size_t wsb = xd_bfs_multi_workspace_size(V);
    void *ws;
    RUN_HIP(hipMalloc(&ws, wsb));

    // serial multi-source BFS limited to `depth` levels
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<uint32_t> ref((size_t)V, XD_BFS_UNVISITED);
    {
        std::vector<int32_t> q;
        q.reserve((size_t)V);
        for (int32_t v : src)
            if (ref[v] != 0u) {
                ref[v] = 0u;
                q.push_back(v);
            }
        for (size_t head = 0; head < q.size(); ++head) {
            const int32_t u = q[head];
            if ((int32_t)ref[u] >= depth) continue;
            for (int32_t e = rowptr[u]; e < rowptr[u + 1]; ++e)
                if (ref[col[e]] == XD_BFS_UNVISITED) {
                    ref[col[e]] = ref[u] + 1;
                    q.push_back(col[e]);
                }
        }
    }
    const double cpu_ms = wall_ms(t0);

    auto launch = [&](int mode) {
        RUN_XD(xd_bfs_multi(drow, dcol, V, nnz, dsrc, nsrc, depth, dside, mode == 0 ? lvl_ref : lvl, mode, ws, wsb, s));
    };
    std::vector<uint32_t> base((size_t)V), got((size_t)V);
    long long bad[3] = {0, 0, 0};
    launch(0);
    RUN_HIP(hipMemcpy(base.data(), lvl_ref, (size_t)V * 4, hipMemcpyDeviceToHost));
    for (int32_t v = 0; v < V; ++v) bad[0] += base[v] != ref[v];
    for (int mode = 1; mode < 3; ++mode) {
        launch(mode);
        RUN_HIP(hipMemcpy(got.data(), lvl, (size_t)V * 4, hipMemcpyDeviceToHost));
        for (int32_t v = 0; v < V; ++v) bad[mode] += got[v] != base[v];
    }
    long long visited = 0;
    double edges = 0;  // edges the search walks: the lists of the vertices it expands
    for (int32_t v = 0; v < V; ++v) {
        visited += base[v] != XD_BFS_UNVISITED;
        if (base[v] != XD_BFS_UNVISITED && (int32_t)base[v] < depth) edges += rowptr[v + 1] - rowptr[v];
    }
    for (int w = 0; w < 2; ++w)
        for (int mode = 0; mode < 3; ++mode) launch(mode);
    std::vector<float> samples[3];
    for (int r = 0; r < runs; ++r)
        for (int mode = 0; mode < 3; ++mode) samples[mode].push_back(time_ms(s, [&] { launch(mode); }));
    const double med[3] = {median(samples[0]), median(samples[1]), median(samples[2])};
    const double mean_deg = (double)nnz / V;
    int lanes = 1;
    while (lanes < 64 && 2.0 * lanes <= mean_deg * 1.5) lanes *= 2;

    printf("=== Locality-aware BFS (XCD domains) ===\n");
    printf("gpu=%s vertices=%d degree=%d sources=%d depth=%d dst_local=%d%% hot/side=%d runs=%d seed=%llu\n", topo.name,
           V, degree, nsrc, depth, dst_local, hot, runs, (unsigned long long)seed);
    printf("config threads=256 grid=2048 lanes_per_vertex=%d queues=2x3 home=measured\n", lanes);
    printf("visited=%lld aware_bad=%lld swapped_bad=%lld overflow=0 groups=%d/%d baseline_bad=%lld\n", visited, bad[1],
           bad[2], topo.num_xcd / 2, topo.num_xcd / 2, bad[0]);
    printf("| mode | median_ms | speedup_vs_baseline |\n");
    printf("|---|---:|---:|\n");
    printf("| baseline | %.6f | 1.000000 |\n", med[0]);
    printf("| aware | %.6f | %.6f |\n", med[1], med[0] / med[1]);
    printf("| swapped | %.6f | %.6f |\n", med[2], med[0] / med[2]);
    printf("gteps baseline=%.3f aware=%.3f swapped=%.3f edges=%.0f\n", edges / (med[0] * 1e6), edges / (med[1] * 1e6),
           edges / (med[2] * 1e6), edges);
    printf("cpu_ms=%.3f cpu_threads=1\n", cpu_ms);
    const bool pass = bad[0] == 0 && bad[1] == 0 && bad[2] == 0;
    char row[640];
    snprintf(row, sizeof row,
             "%s,%s,%s,0,%d,%d,%d,%d,%d,%d,%d,%llu,%lld,%lld,%lld,0,%.6f,%.6f,%.6f,%.6f,%.6f,%s,ref,%lld,%.3f,%lld",
             o.opt("sweep", "run").c_str(), o.opt("value", std::to_string(V).c_str()).c_str(), topo.name, V, degree, nsrc,
             depth, dst_local, hot, runs, (unsigned long long)seed, visited, bad[1], bad[2], med[0], med[1], med[2],
             med[0] / med[1], med[0] / med[2], pass ? "PASS" : "FAIL", (long long)nnz, edges / (med[1] * 1e6), bad[0]);
    csv_append(o.csv, kCsvHeader, row);
    for (void *p : {(void *)drow, (void *)dcol, (void *)dsrc, (void *)dside, (void *)lvl_ref, (void *)lvl, ws})
        (void)hipFree(p);
    return pass ? 0 : 3;
}

int main(int argc, char **argv) {
    Options o(argc, argv);
    const std::string workload = o.opt("workload", "ref");
    if (o.help || (workload != "ref" && workload != "rmat")) {
        printf("usage: %s [--workload=ref|rmat] [vertices=2000000] [degree=64] [sources=4096] [depth=4] "
               "[dst_local_pct=100] [hot_per_side=200000] [runs=5] [seed=8201] [--sweep=NAME --value=V] [--csv=FILE]\n",
               argv[0]);
        return o.help ? 0 : 2;
    }
    return workload == "ref" ? run_ref(o) : run_rmat(o);
}
