// BFS runner: the command line, stdout lines and exit status of the reference's BFS
// benchmark (applications/bfs/src/bfs.cu:324-560, parsed by applications/bfs/run.sh:60-100),
// on libxdom's direction-optimizing BFS over an undirected R-MAT graph.
//
//   xd_bfs_run [vertices=2^22] [degree=32] [sources=1] [depth=0] [dst_local_pct=100]
//              [hot_per_side=0] [runs=5] [seed=8201] [--csv=FILE]
//
// The graph: R-MAT with 2^ceil(log2(vertices)) vertices and edge factor degree / 2
// (a/b/c = 0.57/0.19/0.19, xd_rmat_csr), symmetrised, deduplicated, self-loops dropped.
// `sources` searches run from vertices 0, 1, ...; each runs to completion (depth is echoed:
// the reference stops after a fixed number of top-down levels). dst_local_pct and
// hot_per_side shape the reference's synthetic graph and are echoed only. Times are the
// median over `runs` of the summed searches. "baseline" = XD_MODE_OBLIVIOUS, "aware" =
// XD_MODE_AWARE (bottom-up blocks routed to the die homing their adjacency, with the
// measured home map of col), "swapped" = XD_MODE_ROTATED. visited = vertices reached from
// the first source; aware_bad / swapped_bad count levels that differ from the baseline's
// (the reference's diff_dist_kernel, :310-320), and baseline_bad counts the baseline's
// differences from the runner's serial queue BFS; exit 3 on any difference, as the
// reference does (:558).
#include <math.h>

#include <queue>

#include "runner_common.hpp"

using namespace runner;

int main(int argc, char **argv) {
    Options o(argc, argv);
    if (o.help) {
        printf("usage: %s [vertices=4194304] [degree=32] [sources=1] [depth=0] [dst_local_pct=100] [hot_per_side=0] "
               "[runs=5] [seed=8201] [--csv=FILE]\n",
               argv[0]);
        return 0;
    }
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
    snprintf(row, sizeof row, "run,%d,%s,0,%d,%d,%d,%d,%d,%d,%d,%llu,%lld,%lld,%lld,0,%.6f,%.6f,%.6f,%.6f,%.6f,%s,%lld,%.3f,%lld",
             V, topo.name, V, degree, nsrc, depth, dst_local, hot, runs, (unsigned long long)seed, visited, bad[1], bad[2],
             med[0], med[1], med[2], med[0] / med[1], med[0] / med[2], pass ? "PASS" : "FAIL", (long long)nnz,
             teps_edges / (med[1] * 1e6), bad[0]);
    csv_append(o.csv,
               "sweep,value,gpu_label,gpu_index,vertices,degree,sources,depth,dst_local_pct,hot_per_side,runs,seed,"
               "visited,aware_bad,swapped_bad,overflow,baseline_med_ms,aware_med_ms,swapped_med_ms,aware_speedup,"
               "swapped_speedup,pass,nnz,aware_gteps,baseline_bad",
               row);
    return pass ? 0 : 3;
}
