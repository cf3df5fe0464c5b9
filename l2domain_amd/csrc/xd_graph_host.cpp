// Graph generators (host, multi-threaded): the build's undirected R-MAT graph and the
// reference's own directed hot-pool graph.
//
// The reference's BFS input is a synthetic fixed-degree graph drawn from two "hot pools"
// with std::mt19937 (applications/bfs/src/bfs.cu:354-409). The BFS configuration of this
// build is an undirected R-MAT graph instead, fully specified so that any implementation
// regenerates it bit for bit:
//   edge e (0 <= e < edge_factor * 2^scale) descends `scale` levels, most significant bit
//   first; level l draws r = 32-bit word (l & 1) of xd_rand64(seed, e * ceil(scale/2) + l/2)
//   (low word first) and picks quadrant a (r < A), b (r < A+B), c (r < A+B+C) or d, with
//   A = floor(a * 2^32) etc.; quadrants c and d set the row bit, b and d the column bit.
//   Every edge (u, v) with u != v is stored in both directions; duplicates are removed and
//   each adjacency list is sorted ascending.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <memory>
#include <thread>
#include <vector>

#include "xdom.h"

namespace {

inline uint64_t mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
inline uint64_t rnd(uint64_t seed, uint64_t i) { return mix(seed + (i + 1) * 0x9E3779B97F4A7C15ull); }

template <typename F>
void par(size_t n, F &&body) {
    unsigned hw = std::thread::hardware_concurrency();
    size_t nt = std::max<size_t>(1, std::min<size_t>(hw ? hw : 1, 16));
    if (n < 4096) nt = 1;
    std::vector<std::thread> ts;
    size_t per = (n + nt - 1) / nt;
    for (size_t t = 0; t < nt; ++t) {
        size_t b = t * per, e = std::min(n, b + per);
        if (b >= e) break;
        if (nt == 1) {
            body(b, e);
            return;
        }
        ts.emplace_back([&, b, e] { body(b, e); });
    }
    for (auto &t : ts) t.join();
}

}  // namespace

extern "C" {

int xd_rmat_edge(int scale, double a, double b, double c, uint64_t seed, uint64_t e, int32_t *u_out, int32_t *v_out) {
    if (scale < 1 || scale > 30) return XD_ERR_INVALID_ARG;
    const uint32_t A = (uint32_t)std::floor(a * 4294967296.0);
    const uint32_t AB = (uint32_t)std::floor((a + b) * 4294967296.0);
    const uint32_t ABC = (uint32_t)std::floor((a + b + c) * 4294967296.0);
    const uint64_t W = (uint64_t)(scale + 1) / 2;
    uint32_t u = 0, v = 0;
    uint64_t word = 0;
    for (int l = 0; l < scale; ++l) {
        if ((l & 1) == 0) word = rnd(seed, e * W + (uint64_t)(l / 2));
        const uint32_t r = (uint32_t)(word >> (32 * (l & 1)));
        const uint32_t q = r < A ? 0u : r < AB ? 1u : r < ABC ? 2u : 3u;
        u = (u << 1) | (q >> 1);
        v = (v << 1) | (q & 1u);
    }
    *u_out = (int32_t)u;
    *v_out = (int32_t)v;
    return XD_OK;
}

int xd_rmat_csr(int scale, int edge_factor, double a, double b, double c, uint64_t seed, int32_t *rowptr,
                int32_t *col, int64_t col_capacity, int64_t *nnz_out) {
    if (scale < 1 || scale > 30 || edge_factor < 1 || !rowptr || !nnz_out) return XD_ERR_INVALID_ARG;
    if (!(a >= 0 && b >= 0 && c >= 0 && a + b + c <= 1.0)) return XD_ERR_INVALID_ARG;
    const int64_t V = (int64_t)1 << scale;
    const int64_t E = (int64_t)edge_factor * V;
    if (2 * E > INT32_MAX) return XD_ERR_UNSUPPORTED;
    if (!col || col_capacity < 2 * E) return XD_ERR_INVALID_ARG;
    std::vector<int32_t> src((size_t)E), dst((size_t)E);
    par((size_t)E, [&](size_t lo, size_t hi) {
        for (size_t e = lo; e < hi; ++e) xd_rmat_edge(scale, a, b, c, seed, e, &src[e], &dst[e]);
    });
    std::unique_ptr<std::atomic<int32_t>[]> deg(new std::atomic<int32_t>[(size_t)V]);
    for (int64_t i = 0; i < V; ++i) deg[i].store(0, std::memory_order_relaxed);
    par((size_t)E, [&](size_t lo, size_t hi) {
        for (size_t e = lo; e < hi; ++e)
            if (src[e] != dst[e]) {
                deg[src[e]].fetch_add(1, std::memory_order_relaxed);
                deg[dst[e]].fetch_add(1, std::memory_order_relaxed);
            }
    });
    std::vector<int64_t> off((size_t)V + 1);
    off[0] = 0;
    for (int64_t i = 0; i < V; ++i) off[i + 1] = off[i] + deg[i].load(std::memory_order_relaxed);
    std::vector<int32_t> tmp((size_t)off[V]);
    for (int64_t i = 0; i < V; ++i) deg[i].store(0, std::memory_order_relaxed);
    par((size_t)E, [&](size_t lo, size_t hi) {
        for (size_t e = lo; e < hi; ++e)
            if (src[e] != dst[e]) {
                tmp[off[src[e]] + deg[src[e]].fetch_add(1, std::memory_order_relaxed)] = dst[e];
                tmp[off[dst[e]] + deg[dst[e]].fetch_add(1, std::memory_order_relaxed)] = src[e];
            }
    });
    std::vector<int32_t> ndeg((size_t)V);
    par((size_t)V, [&](size_t lo, size_t hi) {
        for (size_t v = lo; v < hi; ++v) {
            int32_t *beg = tmp.data() + off[v], *end = tmp.data() + off[v + 1];
            std::sort(beg, end);
            ndeg[v] = (int32_t)(std::unique(beg, end) - beg);
        }
    });
    rowptr[0] = 0;
    for (int64_t v = 0; v < V; ++v) rowptr[v + 1] = rowptr[v] + ndeg[v];
    par((size_t)V, [&](size_t lo, size_t hi) {
        for (size_t v = lo; v < hi; ++v) memcpy(col + rowptr[v], tmp.data() + off[v], sizeof(int32_t) * (size_t)ndeg[v]);
    });
    *nnz_out = rowptr[V];
    return XD_OK;
}


// The reference's BFS graph (applications/bfs/src/bfs.cu:354-409). A vertex's side is the
// die homing the start of its adjacency row (col + v * degree); its level entry's die must
// agree for it to enter the hot pool of that side (the first hot_per_side such vertices per
// side, in vertex order). The last cross_per_side = hot_per_side * (100 - dst_local_pct) /
// 100 hot vertices of each pool draw their neighbours from the other pool and are worked on
// by the other side; every other vertex draws from its own side's pool. Neighbour j of v is
// pool[xd_rand64(seed, v * degree + j) mod hot_per_side] (the reference draws from
// std::mt19937(seed)); source i is hot1[(i / 2) mod H] for odd i, hot0[(i / 2) mod H] for even.
int xd_bfs_ref_graph(int32_t V, int32_t degree, int32_t num_sources, int32_t dst_local_pct, int32_t hot_per_side,
                     uint64_t seed, uint64_t col_addr, const uint8_t *col_home_host, uint64_t level_addr,
                     const uint8_t *level_home_host, int32_t *rowptr, int32_t *col, uint8_t *work_side,
                     int32_t *sources) {
    if (V < 1 || degree < 1 || (int64_t)V * degree >= (1ll << 31) || num_sources < 0 || dst_local_pct < 0 ||
        dst_local_pct > 100 || hot_per_side < 1 || !rowptr || !col || !work_side || (num_sources > 0 && !sources))
        return XD_ERR_INVALID_ARG;
    const uint64_t mask = xd_home_mask();
    auto side = [&](uint64_t addr, uint64_t base, const uint8_t *attr) -> uint8_t {
        if (attr) return (uint8_t)(((addr >> 13) & 1u) ^ attr[(addr >> 21) - (base >> 21)]);
        return (uint8_t)(__builtin_popcountll(addr & mask) & 1);
    };
    std::vector<int32_t> hot[2];
    hot[0].reserve((size_t)hot_per_side);
    hot[1].reserve((size_t)hot_per_side);
    for (int32_t v = 0; v < V; ++v) {
        const uint8_t rs = side(col_addr + (uint64_t)v * (uint64_t)degree * 4u, col_addr, col_home_host);
        const uint8_t ds = side(level_addr + (uint64_t)v * 4u, level_addr, level_home_host);
        work_side[v] = rs;
        if (rs == ds && (int32_t)hot[rs].size() < hot_per_side) hot[rs].push_back(v);
    }
    if ((int32_t)hot[0].size() < hot_per_side || (int32_t)hot[1].size() < hot_per_side) return XD_ERR_UNSUPPORTED;
    std::vector<uint8_t> dst_side(work_side, work_side + V);
    const int32_t cross = (int32_t)((int64_t)hot_per_side * (100 - dst_local_pct) / 100);
    for (int32_t i = 0; i < cross; ++i) {
        const int32_t v0 = hot[0][(size_t)(hot_per_side - 1 - i)], v1 = hot[1][(size_t)(hot_per_side - 1 - i)];
        dst_side[v0] = 1;  // its neighbours come from the other pool ...
        dst_side[v1] = 0;
        work_side[v0] = 1;  // ... and the other side works on it
        work_side[v1] = 0;
    }
    const uint64_t H = (uint64_t)hot_per_side;
    par((size_t)V, [&](size_t b, size_t e) {
        for (size_t v = b; v < e; ++v) {
            rowptr[v] = (int32_t)(v * (size_t)degree);
            const std::vector<int32_t> &pool = hot[dst_side[v]];
            for (int32_t j = 0; j < degree; ++j)
                col[v * (size_t)degree + (size_t)j] = pool[(size_t)(rnd(seed, (uint64_t)v * (uint64_t)degree + (uint64_t)j) % H)];
        }
    });
    rowptr[V] = (int32_t)((int64_t)V * degree);
    for (int32_t i = 0; i < num_sources; ++i) sources[i] = hot[i & 1][(size_t)((i / 2) % hot_per_side)];
    return XD_OK;
}

}  // extern "C"
