// R-MAT graph generator producing an undirected CSR graph (host, multi-threaded).
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

}  // extern "C"
