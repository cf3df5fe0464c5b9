// Direction-optimizing BFS over an undirected CSR graph (int32 indices, uint32 levels).
//
// Reference: applications/bfs/src/bfs.cu
//   kUnvisited = 0xffffffff, dist = depth + 1 on the first claim (30, 215-252);
//   luo_baseline_level_kernel (215-252): top-down level, atomicCAS claims, LDS-binned queues
//     flushed with one global atomicAdd per block (176-213);
//   luo_side_level_kernel (254-308): per-side frontiers, winners split by the side of the
//     destination; host level loop with per-level launches (449-491).
//   The reference runs a fixed number of top-down levels from 4096 sources; here one source
//   is searched to completion with Beamer's direction optimisation.
//
// MI355X design.
//   state: level[V]; visited and frontier bitmaps (u64 words, 512 KiB at 2^22 vertices,
//   resident in every XCD's L2); a frontier queue for top-down steps.
//   top-down: one lane per frontier vertex (hubs above kBigDeg are expanded by the whole
//     grid in a second kernel); a claim is a 64-bit atomicOr on the visited word; winners
//     are appended to the next queue with one atomicAdd per wave (ballot + mbcnt).
//   bottom-up: every unvisited vertex scans its neighbours until one is in the frontier
//     bitmap; a wave covers 64 vertices and writes their visited/next bits with one atomic
//     per touched word. Oblivious mode walks 64-vertex blocks in order; XCD-aware mode lets
//     each I/O die take the blocks whose adjacency starts in memory homed on that die
//     (xd_home_map of col), so the dominant traffic -- the neighbour lists -- is read from
//     the near die; rotated hands each die the far blocks.
//   direction: top-down -> bottom-up when m_f > m_u / 14, bottom-up -> top-down when
//     n_f < V / 24 (Beamer, Asanovic, Patterson, SC'12), decided on the host after reading
//     the per-level counters (the call is synchronous).
#include <hip/hip_runtime.h>

#include <string.h>

#include <algorithm>
#include <utility>

#include "xd_common.hpp"

namespace xd {

constexpr uint32_t kUnv = 0xffffffffu;
constexpr int kBfsThreads = 256;
constexpr int kBfsGrid = 2048;          // fixed grid of the level kernels (multiple of 8)
constexpr int32_t kBigDeg = 4096;       // top-down: larger lists are expanded by the whole grid
constexpr double kAlpha = 14.0, kBeta = 24.0;

struct BfsCounters {
    unsigned long long next_count;  // vertices appended to the next queue (top-down)
    unsigned long long big_count;   // hub vertices deferred to the grid-wide expansion
};

struct BfsPartial {  // per workgroup, summed by bfs_reduce_kernel
    unsigned long long verts;
    unsigned long long edges;
};

struct BfsLayout {
    size_t visited, front_a, front_b, queue_a, queue_b, big, counters, partials, sums, blist, bcount, total;
    int64_t words, nblocks;
};

static size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }

static BfsLayout bfs_layout(int32_t V, int64_t nnz) {
    (void)nnz;
    BfsLayout L{};
    L.words = ((int64_t)V + 63) / 64;
    size_t o = 0;
    L.counters = o;
    o = a256(o + sizeof(BfsCounters));
    L.sums = o;
    o = a256(o + sizeof(BfsPartial));
    L.partials = o;
    o = a256(o + sizeof(BfsPartial) * kBfsGrid);
    L.visited = o;
    o = a256(o + 8 * (size_t)L.words);
    L.front_a = o;
    o = a256(o + 8 * (size_t)L.words);
    L.front_b = o;
    o = a256(o + 8 * (size_t)L.words);
    L.queue_a = o;
    o = a256(o + 4 * (size_t)V);
    L.queue_b = o;
    o = a256(o + 4 * (size_t)V);
    L.big = o;
    o = a256(o + 4 * (size_t)V);
    L.nblocks = ((int64_t)V + 63) / 64;
    L.bcount = o;
    o = a256(o + 2 * sizeof(unsigned long long));
    L.blist = o;
    o = a256(o + 2 * 4 * (size_t)L.nblocks);
    L.total = o;
    return L;
}

__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
    return v;
}

// Sums the per-workgroup partials of a level (one workgroup) into `sums`.
__global__ void __launch_bounds__(256) bfs_reduce_kernel(const BfsPartial *__restrict__ parts, int n,
                                                         BfsPartial *__restrict__ sums) {
    __shared__ unsigned long long sv[256 / kWave], se[256 / kWave];
    unsigned long long v = 0, e = 0;
    for (int i = (int)threadIdx.x; i < n; i += 256) {
        v += parts[i].verts;
        e += parts[i].edges;
    }
    v = wave_sum_u64(v);
    e = wave_sum_u64(e);
    const int lane = (int)threadIdx.x % kWave, wave = (int)threadIdx.x / kWave;
    if (lane == 0) {
        sv[wave] = v;
        se[wave] = e;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long tv = 0, te = 0;
        for (int w = 0; w < 256 / kWave; ++w) {
            tv += sv[w];
            te += se[w];
        }
        sums->verts = tv;
        sums->edges = te;
    }
}

// Workgroup partial: wave sums through LDS, thread 0 stores (no atomics on one address).
__device__ __forceinline__ void store_partial(BfsPartial *parts, unsigned long long v, unsigned long long e) {
    __shared__ unsigned long long sv[kBfsThreads / kWave], se[kBfsThreads / kWave];
    v = wave_sum_u64(v);
    e = wave_sum_u64(e);
    const int lane = (int)threadIdx.x % kWave, wave = (int)threadIdx.x / kWave;
    if (lane == 0) {
        sv[wave] = v;
        se[wave] = e;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long tv = 0, te = 0;
        for (int w = 0; w < kBfsThreads / kWave; ++w) {
            tv += sv[w];
            te += se[w];
        }
        parts[blockIdx.x].verts = tv;
        parts[blockIdx.x].edges = te;
    }
}

__global__ void __launch_bounds__(256) bfs_init_kernel(uint32_t *level, int32_t V, unsigned long long *visited,
                                                       int64_t words, int32_t src, int32_t *queue) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < V; i += stride)
        level[i] = (i == src) ? 0u : kUnv;
    for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < words; w += stride)
        visited[w] = (w == src / 64) ? (1ull << (src % 64)) : 0ull;
    if (blockIdx.x == 0 && threadIdx.x == 0) queue[0] = src;
}

__global__ void __launch_bounds__(256) bfs_fill_kernel(unsigned long long *p, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0ull;
}

__global__ void bfs_zero_counters_kernel(BfsCounters *c) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        c->next_count = 0;
        c->big_count = 0;
    }
}

// Claims v for level `lvl`; returns true if this thread won it.
__device__ __forceinline__ bool claim(unsigned long long *visited, uint32_t *level, int32_t v, uint32_t lvl) {
    const unsigned long long bit = 1ull << (v & 63);
    unsigned long long *w = visited + (v >> 6);
    if (__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & bit) return false;
    if (atomicOr(w, bit) & bit) return false;
    level[v] = lvl;
    return true;
}

// Appends the claiming lanes' vertices to `queue` with one atomic per wave.
__device__ __forceinline__ void wave_append(bool won, int32_t v, int32_t *queue, unsigned long long *count) {
    const uint64_t m = __ballot(won);
    if (!m) return;
    const int leader = __builtin_ctzll(m);
    unsigned long long base = 0;
    if (lane_id() == leader) base = atomicAdd(count, (unsigned long long)__builtin_popcountll(m));
    base = __shfl(base, leader, kWave);
    if (won) queue[base + mask_rank(m)] = v;
}

__global__ void __launch_bounds__(kBfsThreads)
bfs_td_kernel(const int32_t *__restrict__ rowptr, const int32_t *__restrict__ col, const int32_t *__restrict__ queue,
              int64_t count, uint32_t *__restrict__ level, unsigned long long *__restrict__ visited,
              int32_t *__restrict__ next, BfsCounters *__restrict__ ctr, int32_t *__restrict__ big,
              BfsPartial *__restrict__ parts, uint32_t lvl) {
    unsigned long long my_edges = 0, my_verts = 0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    // Uniform trip count per wave so that the ballots in wave_append see whole waves.
    const int64_t first = (int64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~(kWave - 1));
    for (int64_t i0 = first; i0 < count; i0 += stride) {
        const int64_t i = i0 + lane_id();
        int32_t beg = 0, end = 0;
        if (i < count) {
            const int32_t u = queue[i];
            beg = rowptr[u];
            end = rowptr[u + 1];
            if (end - beg > kBigDeg) {
                const unsigned long long slot = atomicAdd(&ctr->big_count, 1ull);
                big[slot] = u;
                end = beg;
            }
        }
        // lanes walk their own lists; iterations stay wave-uniform up to the longest list
        int32_t len = end - beg;
        int32_t maxlen = len;
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) maxlen = max(maxlen, __shfl_xor(maxlen, d, kWave));
        for (int32_t j = 0; j < maxlen; ++j) {
            bool won = false;
            int32_t v = 0;
            if (j < len) {
                v = col[beg + j];
                won = claim(visited, level, v, lvl);
                if (won) {
                    my_verts += 1;
                    my_edges += (unsigned long long)(rowptr[v + 1] - rowptr[v]);
                }
            }
            wave_append(won, v, next, &ctr->next_count);
        }
    }
    store_partial(parts, my_verts, my_edges);
}

// Grid-wide expansion of the hub vertices deferred by bfs_td_kernel.
__global__ void __launch_bounds__(kBfsThreads)
bfs_td_big_kernel(const int32_t *__restrict__ rowptr, const int32_t *__restrict__ col, const int32_t *__restrict__ big,
                  const BfsCounters *__restrict__ cnt_in, uint32_t *__restrict__ level,
                  unsigned long long *__restrict__ visited, int32_t *__restrict__ next, BfsCounters *__restrict__ ctr,
                  BfsPartial *__restrict__ parts, uint32_t lvl) {
    unsigned long long my_edges = 0, my_verts = 0;
    const int64_t nbig = (int64_t)cnt_in->big_count;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t h = 0; h < nbig; ++h) {
        const int32_t u = big[h];
        const int32_t beg = rowptr[u], end = rowptr[u + 1];
        const int64_t first = (int64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~(kWave - 1));
        for (int64_t e0 = beg + first; e0 < end; e0 += stride) {
            const int64_t e = e0 + lane_id();
            bool won = false;
            int32_t v = 0;
            if (e < end) {
                v = col[e];
                won = claim(visited, level, v, lvl);
                if (won) {
                    my_verts += 1;
                    my_edges += (unsigned long long)(rowptr[v + 1] - rowptr[v]);
                }
            }
            wave_append(won, v, next, &ctr->next_count);
        }
    }
    // add to the partials of the first kernel
    __shared__ unsigned long long sv[kBfsThreads / kWave], se[kBfsThreads / kWave];
    my_verts = wave_sum_u64(my_verts);
    my_edges = wave_sum_u64(my_edges);
    if (lane_id() == 0) {
        sv[threadIdx.x / kWave] = my_verts;
        se[threadIdx.x / kWave] = my_edges;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long tv = 0, te = 0;
        for (int w = 0; w < kBfsThreads / kWave; ++w) {
            tv += sv[w];
            te += se[w];
        }
        parts[blockIdx.x].verts += tv;
        parts[blockIdx.x].edges += te;
    }
}

// Bottom-up step over the vertices [v0, v1): lanes take v0 + lane, v0 + 64 + lane, ...
__device__ __forceinline__ void bu_range(int32_t v0, int32_t v1, const int32_t *__restrict__ rowptr,
                                         const int32_t *__restrict__ col, const unsigned long long *__restrict__ front,
                                         uint32_t *__restrict__ level, unsigned long long *__restrict__ visited,
                                         unsigned long long *__restrict__ next, uint32_t lvl,
                                         unsigned long long &my_verts, unsigned long long &my_edges) {
    const int lane = lane_id();
    for (int32_t vb = v0; vb < v1; vb += kWave) {
        const int32_t v = vb + lane;
        bool found = false;
        int32_t deg = 0;
        if (v < v1) {
            const unsigned long long vis = visited[v >> 6];
            if (!((vis >> (v & 63)) & 1ull)) {
                const int32_t beg = rowptr[v], end = rowptr[v + 1];
                deg = end - beg;
                for (int32_t e = beg; e < end; ++e) {
                    const int32_t u = col[e];
                    if ((front[u >> 6] >> (u & 63)) & 1ull) {
                        found = true;
                        break;
                    }
                }
            }
        }
        if (found) {
            level[v] = lvl;
            my_verts += 1;
            my_edges += (unsigned long long)deg;
        }
        // vb is a multiple of 64, so the block's found bits are exactly bitmap word vb / 64,
        // which no other wave touches during this step: a plain update suffices
        const uint64_t m = __ballot(found);
        if (m && lane == 0) {
            const int32_t w0 = vb >> 6;
            visited[w0] |= m;
            next[w0] |= m;
        }
    }
}

// Sorts the 64-vertex blocks by the I/O die that homes the start of their adjacency (the
// block's first vertex on): list[d * nblocks + i] is the i-th block of die d. The
// assignment depends only on the graph and the page map, so it is built once per search;
// the bottom-up steps of the home modes then walk their die's list with no skipped blocks.
// A workgroup classifies 1024 blocks and reserves its list space with one atomic per die.
constexpr int kBlkThreads = 1024;
__global__ void __launch_bounds__(kBlkThreads)
bfs_blocks_kernel(const int32_t *__restrict__ rowptr, int64_t nblocks, uint64_t cbase, int64_t col_bytes,
                  HomeMap home, int32_t *__restrict__ list, unsigned long long *__restrict__ count) {
    __shared__ uint32_t wcnt[2][kBlkThreads / kWave];
    __shared__ unsigned long long wbase[2][kBlkThreads / kWave];
    const int tid = (int)threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const int64_t blk = (int64_t)blockIdx.x * kBlkThreads + tid;
    uint32_t d = 2;
    if (blk < nblocks) {
        uint64_t off = (uint64_t)rowptr[blk * kWave] * sizeof(int32_t);
        if (off >= (uint64_t)col_bytes) off = (uint64_t)col_bytes - 1;  // trailing isolated vertices
        d = home(cbase + off);
    }
    const uint64_t m0 = __ballot(d == 0), m1 = __ballot(d == 1);
    if (lane == 0) {
        wcnt[0][wave] = (uint32_t)__builtin_popcountll(m0);
        wcnt[1][wave] = (uint32_t)__builtin_popcountll(m1);
    }
    __syncthreads();
    if (tid < 2) {
        unsigned long long tot = 0;
        for (int w = 0; w < kBlkThreads / kWave; ++w) {
            wbase[tid][w] = tot;
            tot += wcnt[tid][w];
        }
        const unsigned long long b = tot ? atomicAdd(&count[tid], tot) : 0ull;
        for (int w = 0; w < kBlkThreads / kWave; ++w) wbase[tid][w] += b;
    }
    __syncthreads();
    if (d < 2) {
        const uint64_t m = d ? m1 : m0;
        list[(int64_t)d * nblocks + (int64_t)(wbase[d][wave] + mask_rank(m))] = (int32_t)blk;
    }
}

__global__ void __launch_bounds__(kBfsThreads)
bfs_bu_kernel(const int32_t *__restrict__ rowptr, const int32_t *__restrict__ col, int32_t V,
              const unsigned long long *__restrict__ front, uint32_t *__restrict__ level,
              unsigned long long *__restrict__ visited, unsigned long long *__restrict__ next, int mode,
              const int32_t *__restrict__ blist, const unsigned long long *__restrict__ bcount, int64_t nblocks,
              BfsPartial *__restrict__ parts, uint32_t lvl) {
    unsigned long long my_verts = 0, my_edges = 0;
    const int wave = (int)threadIdx.x / kWave;
    constexpr int kWavesPerWg = kBfsThreads / kWave;
    if (mode == XD_MODE_OBLIVIOUS) {
        for (int64_t blk = (int64_t)blockIdx.x * kWavesPerWg + wave; blk < nblocks;
             blk += (int64_t)gridDim.x * kWavesPerWg) {
            const int32_t v0 = (int32_t)(blk * kWave);
            const int32_t v1 = (int32_t)min((int64_t)V, (int64_t)v0 + kWave);
            bu_range(v0, v1, rowptr, col, front, level, visited, next, lvl, my_verts, my_edges);
        }
    } else {
        // The workgroups of a die walk that die's block list (aware) or the other die's
        // (rotated), so the neighbour lists are read from the near (far) die.
        const int b = (int)blockIdx.x;
        const int per_die = (int)gridDim.x / 2;
        const int rank = (b / kNumXcd) * (kNumXcd / 2) + (b % (kNumXcd / 2));
        const uint32_t die = wg_die(b);
        const uint32_t want = (mode == XD_MODE_AWARE) ? die : (die ^ 1u);
        const int32_t *mine = blist + (int64_t)want * nblocks;
        const int64_t cnt = (int64_t)bcount[want];
        for (int64_t i = (int64_t)rank * kWavesPerWg + wave; i < cnt; i += (int64_t)per_die * kWavesPerWg) {
            const int32_t v0 = mine[i] * kWave;
            const int32_t v1 = (int32_t)min((int64_t)V, (int64_t)v0 + kWave);
            bu_range(v0, v1, rowptr, col, front, level, visited, next, lvl, my_verts, my_edges);
        }
    }
    store_partial(parts, my_verts, my_edges);
}

// queue -> bitmap (top-down to bottom-up switch)
__global__ void __launch_bounds__(256) bfs_q2b_kernel(const int32_t *__restrict__ queue, int64_t count,
                                                      unsigned long long *__restrict__ bits) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        const int32_t v = queue[i];
        atomicOr(&bits[v >> 6], 1ull << (v & 63));
    }
}

// bitmap -> queue (bottom-up to top-down switch); one atomic per wave
__global__ void __launch_bounds__(256) bfs_b2q_kernel(const unsigned long long *__restrict__ bits, int64_t words,
                                                      int32_t *__restrict__ queue, unsigned long long *__restrict__ count) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t first = (int64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~(kWave - 1));
    for (int64_t w0 = first; w0 < words; w0 += stride) {
        const int64_t w = w0 + lane_id();
        unsigned long long m = w < words ? bits[w] : 0ull;
        const uint32_t c = (uint32_t)__builtin_popcountll(m);
        // exclusive wave scan of c
        uint32_t incl = c;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const uint32_t t = __shfl_up(incl, d, kWave);
            if (lane_id() >= d) incl += t;
        }
        const uint32_t total = (uint32_t)__shfl(incl, kWave - 1, kWave);
        unsigned long long base = 0;
        if (lane_id() == 0 && total) base = atomicAdd(count, (unsigned long long)total);
        base = __shfl(base, 0, kWave) + (incl - c);
        while (m) {
            const int bit = __builtin_ctzll(m);
            queue[base++] = (int32_t)(w * 64 + bit);
            m &= m - 1;
        }
    }
}

}  // namespace xd

using namespace xd;

extern "C" {

size_t xd_bfs_workspace_size(int32_t num_vertices, int64_t nnz) {
    if (num_vertices <= 0 || nnz < 0) return 0;
    return bfs_layout(num_vertices, nnz).total;
}

int xd_bfs_csr(const int32_t *rowptr, const int32_t *col, int32_t V, int64_t nnz, int32_t src, uint32_t *level,
               int mode, const uint8_t *home_attr, void *workspace, size_t workspace_bytes, void *stream,
               xd_bfs_stats_t *stats) {
    XD_REQUIRE(rowptr != nullptr && level != nullptr && (nnz == 0 || col != nullptr), "xd_bfs_csr: NULL pointer");
    XD_REQUIRE(V > 0 && nnz >= 0 && nnz < (1ll << 31), "xd_bfs_csr: need 0 < V and 0 <= nnz < 2^31");
    XD_REQUIRE(src >= 0 && src < V, "xd_bfs_csr: src out of range");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "xd_bfs_csr: bad mode");
    const BfsLayout L = bfs_layout(V, nnz);
    if (workspace == nullptr || workspace_bytes < L.total || !aligned16(workspace))
        return fail(XD_ERR_WORKSPACE, "xd_bfs_csr: workspace missing or smaller than xd_bfs_workspace_size()");
    hipStream_t s = (hipStream_t)stream;
    char *ws = static_cast<char *>(workspace);
    auto *visited = reinterpret_cast<unsigned long long *>(ws + L.visited);
    auto *fa = reinterpret_cast<unsigned long long *>(ws + L.front_a);
    auto *fb = reinterpret_cast<unsigned long long *>(ws + L.front_b);
    auto *qa = reinterpret_cast<int32_t *>(ws + L.queue_a);
    auto *qb = reinterpret_cast<int32_t *>(ws + L.queue_b);
    auto *big = reinterpret_cast<int32_t *>(ws + L.big);
    auto *ctr = reinterpret_cast<BfsCounters *>(ws + L.counters);
    auto *parts = reinterpret_cast<BfsPartial *>(ws + L.partials);
    auto *sums = reinterpret_cast<BfsPartial *>(ws + L.sums);
    auto *blist = reinterpret_cast<int32_t *>(ws + L.blist);
    auto *bcount = reinterpret_cast<unsigned long long *>(ws + L.bcount);
    const HomeMap home{nnz > 0 ? home_attr : nullptr, reinterpret_cast<uint64_t>(col) / kHomePage, home_mask()};
    const int bmode = nnz > 0 ? mode : XD_MODE_OBLIVIOUS;  // no adjacency to route by
    const unsigned g256 = (unsigned)std::min<int64_t>(8192, ((int64_t)V + 255) / 256 + 1);

    int32_t src_rows[2];
    XD_HIP(hipMemcpyAsync(src_rows, rowptr + src, sizeof(src_rows), hipMemcpyDeviceToHost, s));
    XD_HIP(hipStreamSynchronize(s));
    {
        KernelTimer kt("bfs_init", s);
        hipLaunchKernelGGL(bfs_init_kernel, dim3(g256), dim3(256), 0, s, level, V, visited, L.words, src, qa);
        if (int rc = launch_status("bfs_init_kernel")) return rc;
        if (bmode != XD_MODE_OBLIVIOUS) {
            hipLaunchKernelGGL(bfs_fill_kernel, dim3(1), dim3(64), 0, s, bcount, (int64_t)2);
            hipLaunchKernelGGL(bfs_blocks_kernel, dim3((unsigned)((L.nblocks + kBlkThreads - 1) / kBlkThreads)),
                               dim3(kBlkThreads), 0, s, rowptr, L.nblocks, reinterpret_cast<uint64_t>(col),
                               nnz * (int64_t)sizeof(int32_t), home, blist, bcount);
            if (int rc = launch_status("bfs_blocks_kernel")) return rc;
        }
    }
    int64_t m_u = nnz - (src_rows[1] - src_rows[0]);
    int64_t n_f = 1, m_f = src_rows[1] - src_rows[0];
    int64_t reached_v = 1, reached_e = m_f;
    bool bottom_up = false;
    int32_t *qcur = qa, *qnext = qb;
    unsigned long long *fcur = fa, *fnext = fb;
    int td = 0, bu = 0, depth = 0;
    for (;; ++depth) {
        const uint32_t lvl = (uint32_t)depth + 1;
        hipLaunchKernelGGL(bfs_zero_counters_kernel, dim3(1), dim3(64), 0, s, ctr);
        if (!bottom_up) {
            ++td;
            {
                KernelTimer kt("bfs_topdown", s);
                hipLaunchKernelGGL(bfs_td_kernel, dim3(kBfsGrid), dim3(kBfsThreads), 0, s, rowptr, col, qcur, n_f,
                                   level, visited, qnext, ctr, big, parts, lvl);
                if (int rc = launch_status("bfs_td_kernel")) return rc;
                hipLaunchKernelGGL(bfs_td_big_kernel, dim3(kBfsGrid), dim3(kBfsThreads), 0, s, rowptr, col, big, ctr,
                                   level, visited, qnext, ctr, parts, lvl);
                if (int rc = launch_status("bfs_td_big_kernel")) return rc;
            }
        } else {
            ++bu;
            KernelTimer kt("bfs_bottomup", s);
            hipLaunchKernelGGL(bfs_fill_kernel, dim3((unsigned)std::min<int64_t>(2048, L.words / 256 + 1)), dim3(256), 0,
                               s, fnext, L.words);
            hipLaunchKernelGGL(bfs_bu_kernel, dim3(kBfsGrid), dim3(kBfsThreads), 0, s, rowptr, col, V, fcur, level,
                               visited, fnext, bmode, blist, bcount, L.nblocks, parts, lvl);
            if (int rc = launch_status("bfs_bu_kernel")) return rc;
        }
        hipLaunchKernelGGL(bfs_reduce_kernel, dim3(1), dim3(256), 0, s, parts, kBfsGrid, sums);
        BfsPartial h{};
        XD_HIP(hipMemcpyAsync(&h, sums, sizeof(h), hipMemcpyDeviceToHost, s));
        XD_HIP(hipStreamSynchronize(s));
        n_f = (int64_t)h.verts;
        m_f = (int64_t)h.edges;
        if (n_f == 0) break;
        reached_v += n_f;
        reached_e += m_f;
        m_u -= m_f;
        if (!bottom_up) {
            if ((double)m_f > (double)m_u / kAlpha) {
                bottom_up = true;
                hipLaunchKernelGGL(bfs_fill_kernel, dim3((unsigned)std::min<int64_t>(2048, L.words / 256 + 1)), dim3(256),
                                   0, s, fcur, L.words);
                hipLaunchKernelGGL(bfs_q2b_kernel, dim3((unsigned)std::min<int64_t>(4096, n_f / 256 + 1)), dim3(256), 0, s,
                                   qnext, n_f, fcur);
                if (int rc = launch_status("bfs_q2b_kernel")) return rc;
            } else {
                std::swap(qcur, qnext);
            }
        } else {
            if ((double)n_f < (double)V / kBeta) {
                bottom_up = false;
                hipLaunchKernelGGL(bfs_zero_counters_kernel, dim3(1), dim3(64), 0, s, ctr);
                hipLaunchKernelGGL(bfs_b2q_kernel, dim3((unsigned)std::min<int64_t>(4096, L.words / 256 + 1)), dim3(256), 0,
                                   s, fnext, L.words, qcur, &ctr->next_count);
                if (int rc = launch_status("bfs_b2q_kernel")) return rc;
            } else {
                std::swap(fcur, fnext);
            }
        }
    }
    if (stats) {
        stats->levels = depth + 1;
        stats->topdown_steps = td;
        stats->bottomup_steps = bu;
        stats->reached_vertices = reached_v;
        stats->reached_edges = reached_e;
    }
    return XD_OK;
}

}  // extern "C"
