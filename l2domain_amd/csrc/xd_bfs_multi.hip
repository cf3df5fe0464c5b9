// Multi-source, fixed-depth, top-down BFS over a directed CSR graph: the reference's own BFS
// workload. level[v] = the distance from the nearest source when it is at most max_depth,
// 0xFFFFFFFF otherwise.
//
// Reference: applications/bfs/src/bfs.cu
//   init_dist_kernel / seed_baseline_kernel / seed_side_kernel (151-174): every source at
//     distance 0 in the first frontier (per-side frontiers for the aware run);
//   luo_baseline_level_kernel (215-252): one top-down level, atomicCAS claims, winners
//     appended through LDS-binned queues with one global atomicAdd per flush (176-213);
//   luo_side_level_kernel (254-308): the SMs of each L2 side consume that side's frontier,
//     and winners go to the frontier of work_side[dst]; the host enqueues max_depth levels
//     (449-491); swapped = each side consumes the other side's frontier (invert, :258).
//
// MI355X design.
//   claims: a visited bitmap (V bits, resident in every XCD's L2) filters with a plain load,
//     then a 64-bit atomicOr decides; the winner writes level[dst] = depth + 1.
//   expansion: a group of G lanes per frontier vertex walks its adjacency list (G = the
//     power of two nearest the mean degree, at most 64), so the list is read in coalesced
//     runs; winners are appended with one atomicAdd per wave and target queue (ballot +
//     mbcnt), no LDS staging and no overflow.
//   queues: two per level (one per I/O die, chosen by work_side[v]); XCD-aware: the
//     workgroups of die d (XCDs 4d..4d+3) consume queue d, and a winner goes to the queue of
//     its own work side; rotated: die d consumes queue 1 - d; oblivious: one queue, every
//     workgroup. Three queue pairs rotate, and the kernel of level k clears the counters of
//     the pair level k + 1 will fill, so the whole search is enqueued without host round
//     trips and without memsets.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "xd_common.hpp"

namespace xd {

constexpr uint32_t kMUnv = 0xffffffffu;
constexpr int kMThreads = 256;
constexpr int kMWaves = kMThreads / kWave;
constexpr int kMGrid = 2048;  // level kernels (a multiple of 8)

struct MultiLayout {
    size_t visited, queues, counts, total;
};

static size_t m_a256(size_t x) { return (x + 255) & ~(size_t)255; }

static MultiLayout multi_layout(int32_t V) {
    MultiLayout L;
    const size_t words = ((size_t)V + 63) / 64;
    L.visited = 0;
    L.queues = m_a256(L.visited + words * 8);
    L.counts = m_a256(L.queues + (size_t)6 * (size_t)V * 4);  // 3 levels x 2 dies
    L.total = L.counts + 256;
    return L;
}

__global__ void __launch_bounds__(kMThreads) multi_init_kernel(uint32_t *level, unsigned long long *visited,
                                                               uint32_t *counts, int32_t V) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t i = i0; i < V; i += stride) level[i] = kMUnv;
    for (int64_t i = i0; i < ((int64_t)V + 63) / 64; i += stride) visited[i] = 0ull;
    if (i0 < 6) counts[i0] = 0u;
}

// Appends v (for the lanes with take == true) to queue[side] with one atomic per wave and side.
__device__ __forceinline__ void multi_append(bool take, uint32_t side, int32_t v, int32_t *q0, int32_t *q1,
                                             uint32_t *cnt) {
    const int lane = (int)__lane_id();
#pragma unroll
    for (uint32_t s = 0; s < 2; ++s) {
        const uint64_t m = __ballot(take && side == s);
        if (m == 0) continue;
        const int leader = __ffsll((long long)m) - 1;
        uint32_t base = 0;
        if (lane == leader) base = atomicAdd(&cnt[s], (uint32_t)__popcll(m));
        base = __shfl(base, leader);
        if (take && side == s) {
            const uint32_t pos = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
            (s == 0 ? q0 : q1)[pos] = v;
        }
    }
}

// Claims v at distance lvl: true for the one thread that set its visited bit.
__device__ __forceinline__ bool multi_claim(unsigned long long *visited, int32_t v) {
    const unsigned long long bit = 1ull << (v & 63);
    unsigned long long *w = visited + (v >> 6);
    if (*w & bit) return false;  // bits only go from 0 to 1: a set bit is final
    return (atomicOr(w, bit) & bit) == 0ull;
}

__global__ void __launch_bounds__(kMThreads)
multi_seed_kernel(const int32_t *__restrict__ sources, int32_t nsrc, const uint8_t *__restrict__ work_side, int routed,
                  uint32_t *__restrict__ level, unsigned long long *visited, int32_t *queues, uint32_t *counts,
                  int32_t V) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool take = false;
    int32_t v = 0;
    uint32_t side = 0;
    if (i < nsrc) {
        v = sources[i];
        take = multi_claim(visited, v);
        if (take) {
            level[v] = 0u;
            side = routed ? (uint32_t)(work_side[v] & 1u) : 0u;
        }
    }
    multi_append(take, side, v, queues, queues + V, counts);
}

// One top-down level: consumes queue pair `cur`, fills pair (cur + 1) % 3 and clears the
// counters of pair (cur + 2) % 3. lg = log2 of the lanes per frontier vertex.
__global__ void __launch_bounds__(kMThreads)
multi_level_kernel(const int32_t *__restrict__ rowptr, const int32_t *__restrict__ col,
                   const uint8_t *__restrict__ work_side, uint32_t *__restrict__ level, unsigned long long *visited,
                   int32_t *queues, uint32_t *counts, int32_t V, uint32_t depth, int lg, int mode, int cur) {
    const int nxt = (cur + 1) % 3, clr = (cur + 2) % 3;
    const int b = (int)blockIdx.x, grid = (int)gridDim.x;
    if (b == 0 && threadIdx.x < 2) counts[2 * clr + threadIdx.x] = 0u;
    const bool routed = mode != XD_MODE_OBLIVIOUS;
    int rank, nwg;
    uint32_t side = 0;
    if (!routed) {
        rank = b;
        nwg = grid;
    } else {
        rank = (b / kNumXcd) * (kNumXcd / 2) + (b % (kNumXcd / 2));
        nwg = grid / 2;
        side = wg_die(b) ^ (mode == XD_MODE_ROTATED ? 1u : 0u);
    }
    const uint32_t n = counts[2 * cur + side];
    const int32_t *q = queues + (size_t)(2 * cur + side) * V;
    int32_t *n0 = queues + (size_t)(2 * nxt) * V, *n1 = n0 + V;
    uint32_t *ncnt = counts + 2 * nxt;
    const int G = 1 << lg;
    const int lane = (int)__lane_id(), wave = (int)threadIdx.x / kWave;
    const int sub = lane & (G - 1);
    const uint32_t per_wave = (uint32_t)(kWave >> lg);  // frontier vertices per wave and pass
    const uint32_t stride = (uint32_t)nwg * kMWaves * per_wave;
    for (uint32_t base = ((uint32_t)rank * kMWaves + (uint32_t)wave) * per_wave; base < n; base += stride) {
        const uint32_t i = base + (uint32_t)(lane >> lg);
        int32_t beg = 0, end = 0;
        if (i < n) {
            const int32_t v = q[i];
            beg = rowptr[v];
            end = rowptr[v + 1];
        }
        // the wave walks the longest list of its vertices; every lane takes part in the
        // appends, so the ballots see the whole wave
        int32_t len = end - beg;
        for (int off = kWave / 2; off >= G; off >>= 1) len = max(len, __shfl_xor(len, off));
        for (int32_t j = sub; j < len; j += G) {
            bool take = false;
            int32_t dst = 0;
            uint32_t ds = 0;
            if (beg + j < end) {
                dst = col[beg + j];
                take = multi_claim(visited, dst);
                if (take) {
                    level[dst] = depth + 1u;
                    ds = routed ? (uint32_t)(work_side[dst] & 1u) : 0u;
                }
            }
            multi_append(take, ds, dst, n0, n1, ncnt);
        }
    }
}

}  // namespace xd

using namespace xd;

extern "C" {

size_t xd_bfs_multi_workspace_size(int32_t num_vertices) {
    if (num_vertices <= 0) return 0;
    return multi_layout(num_vertices).total;
}

int xd_bfs_multi(const int32_t *rowptr, const int32_t *col, int32_t num_vertices, int64_t nnz, const int32_t *sources,
                 int32_t num_sources, int32_t max_depth, const uint8_t *work_side, uint32_t *level, int mode,
                 void *workspace, size_t workspace_bytes, void *stream) {
    const int32_t V = num_vertices;
    XD_REQUIRE(V > 0 && rowptr != nullptr && level != nullptr, "xd_bfs_multi: empty graph or NULL rowptr/level");
    XD_REQUIRE(nnz >= 0 && nnz < (1ll << 31) && (nnz == 0 || col != nullptr), "xd_bfs_multi: nnz out of range");
    XD_REQUIRE(num_sources >= 0 && (num_sources == 0 || sources != nullptr), "xd_bfs_multi: bad sources");
    XD_REQUIRE(max_depth >= 0 && max_depth < (1 << 30), "xd_bfs_multi: max_depth out of range");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "xd_bfs_multi: bad mode");
    XD_REQUIRE(mode == XD_MODE_OBLIVIOUS || work_side != nullptr, "xd_bfs_multi: the home modes need work_side");
    const MultiLayout L = multi_layout(V);
    if (workspace == nullptr || workspace_bytes < L.total || !aligned16(workspace))
        return fail(XD_ERR_WORKSPACE, "xd_bfs_multi: workspace missing, misaligned or smaller than "
                                      "xd_bfs_multi_workspace_size()");
    hipStream_t s = (hipStream_t)stream;
    char *ws = static_cast<char *>(workspace);
    unsigned long long *visited = reinterpret_cast<unsigned long long *>(ws + L.visited);
    int32_t *queues = reinterpret_cast<int32_t *>(ws + L.queues);
    uint32_t *counts = reinterpret_cast<uint32_t *>(ws + L.counts);
    const int routed = mode != XD_MODE_OBLIVIOUS ? 1 : 0;
    // lanes per frontier vertex: the power of two nearest the mean degree, in [1, 64]
    const double mean = (double)nnz / (double)V;
    int lg = 0;
    while (lg < 6 && (double)(2 << lg) <= mean * 1.5) ++lg;

    KernelTimer kt("bfs_multi", s);
    const int igrid = (int)std::min<int64_t>(4096, ((int64_t)V + kMThreads - 1) / kMThreads);
    hipLaunchKernelGGL(multi_init_kernel, dim3(std::max(igrid, 1)), dim3(kMThreads), 0, s, level, visited, counts, V);
    if (int rc = launch_status("multi_init_kernel")) return rc;
    if (num_sources > 0) {
        hipLaunchKernelGGL(multi_seed_kernel, dim3((num_sources + kMThreads - 1) / kMThreads), dim3(kMThreads), 0, s,
                           sources, num_sources, work_side, routed, level, visited, queues, counts, V);
        if (int rc = launch_status("multi_seed_kernel")) return rc;
    }
    for (int32_t d = 0; d < max_depth; ++d) {
        hipLaunchKernelGGL(multi_level_kernel, dim3(kMGrid), dim3(kMThreads), 0, s, rowptr, col, work_side, level,
                           visited, queues, counts, V, (uint32_t)d, lg, mode, d % 3);
        if (int rc = launch_status("multi_level_kernel")) return rc;
    }
    return XD_OK;
}

}  // extern "C"
