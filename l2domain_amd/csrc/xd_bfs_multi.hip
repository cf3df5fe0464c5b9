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
//   claims: a visited bitmap (V bits, resident in every XCD's L2) filters with a plain load
//     (it holds every vertex claimed in earlier levels); a compare-and-swap of level[dst]
//     from 0xFFFFFFFF to depth + 1 decides, and the winner sets the bitmap bit with an
//     atomic whose result it does not wait for. (A 64-bit atomicOr on the bitmap as the
//     claim put 512 vertices on each contended line and made every claim slow.)
//   expansion: a group of G lanes per frontier vertex walks its adjacency list, eight
//     neighbours per lane and step with their loads and claims issued together (G = the
//     power of two nearest an eighth of the mean degree, at most 64).
//   appends: winners are staged in a per-wave LDS buffer (ballot + mbcnt) and flushed 256 at
//     a time with one atomicAdd; each frontier is split into 8 sub-queues, one per producing
//     XCD slot (workgroup mod 8), so the flushes spread over 8 counters. A counter taking one
//     atomic per wave and step was the bound of an earlier version (memory-side atomics on
//     one address serialise).
//   queues: two frontiers per level (one per I/O die, chosen by work_side[v]); XCD-aware:
//     the workgroups of die d (XCDs 4d..4d+3) consume frontier d, and a winner goes to the
//     frontier of its own work side; rotated: die d consumes frontier 1 - d; oblivious: one
//     frontier, every workgroup. Three frontier pairs rotate, and the kernel of level k clears
//     the counters of the pair level k + 1 will fill, so the whole search is enqueued without
//     host round trips and without memsets.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "xd_common.hpp"

namespace xd {

constexpr uint32_t kMUnv = 0xffffffffu;
constexpr int kMThreads = 256;
constexpr int kMWaves = kMThreads / kWave;
constexpr int kMGrid = 2048;  // level kernels (a multiple of 8)

constexpr int kMSub = kNumXcd;   // sub-queues per frontier (one per producing XCD slot)
constexpr int kMStage = 256;     // staged winners per wave and frontier before a flush
constexpr int kMUnroll = 8;      // neighbours per lane and step

struct MultiLayout {
    size_t visited, queues, counts, total;
};

static size_t m_a256(size_t x) { return (x + 255) & ~(size_t)255; }

// queue q of level slot l (0..2), frontier f (0..1), sub-queue k (0..7): index (l*2+f)*8+k
static MultiLayout multi_layout(int32_t V) {
    MultiLayout L;
    const size_t words = ((size_t)V + 63) / 64;
    L.visited = 0;
    L.queues = m_a256(L.visited + words * 8);
    L.counts = m_a256(L.queues + (size_t)6 * kMSub * (size_t)V * 4);
    L.total = L.counts + 6 * kMSub * 4;
    return L;
}

__global__ void __launch_bounds__(kMThreads) multi_init_kernel(uint32_t *level, unsigned long long *visited,
                                                               uint32_t *counts, int32_t V) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t i = i0; i < V; i += stride) level[i] = kMUnv;
    for (int64_t i = i0; i < ((int64_t)V + 63) / 64; i += stride) visited[i] = 0ull;
    if (i0 < 6 * kMSub) counts[i0] = 0u;
}

// Claims v: true for the one thread that set its visited bit.
__device__ __forceinline__ bool multi_claim(unsigned long long *visited, int32_t v) {
    const unsigned long long bit = 1ull << (v & 63);
    unsigned long long *w = visited + (v >> 6);
    if (*w & bit) return false;  // bits only go from 0 to 1: a set bit is final
    return (atomicOr(w, bit) & bit) == 0ull;
}

// Per-wave staging of the winners of one level. Every call is made by the whole wave.
struct Stager {
    int32_t *buf;      // this wave's LDS buffer, kMStage entries per frontier
    uint32_t fill[2];  // wave-uniform
    int32_t *q[2];     // the sub-queue of each frontier this workgroup fills
    uint32_t *cnt[2];

    __device__ __forceinline__ void flush(int f) {
        const uint32_t n = fill[f];
        if (n == 0) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // the staged entries are visible to the wave
        const int lane = (int)__lane_id();
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(cnt[f], n);
        base = __shfl(base, 0);
        for (uint32_t k = (uint32_t)lane; k < n; k += kWave) q[f][base + k] = buf[f * kMStage + k];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // read before the buffer is refilled
        fill[f] = 0;
    }
    __device__ __forceinline__ void append(bool take, uint32_t f_of, int32_t v) {
        const int lane = (int)__lane_id();
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const uint64_t m = __ballot(take && f_of == (uint32_t)f);
            if (m == 0) continue;
            const uint32_t c = (uint32_t)__popcll(m);
            if (fill[f] + c > (uint32_t)kMStage) flush(f);
            if (take && f_of == (uint32_t)f) buf[f * kMStage + fill[f] + (uint32_t)__popcll(m & ((1ull << lane) - 1ull))] = v;
            fill[f] += c;
        }
    }
};

// Position i of a frontier made of kMSub sub-queues (counts c[0..7], concatenated in order).
__device__ __forceinline__ int32_t sub_index(uint32_t i, const uint32_t *pre, const int32_t *q0, int32_t V) {
    int k = 0;
#pragma unroll
    for (int j = 1; j < kMSub; ++j) k += i >= pre[j] ? 1 : 0;
    return q0[(size_t)k * V + (i - pre[k])];
}

__global__ void __launch_bounds__(kMThreads)
multi_seed_kernel(const int32_t *__restrict__ sources, int32_t nsrc, const uint8_t *__restrict__ work_side, int routed,
                  uint32_t *__restrict__ level, unsigned long long *visited, int32_t *queues, uint32_t *counts,
                  int32_t V) {
    __shared__ int32_t sbuf[kMWaves][2 * kMStage];
    const int wave = (int)threadIdx.x / kWave;
    const int k = (int)blockIdx.x % kMSub;
    Stager st{sbuf[wave], {0u, 0u}, {queues + (size_t)k * V, queues + (size_t)(kMSub + k) * V},
              {counts + k, counts + kMSub + k}};
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool take = false;
    int32_t v = 0;
    uint32_t f = 0;
    if (i < nsrc) {
        v = sources[i];
        take = multi_claim(visited, v);
        if (take) {
            level[v] = 0u;
            f = routed ? (uint32_t)(work_side[v] & 1u) : 0u;
        }
    }
    st.append(take, f, v);
    st.flush(0);
    st.flush(1);
}

// One top-down level: consumes frontier pair `cur`, fills pair (cur + 1) % 3 and clears the
// counters of pair (cur + 2) % 3. A group of G = 2^lg lanes takes one frontier vertex, and
// each lane handles kMUnroll neighbours per step with their loads issued together.
__global__ void __launch_bounds__(kMThreads)
multi_level_kernel(const int32_t *__restrict__ rowptr, const int32_t *__restrict__ col,
                   const uint8_t *__restrict__ work_side, uint32_t *__restrict__ level, unsigned long long *visited,
                   int32_t *queues, uint32_t *counts, int32_t V, uint32_t depth, int lg, int mode, int cur,
                   XcdHint xh) {
    __shared__ int32_t sbuf[kMWaves][2 * kMStage];
    report_xcd(xh);
    const int nxt = (cur + 1) % 3, clr = (cur + 2) % 3;
    const int b = (int)blockIdx.x, grid = (int)gridDim.x;
    if (b == 0 && threadIdx.x < 2 * kMSub) counts[2 * kMSub * clr + threadIdx.x] = 0u;
    const bool routed = mode != XD_MODE_OBLIVIOUS;
    int rank, nwg;
    uint32_t side = 0;
    if (!routed) {
        rank = b;
        nwg = grid;
    } else {
        rank = die_rank(b, xh);
        nwg = grid / 2;
        side = wg_die(b, xh) ^ (mode == XD_MODE_ROTATED ? 1u : 0u);
    }
    // the frontier this workgroup consumes: kMSub sub-queues, prefix sums of their lengths
    const uint32_t *ccnt = counts + (size_t)(2 * cur + side) * kMSub;
    const int32_t *cq = queues + (size_t)(2 * cur + side) * kMSub * V;
    uint32_t pre[kMSub];
    uint32_t n = 0;
#pragma unroll
    for (int k = 0; k < kMSub; ++k) {
        pre[k] = n;
        n += ccnt[k];
    }
    const int wave = (int)threadIdx.x / kWave;
    const int sq = b % kMSub;  // the sub-queue this workgroup fills
    Stager st{sbuf[wave], {0u, 0u},
              {queues + ((size_t)(2 * nxt) * kMSub + sq) * V, queues + ((size_t)(2 * nxt + 1) * kMSub + sq) * V},
              {counts + (size_t)(2 * nxt) * kMSub + sq, counts + (size_t)(2 * nxt + 1) * kMSub + sq}};
    const int G = 1 << lg;
    const int lane = (int)__lane_id();
    const int sub = lane & (G - 1);
    const uint32_t per_wave = (uint32_t)(kWave >> lg);  // frontier vertices per wave and pass
    const uint32_t stride = (uint32_t)nwg * kMWaves * per_wave;
    for (uint32_t base = ((uint32_t)rank * kMWaves + (uint32_t)wave) * per_wave; base < n; base += stride) {
        const uint32_t i = base + (uint32_t)(lane >> lg);
        int32_t beg = 0, end = 0;
        if (i < n) {
            const int32_t v = sub_index(i, pre, cq, V);
            beg = rowptr[v];
            end = rowptr[v + 1];
        }
        // the wave walks the longest list of its vertices in lock step, so that every lane
        // takes part in the ballots and flushes
        int32_t len = end - beg;
        for (int off = kWave / 2; off >= 1; off >>= 1) len = max(len, __shfl_xor(len, off));
        for (int32_t jb = 0; jb < len; jb += G * kMUnroll) {
            int32_t dst[kMUnroll];
            unsigned long long w[kMUnroll];
#pragma unroll
            for (int u = 0; u < kMUnroll; ++u) {
                const int32_t e = beg + jb + sub + u * G;
                dst[u] = e < end ? col[e] : -1;
            }
#pragma unroll
            for (int u = 0; u < kMUnroll; ++u) w[u] = dst[u] >= 0 ? visited[dst[u] >> 6] : ~0ull;
            // the claim is a compare-and-swap on the vertex's own level entry (16 vertices per
            // line, where a bitmap word shares its line with 512 and serialises), and all
            // claims of a step are issued before any result is used. A claim's result is left
            // undefined on the path that skips it and read only where it was issued: a value
            // merged at a branch join with a constant makes the compiler wait for the atomic
            // right there, which put the 8 claims of a step one after another. The work side
            // is read with the claim, in the home modes, and likewise left undefined elsewhere.
            // All filters are decided before the first claim is issued: once a conditional
            // atomic is in flight the compiler cannot count what is outstanding, and it would
            // wait for everything (the claim included) before testing the next bitmap word.
            bool pass[kMUnroll];
            uint32_t old[kMUnroll], f[kMUnroll];
#pragma unroll
            for (int u = 0; u < kMUnroll; ++u) pass[u] = dst[u] >= 0 && !(w[u] & (1ull << (dst[u] & 63)));
            uint32_t fw[kMUnroll];
#pragma unroll
            for (int u = 0; u < kMUnroll; ++u)
                if (pass[u]) {
                    old[u] = atomicCAS(level + dst[u], kMUnv, depth + 1u);
                    if (routed) fw[u] = work_side[dst[u]];
                }
            bool take[kMUnroll];
#pragma unroll
            for (int u = 0; u < kMUnroll; ++u) {
                take[u] = pass[u] && old[u] == kMUnv;
                f[u] = (routed && take[u]) ? (fw[u] & 1u) : 0u;
                if (take[u]) atomicOr(visited + (dst[u] >> 6), 1ull << (dst[u] & 63));  // filter of later levels
            }
#pragma unroll
            for (int u = 0; u < kMUnroll; ++u) st.append(take[u], f[u], dst[u]);
        }
    }
    st.flush(0);
    st.flush(1);
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
    // lanes per frontier vertex: the power of two nearest mean degree / kMUnroll, in [1, 64]
    const double mean = (double)nnz / (double)V / kMUnroll;
    int lg = 0;
    while (lg < 6 && (double)(2 << lg) <= mean * 1.5) ++lg;

    const int igrid = (int)std::min<int64_t>(4096, ((int64_t)V + kMThreads - 1) / kMThreads);
    launch("multi_init_kernel", multi_init_kernel, dim3(std::max(igrid, 1)), dim3(kMThreads), 0, s, level, visited, counts, V);
    if (int rc = launch_status("multi_init_kernel")) return rc;
    if (num_sources > 0) {
        launch("multi_seed_kernel", multi_seed_kernel, dim3((num_sources + kMThreads - 1) / kMThreads), dim3(kMThreads), 0, s,
                           sources, num_sources, work_side, routed, level, visited, queues, counts, V);
        if (int rc = launch_status("multi_seed_kernel")) return rc;
    }
    const XcdHint xh = xcd_hint(s);
    for (int32_t d = 0; d < max_depth; ++d) {
        launch("multi_level_kernel", multi_level_kernel, dim3(kMGrid), dim3(kMThreads), 0, s, rowptr, col, work_side, level,
                           visited, queues, counts, V, (uint32_t)d, lg, mode, d % 3, xh);
        if (int rc = launch_status("multi_level_kernel")) return rc;
    }
    return XD_OK;
}

}  // extern "C"
