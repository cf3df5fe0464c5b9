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
//   state: level[V]; a visited bitmap and three rotating frontier bitmaps (u64 words, 512 KiB
//   each at 2^22 vertices, resident in every XCD's L2); a control block. There is no frontier
//   queue: every level writes the next frontier as a bitmap only, and a top-down level reads
//   its frontier from the bitmap. (Appending the winners of a top-down level to a queue as
//   they claim costs one atomic per wave on a single counter, which serialises: a hub's
//   expansion took 54 us of a 260 us search; a conversion pass from bitmap to queue before
//   every top-down level cost a launch per level.) Each level zeroes the bitmap the level
//   after it will fill.
//   top-down: a wave per frontier bitmap word, lane l expanding vertex 64 w + l when its bit
//     is set (hubs above kBigDeg are expanded by the whole grid in a second kernel); a claim
//     is a 64-bit atomicOr on the visited word.
//   bottom-up: every unvisited vertex scans its neighbours until one is in the frontier
//     bitmap; a wave covers one 64-vertex block, i.e. exactly one bitmap word, so it updates
//     its visited and next words with plain stores. Oblivious mode walks the blocks in order;
//     XCD-aware mode lets each I/O die take the blocks whose adjacency starts in memory homed
//     on that die (xd_home_map of col), so the neighbour lists are read from the near die;
//     rotated hands each die the far blocks.
//   direction: top-down -> bottom-up when m_f > m_u / 14, bottom-up -> top-down when
//     n_f < V / 24 (Beamer, Asanovic, Patterson, SC'12). No control kernel runs between
//     levels: every workgroup adds its level totals to that level's accumulator (two
//     memory-side atomics), and every workgroup of the next level recomputes the decision
//     itself from the previous control state and that accumulator (the same few scalar
//     steps everywhere, so all agree); workgroup 0 publishes the new state into the other of
//     two buffers. The host enqueues levels in batches (level, hub expansion) of six, then
//     four, and replays the same step on the copied state once per batch; the kernels of
//     levels enqueued after the search ended return at once.
#include <hip/hip_runtime.h>

#include <string.h>

#include <algorithm>
#include <chrono>
#include <memory>
#include <mutex>
#include <vector>

#include "xd_common.hpp"

namespace xd {

constexpr uint32_t kUnv = 0xffffffffu;
constexpr int kBfsThreads = 256;
constexpr int kBfsGrid = 2048;      // fixed grid of the level kernels (multiple of 8)
constexpr int kBigGrid = 1024;      // grid of the hub expansion
constexpr int32_t kBigDeg = 4096;   // top-down: larger lists are expanded by the whole grid
constexpr double kAlpha = 14.0, kBeta = 24.0;
constexpr int kFirstBatch = 6;      // levels enqueued before the first host round trip
constexpr int kLevelBatch = 4;      // levels enqueued per later round trip
constexpr int kTdWords = 4;         // frontier words a wave loads at once in a top-down level
constexpr int kTopDown = 0, kBottomUp = 1, kDone = 2;

// S_j: the control state after j completed levels.
struct BfsCtl {
    int32_t dir;    // direction of level j + 1: kTopDown, kBottomUp or kDone
    int32_t depth;  // completed levels
    int32_t td_steps, bu_steps;
    long long n_f;  // frontier vertices
    long long m_f;  // frontier edges
    long long m_u;  // edges of unvisited vertices
    long long reached_v, reached_e;
};

// Totals of one level, accumulated by every workgroup of its level and hub kernels into
// kAccSlots slots of their own 128-byte line (workgroup b adds into slot b mod kAccSlots):
// thousands of same-address memory-side atomics would serialise at the line's atomic unit.
constexpr int kAccSlots = 64;
struct alignas(128) BfsAccSlot {
    unsigned long long verts, edges;
    unsigned long long pad[14];
};
struct BfsAcc {
    BfsAccSlot slot[kAccSlots];
    unsigned long long big;  // hub vertices the level deferred to the grid-wide expansion
    unsigned long long pad[15];
};

// S_j lives in s[j % 2] (level j + 1 reads it: level L publishes S_{L-1}); level L
// accumulates into acc[L % 3] and clears acc[(L + 1) % 3] for the level after it.
struct BfsCtlBlock {
    BfsCtl s[2];
    BfsAcc acc[3];
};

// S_{j+1} from S_j and level j + 1's totals (the host replays the same step).
__host__ __device__ inline BfsCtl ctl_step(BfsCtl c, unsigned long long v, unsigned long long e, int32_t V) {
    if (c.dir == kDone) return c;
    const int dir = c.dir;
    if (dir == kTopDown) ++c.td_steps;
    else ++c.bu_steps;
    c.depth += 1;
    c.n_f = (long long)v;
    c.m_f = (long long)e;
    if (v == 0) {
        c.dir = kDone;
        return c;
    }
    c.reached_v += (long long)v;
    c.reached_e += (long long)e;
    c.m_u -= (long long)e;
    if (dir == kTopDown) {
        if ((double)c.m_f > (double)c.m_u / kAlpha) c.dir = kBottomUp;
    } else if ((double)c.n_f < (double)V / kBeta) {
        c.dir = kTopDown;
    }
    return c;
}

struct BfsLayout {
    size_t visited, front[3], big, ctl, route, total;
    int64_t words, nblocks;
};

static size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }

// Route buffer: two block counters, then the per-die block lists (nblocks entries each).
constexpr size_t kRouteHeader = 256;
static size_t route_bytes(int32_t V) { return kRouteHeader + 2 * 4 * (size_t)(((int64_t)V + 63) / 64); }

static BfsLayout bfs_layout(int32_t V, int64_t nnz) {
    (void)nnz;
    BfsLayout L{};
    L.words = ((int64_t)V + 63) / 64;
    L.nblocks = ((int64_t)V + 63) / 64;
    size_t o = 0;
    L.ctl = o;
    o = a256(o + sizeof(BfsCtlBlock));
    L.visited = o;
    o = a256(o + 8 * (size_t)L.words);
    for (int i = 0; i < 3; ++i) {
        L.front[i] = o;
        o = a256(o + 8 * (size_t)L.words);
    }
    L.big = o;
    o = a256(o + 4 * (size_t)V);
    L.route = o;  // per-call block lists when the caller passes no route
    o = a256(o + route_bytes(V));
    L.total = o;
    return L;
}

// Device view of the workspace.
struct BfsState {
    const int32_t *rowptr;
    const int32_t *col;
    int32_t V;
    int64_t words;
    uint32_t *level;
    unsigned long long *visited;
    unsigned long long *front[3];
    int32_t *big;
    BfsCtlBlock *ctl;
};

__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
    return v;
}

// Workgroup sum of (v, e) through LDS; thread 0 gets the totals.
__device__ __forceinline__ void block_sum2(unsigned long long &v, unsigned long long &e) {
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
        v = tv;
        e = te;
    }
}

__global__ void __launch_bounds__(256) bfs_init_kernel(BfsState st, int32_t src, int64_t nnz) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t i = t0; i < st.V; i += stride) st.level[i] = (i == src) ? 0u : kUnv;
    for (int64_t w = t0; w < st.words; w += stride) {
        const unsigned long long b = (w == src / 64) ? (1ull << (src % 64)) : 0ull;
        st.visited[w] = b;
        st.front[0][w] = b;  // the first level's frontier: the source
        st.front[1][w] = 0ull;
    }
    if (t0 == 0) {
        const long long deg = st.rowptr[src + 1] - st.rowptr[src];
        BfsCtl c{};
        c.dir = kTopDown;
        c.n_f = 1;
        c.m_f = deg;
        c.m_u = nnz - deg;
        c.reached_v = 1;
        c.reached_e = deg;
        st.ctl->s[0] = c;
    }
    // the accumulators of levels 1 and 2 (level L clears the one of level L + 1 from then on)
    if (t0 < 2 * kAccSlots) {
        BfsAccSlot &a = st.ctl->acc[1 + t0 / kAccSlots].slot[t0 % kAccSlots];
        a.verts = 0ull;
        a.edges = 0ull;
    }
    if (t0 < 3) st.ctl->acc[t0].big = 0ull;
}

// The control state of level L (S_{L-1}) as every workgroup of the level derives it: the
// first wave sums level L - 1's slots; workgroup 0 publishes the state for level L + 1 and
// clears the accumulator of level L + 1. Returns the direction of level L; *heavy says
// whether more than 1/64 of the adjacency is still unvisited (the bottom-up walk of the home
// modes routes by home only then: in the sparse levels after that, nearly every block is
// already visited, so a wave's cost is its per-block loads, not the adjacency stream).
__device__ __forceinline__ int level_dir(const BfsState &st, int L, bool *heavy) {
    __shared__ int sdir, sheavy;
    if (threadIdx.x < kWave) {
        BfsCtl c = st.ctl->s[(L - 1) % 2];
        if (L >= 2) {
            const BfsAccSlot &a = st.ctl->acc[(L - 1) % 3].slot[threadIdx.x % kAccSlots];
            unsigned long long v = threadIdx.x < kAccSlots ? a.verts : 0ull;
            unsigned long long e = threadIdx.x < kAccSlots ? a.edges : 0ull;
            v = wave_sum_u64(v);
            e = wave_sum_u64(e);
            c = ctl_step(st.ctl->s[L % 2], v, e, st.V);  // S_{L-2} and level L - 1's totals
            if (blockIdx.x == 0 && threadIdx.x == 0) st.ctl->s[(L - 1) % 2] = c;
        }
        if (threadIdx.x == 0) {
            sdir = c.dir;
            sheavy = c.m_u > (c.m_u + c.reached_e) / 64;
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < kAccSlots) {
        BfsAccSlot &n = st.ctl->acc[(L + 1) % 3].slot[threadIdx.x];
        n.verts = 0ull;
        n.edges = 0ull;
        if (threadIdx.x == 0) st.ctl->acc[(L + 1) % 3].big = 0ull;
    }
    __syncthreads();
    *heavy = sheavy != 0;
    return sdir;
}

// Adds a workgroup's level totals (thread 0 holds them after block_sum2).
__device__ __forceinline__ void add_totals(const BfsState &st, int L, unsigned long long v, unsigned long long e) {
    if (threadIdx.x == 0) {
        BfsAccSlot &a = st.ctl->acc[L % 3].slot[blockIdx.x % kAccSlots];
        if (v) atomicAdd(&a.verts, v);
        if (e) atomicAdd(&a.edges, e);
    }
}

// Claims v for level `lvl`; returns true if this thread won it. Visited bits only go from 0
// to 1, so a plain (possibly stale) read can only show a set bit as clear; the atomicOr then
// decides.
__device__ __forceinline__ bool claim(unsigned long long *visited, uint32_t *level, int32_t v, uint32_t lvl) {
    const unsigned long long bit = 1ull << (v & 63);
    unsigned long long *w = visited + (v >> 6);
    if (__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) & bit) return false;
    if (atomicOr(w, bit) & bit) return false;
    level[v] = lvl;
    return true;
}

// A top-down claim of v by this lane: level, visited and next bitmap.
__device__ __forceinline__ void td_visit(const BfsState &st, bool have, int32_t v, uint32_t lvl,
                                         unsigned long long *next_bits, unsigned long long &my_verts,
                                         unsigned long long &my_edges) {
    if (have && claim(st.visited, st.level, v, lvl)) {
        atomicOr(&next_bits[v >> 6], 1ull << (v & 63));
        my_verts += 1;
        my_edges += (unsigned long long)(st.rowptr[v + 1] - st.rowptr[v]);
    }
}

// Top-down claims of up to 64 consecutive entries of one adjacency list, one per lane (lanes
// without an entry have have == false). Lanes whose vertices share a visited word form
// contiguous runs when the list is sorted, as a hub's lists are here: a segmented OR across
// each run gathers the bits that still look clear, the run's last lane claims them with one
// atomicOr and sets the won ones in the next bitmap with one more, and every lane learns from
// the returned word whether it won (the first lane holding a bit, should a list repeat a
// vertex). Unsorted lists only make the runs shorter.
__device__ __forceinline__ void td_visit_runs(const BfsState &st, bool have, int32_t v, uint32_t lvl,
                                              unsigned long long *next_bits, unsigned long long &my_verts,
                                              unsigned long long &my_edges) {
    const int lane = lane_id();
    const int32_t w = have ? (v >> 6) : -1 - lane;  // a lane without an entry is a run of its own
    const unsigned long long bit = have ? 1ull << (v & 63) : 0ull;
    const unsigned long long cur =
        __hip_atomic_load(st.visited + (have ? w : 0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const unsigned long long mine = (cur & bit) ? 0ull : bit;
    // Every shuffle runs on the whole wave and its result is pinned by an empty asm: left to
    // itself the compiler sinks a shuffle feeding a `||` or `?:` into the branch that needs
    // it, where the lanes it reads from are switched off and read as 0.
    int32_t wu = __shfl_up(w, 1, kWave);
    asm volatile("" : "+v"(wu));
    const bool head = (lane == 0) | (wu != w);
    const uint64_t heads = __ballot(head);
    unsigned long long x = mine;  // OR of `mine` from the run's head to this lane
    bool f = head;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        unsigned long long y = __shfl_up(x, d, kWave);
        int fy = __shfl_up(f ? 1 : 0, d, kWave);
        asm volatile("" : "+v"(y), "+v"(fy));
        const bool on = lane >= d;
        x = (on & !f) ? (x | y) : x;
        f = f | (on & (fy != 0));
    }
    unsigned long long xu = __shfl_up(x, 1, kWave);
    asm volatile("" : "+v"(xu));
    const unsigned long long before = head ? 0ull : xu;  // earlier lanes of the run
    const unsigned long long rest = lane == kWave - 1 ? 0ull : (heads >> (lane + 1));
    const bool tail = rest & 1ull || lane == kWave - 1;
    unsigned long long old = 0;
    if (tail && x) old = atomicOr(st.visited + w, x);
    const int tl = rest ? lane + __builtin_ctzll(rest) : kWave - 1;  // the run's last lane
    unsigned long long run_old = __shfl(old, tl, kWave);
    asm volatile("" : "+v"(run_old));
    if (mine & ~before & ~run_old) {
        st.level[v] = lvl;
        my_edges += (unsigned long long)(st.rowptr[v + 1] - st.rowptr[v]);
    }
    if (tail && x) {
        const unsigned long long won = x & ~old;
        if (won) {
            atomicOr(&next_bits[w], won);
            my_verts += (unsigned long long)__builtin_popcountll(won);
        }
    }
}

// Bottom-up over two 64-vertex blocks starting at v0a and v0b (multiples of 64; the second
// only if hasb): exactly bitmap words v0a / 64 and v0b / 64, which no other wave touches
// during this level. Every lane scans the lists of its vertex in both blocks together, so
// two chains of (list entry, frontier word) loads are in flight, until it finds a neighbour
// in the frontier or runs out of neighbours. Loads are unconditional (a finished chain reads
// entry 0, which exists whenever a chain is active), so no load sits under a branch.
__device__ __forceinline__ void bu_blocks(const BfsState &st, int32_t v0a, int32_t v0b, bool hasb,
                                          const unsigned long long *front, unsigned long long *next_bits,
                                          uint32_t lvl, unsigned long long &my_verts, unsigned long long &my_edges) {
    const int lane = lane_id();
    const int32_t va = v0a + lane, vb = v0b + lane;
    const int32_t wa = v0a >> 6, wb = v0b >> 6;
    const unsigned long long visa = st.visited[wa];
    const unsigned long long visb = st.visited[hasb ? wb : wa];
    bool ta = va < st.V && !((visa >> lane) & 1ull);  // still searching
    bool tb = hasb && vb < st.V && !((visb >> lane) & 1ull);
    const int32_t ia = ta ? va : 0, ib = tb ? vb : 0;
    int32_t ea = st.rowptr[ia], eb = st.rowptr[ib];
    int32_t ra = st.rowptr[ia + 1], rb = st.rowptr[ib + 1];
    asm volatile("" : "+v"(ea), "+v"(eb), "+v"(ra), "+v"(rb));
    const int32_t enda = ta ? ra : ea, endb = tb ? rb : eb;
    const int32_t dega = enda - ea, degb = endb - eb;
    bool fa = false, fb = false;
    for (;;) {
        const bool aa = ta && ea < enda, ab = tb && eb < endb;
        if (!(aa | ab)) break;
        // both chains' loads on every lane, pinned so the compiler cannot sink either under its
        // chain's condition (which would serialise the two chains again)
        int32_t ua = st.col[aa ? ea : 0];
        int32_t ub = st.col[ab ? eb : 0];
        asm volatile("" : "+v"(ua), "+v"(ub));
        unsigned long long fwa = front[ua >> 6];
        unsigned long long fwb = front[ub >> 6];
        asm volatile("" : "+v"(fwa), "+v"(fwb));
        const bool ha = aa && ((fwa >> (ua & 63)) & 1ull);
        const bool hb = ab && ((fwb >> (ub & 63)) & 1ull);
        fa = fa | ha;
        fb = fb | hb;
        ta = ta && !ha;
        tb = tb && !hb;
        ea += aa ? 1 : 0;
        eb += ab ? 1 : 0;
    }
    if (fa) {
        st.level[va] = lvl;
        my_verts += 1;
        my_edges += (unsigned long long)dega;
    }
    if (fb) {
        st.level[vb] = lvl;
        my_verts += 1;
        my_edges += (unsigned long long)degb;
    }
    const uint64_t ma = __ballot(fa), mb = __ballot(fb);
    if (lane == 0) {
        if (ma) {
            st.visited[wa] = visa | ma;
            next_bits[wa] = ma;
        }
        if (mb) {
            st.visited[wb] = visb | mb;
            next_bits[wb] = mb;
        }
    }
}

// One level in the direction the control block names.
__global__ void __launch_bounds__(kBfsThreads)
bfs_level_kernel(BfsState st, int L, int mode, const int32_t *__restrict__ blist,
                 const unsigned long long *__restrict__ bcount, int64_t nblocks, XcdHint xh) {
    report_xcd(xh);
    bool heavy = false;
    const int dir = level_dir(st, L, &heavy);
    if (dir == kDone) return;
    const uint32_t lvl = (uint32_t)L;
    const unsigned long long *cur_bits = st.front[(L - 1) % 3];
    unsigned long long *next_bits = st.front[L % 3];
    unsigned long long *later_bits = st.front[(L + 1) % 3];
    const int64_t tstride = (int64_t)gridDim.x * blockDim.x;
    const int64_t tid0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t w = tid0; w < st.words; w += tstride) later_bits[w] = 0ull;  // filled by the next level

    unsigned long long my_verts = 0, my_edges = 0;
    const int wave = (int)threadIdx.x / kWave;
    constexpr int kWavesPerWg = kBfsThreads / kWave;
    if (dir == kTopDown) {
        // a wave per frontier bitmap word: lane l expands vertex 64 w + l when its bit is set;
        // a wave's next kTdWords words are loaded together (one round trip, not one each)
        const int lane = lane_id();
        const int64_t wstride = (int64_t)gridDim.x * kWavesPerWg;
        for (int64_t w0 = (int64_t)blockIdx.x * kWavesPerWg + wave; w0 < st.words; w0 += kTdWords * wstride) {
            unsigned long long m[kTdWords];
#pragma unroll
            for (int k = 0; k < kTdWords; ++k) m[k] = cur_bits[min(w0 + k * wstride, st.words - 1)];
#pragma unroll
            for (int k = 0; k < kTdWords; ++k) asm volatile("" : "+v"(m[k]));
#pragma unroll
            for (int k = 0; k < kTdWords; ++k) {
                const int64_t w = w0 + k * wstride;
                if (w >= st.words || !((m[k] >> lane) & 1ull)) continue;
                const int32_t u = (int32_t)(w * kWave + lane);
                const int32_t beg = st.rowptr[u];
                int32_t end = st.rowptr[u + 1];
                if (end - beg > kBigDeg) {  // a hub: expanded by the whole grid in bfs_hubs_kernel
                    const unsigned long long slot = atomicAdd(&st.ctl->acc[L % 3].big, 1ull);
                    st.big[slot] = u;
                    end = beg;
                }
                for (int32_t j = beg; j < end; ++j) td_visit(st, true, st.col[j], lvl, next_bits, my_verts, my_edges);
            }
        }
    } else if (mode == XD_MODE_OBLIVIOUS || !heavy) {
        const int64_t bstride = (int64_t)gridDim.x * kWavesPerWg;
        for (int64_t blk = (int64_t)blockIdx.x * kWavesPerWg + wave; blk < nblocks; blk += 2 * bstride) {
            const bool hasb = blk + bstride < nblocks;
            bu_blocks(st, (int32_t)(blk * kWave), (int32_t)((hasb ? blk + bstride : blk) * kWave), hasb, cur_bits,
                      next_bits, lvl, my_verts, my_edges);
        }
    } else {
        // The waves of a die walk that die's block list (aware) or the other die's (rotated),
        // so the neighbour lists are read from the near (far) die; each wave takes two
        // consecutive list entries and the die's waves interleave over the whole list, as the
        // oblivious walk interleaves over all blocks. (Giving each XCD of the die a contiguous
        // quarter instead, so that a vertex range's lines stay in one L2 from level to level,
        // measured slower: the heavy first bottom-up level took 33.6 against 31.3 us.)
        const int b = (int)blockIdx.x;
        const uint32_t die = wg_die(b, xh);
        const uint32_t want = (mode == XD_MODE_AWARE) ? die : (die ^ 1u);
        const int32_t *mine = blist + (int64_t)want * nblocks;
        const int64_t cnt = (int64_t)bcount[want];
        const int64_t rank = (int64_t)die_rank(b, xh);
        const int64_t wd = rank * kWavesPerWg + wave;  // wave of the die
        const int64_t xstride = 2 * (int64_t)(gridDim.x / 2) * kWavesPerWg;
        for (int64_t i = 2 * wd; i < cnt; i += xstride) {
            const bool hasb = i + 1 < cnt;
            bu_blocks(st, mine[i] * kWave, mine[hasb ? i + 1 : i] * kWave, hasb, cur_bits, next_bits, lvl, my_verts,
                      my_edges);
        }
    }
    block_sum2(my_verts, my_edges);
    add_totals(st, L, my_verts, my_edges);
}

// Grid-wide expansion of the hub vertices top-down level L deferred (its state S_{L-1} was
// published by level L's workgroup 0).
__global__ void __launch_bounds__(kBfsThreads) bfs_hubs_kernel(BfsState st, int L) {
    if (st.ctl->s[(L - 1) % 2].dir != kTopDown) return;
    const int64_t nbig = (int64_t)st.ctl->acc[L % 3].big;
    if (nbig == 0) return;
    const uint32_t lvl = (uint32_t)L;
    unsigned long long *next_bits = st.front[L % 3];
    unsigned long long my_verts = 0, my_edges = 0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    // every wave takes 64 consecutive list entries at a time (a wave-uniform loop: the runs
    // of td_visit_runs need whole waves)
    const int64_t first = (int64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~(kWave - 1));
    for (int64_t h = 0; h < nbig; ++h) {
        const int32_t u = st.big[h];
        const int32_t beg = st.rowptr[u], end = st.rowptr[u + 1];
        for (int64_t e0 = beg + first; e0 < end; e0 += stride) {
            const int64_t e = e0 + lane_id();
            const bool have = e < end;
            const int32_t v = st.col[have ? e : end - 1];
            td_visit_runs(st, have, v, lvl, next_bits, my_verts, my_edges);
        }
    }
    block_sum2(my_verts, my_edges);
    add_totals(st, L, my_verts, my_edges);
}

// Sorts the 64-vertex blocks by the I/O die that homes the start of their adjacency (the
// block's first vertex on): list[d * nblocks + i] is the i-th block of die d, in ascending
// block order. The assignment depends only on the graph and the page map, so it is built
// once per graph (one workgroup walks the blocks in order, 1024 at a time); the bottom-up
// steps of the home modes interleave the waves of a die over its list.
constexpr int kBlkThreads = 1024;
__global__ void __launch_bounds__(kBlkThreads)
bfs_blocks_kernel(const int32_t *__restrict__ rowptr, int64_t nblocks, uint64_t cbase, int64_t col_bytes,
                  HomeMap home, int32_t *__restrict__ list, unsigned long long *__restrict__ count) {
    __shared__ uint32_t wcnt[2][kBlkThreads / kWave];
    __shared__ uint32_t wbase[2][kBlkThreads / kWave];
    __shared__ unsigned long long base[2];
    const int tid = (int)threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    if (tid < 2) base[tid] = 0ull;
    __syncthreads();
    for (int64_t blk0 = 0; blk0 < nblocks; blk0 += kBlkThreads) {
        const int64_t blk = blk0 + tid;
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
            uint32_t tot = 0;
            for (int w = 0; w < kBlkThreads / kWave; ++w) {
                wbase[tid][w] = tot;
                tot += wcnt[tid][w];
            }
        }
        __syncthreads();
        if (d < 2) {
            const uint64_t m = d ? m1 : m0;
            list[(int64_t)d * nblocks + (int64_t)(base[d] + wbase[d][wave] + mask_rank(m))] = (int32_t)blk;
        }
        __syncthreads();
        if (tid < 2) base[tid] += wbase[tid][kBlkThreads / kWave - 1] + wcnt[tid][kBlkThreads / kWave - 1];
        __syncthreads();
    }
    if (tid < 2) count[tid] = base[tid];
}

__global__ void bfs_clear2_kernel(unsigned long long *p) {
    if (threadIdx.x < 2) p[threadIdx.x] = 0ull;
}

// Per-die block lists of a graph into `route` (header: the two counts).
static int build_route(const int32_t *rowptr, const int32_t *col, int32_t V, int64_t nnz, const uint8_t *home_attr,
                       void *route, hipStream_t s) {
    const int64_t nblocks = ((int64_t)V + 63) / 64;
    auto *bcount = static_cast<unsigned long long *>(route);
    auto *blist = reinterpret_cast<int32_t *>(static_cast<char *>(route) + kRouteHeader);
    launch("bfs_clear2_kernel", bfs_clear2_kernel, dim3(1), dim3(64), 0, s, bcount);
    if (nnz == 0) return launch_status("bfs_clear2_kernel");
    const HomeMap home{home_attr, reinterpret_cast<uint64_t>(col) / kHomePage, home_mask()};
    launch("bfs_blocks_kernel", bfs_blocks_kernel, dim3(1), dim3(kBlkThreads),
                       0, s, rowptr, nblocks, reinterpret_cast<uint64_t>(col), nnz * (int64_t)sizeof(int32_t), home, blist,
                       bcount);
    return launch_status("bfs_blocks_kernel");
}

}  // namespace xd

using namespace xd;

namespace {

// Host side of the per-batch control copy: a pinned copy of the control block (a copy into
// pageable memory is staged by the runtime and cost ~15 us a search) and an event to wait
// on. Entries are shared by all host threads through one process-wide pool: a call takes an
// entry of its device (or makes one) and gives it back when it returns, so the pool never
// holds more entries per device than calls have run at once on it.
struct CtlHost {
    int device = -1;
    BfsCtlBlock *pinned = nullptr;          // hipHostMalloc'd, or null when that failed
    std::unique_ptr<BfsCtlBlock> pageable;  // fallback copy target
    hipEvent_t done = nullptr;
    BfsCtlBlock &block() { return pinned ? *pinned : *pageable; }
};

std::mutex g_ctl_mu;
std::vector<CtlHost *> g_ctl_free;

CtlHost *ctl_take(int device) {
    {
        std::lock_guard<std::mutex> g(g_ctl_mu);
        for (size_t i = 0; i < g_ctl_free.size(); ++i)
            if (g_ctl_free[i]->device == device) {
                CtlHost *c = g_ctl_free[i];
                g_ctl_free.erase(g_ctl_free.begin() + (long)i);
                return c;
            }
    }
    CtlHost *c = new CtlHost;
    c->device = device;
    if (hipHostMalloc(reinterpret_cast<void **>(&c->pinned), sizeof(BfsCtlBlock), hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        c->pinned = nullptr;
        c->pageable.reset(new BfsCtlBlock);
    }
    return c;
}

void ctl_give(CtlHost *c) {
    std::lock_guard<std::mutex> g(g_ctl_mu);
    g_ctl_free.push_back(c);
}

struct CtlLease {
    CtlHost *c;
    explicit CtlLease(int device) : c(ctl_take(device)) {}
    ~CtlLease() { ctl_give(c); }
};

// Waits for `ev` (made with hipEventBlockingSync): polls for up to 200 us (a level batch
// usually lands within that, and a blocking wait woke the host later: R-MAT scale 22 ran at
// 466 instead of 477 GTEPS), then blocks in hipEventSynchronize so that a long batch does not
// hold a host core.
hipError_t wait_event(hipEvent_t ev) {
    const auto t0 = std::chrono::steady_clock::now();
    hipError_t q;
    while ((q = hipEventQuery(ev)) == hipErrorNotReady) {
        if (std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(200)) return hipEventSynchronize(ev);
    }
    return q;
}

}  // namespace

extern "C" {

size_t xd_bfs_workspace_size(int32_t num_vertices, int64_t nnz) {
    if (num_vertices <= 0 || nnz < 0) return 0;
    return bfs_layout(num_vertices, nnz).total;
}

size_t xd_bfs_route_bytes(int32_t num_vertices) { return num_vertices > 0 ? route_bytes(num_vertices) : 0; }

int xd_bfs_route(const int32_t *rowptr, const int32_t *col, int32_t V, int64_t nnz, const uint8_t *home_attr,
                 void *route, size_t route_bytes_avail, void *stream) {
    XD_REQUIRE(rowptr != nullptr && route != nullptr && (nnz == 0 || col != nullptr), "xd_bfs_route: NULL pointer");
    XD_REQUIRE(V > 0 && nnz >= 0 && nnz < (1ll << 31), "xd_bfs_route: need 0 < V and 0 <= nnz < 2^31");
    XD_REQUIRE(route_bytes_avail >= route_bytes(V) && aligned16(route), "xd_bfs_route: route buffer too small");
    return build_route(rowptr, col, V, nnz, home_attr, route, (hipStream_t)stream);
}

int xd_bfs_csr(const int32_t *rowptr, const int32_t *col, int32_t V, int64_t nnz, int32_t src, uint32_t *level,
               int mode, const void *route, void *workspace, size_t workspace_bytes, void *stream,
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
    BfsState st{};
    st.rowptr = rowptr;
    st.col = col;
    st.V = V;
    st.words = L.words;
    st.level = level;
    st.visited = reinterpret_cast<unsigned long long *>(ws + L.visited);
    for (int i = 0; i < 3; ++i) st.front[i] = reinterpret_cast<unsigned long long *>(ws + L.front[i]);
    st.big = reinterpret_cast<int32_t *>(ws + L.big);
    st.ctl = reinterpret_cast<BfsCtlBlock *>(ws + L.ctl);
    const int bmode = nnz > 0 ? mode : XD_MODE_OBLIVIOUS;  // no adjacency to route by
    const unsigned g256 = (unsigned)std::min<int64_t>(8192, ((int64_t)V + 255) / 256 + 1);
    const void *rt = route;
    {
        launch("bfs_init_kernel", bfs_init_kernel, dim3(g256), dim3(256), 0, s, st, src, nnz);
        if (int rc = launch_status("bfs_init_kernel")) return rc;
        if (bmode != XD_MODE_OBLIVIOUS && rt == nullptr) {  // no prepared route: build one here
            if (int rc = build_route(rowptr, col, V, nnz, nullptr, ws + L.route, s)) return rc;
            rt = ws + L.route;
        }
    }
    const auto *bcount = static_cast<const unsigned long long *>(rt);
    const auto *blist =
        rt ? reinterpret_cast<const int32_t *>(static_cast<const char *>(rt) + kRouteHeader) : nullptr;
    BfsCtl h{};
    int device = 0;
    XD_HIP(hipGetDevice(&device));
    CtlLease lease(device);
    if (lease.c->done == nullptr)  // (blocking sync: the wait past its polling window sleeps)
        XD_HIP(hipEventCreateWithFlags(&lease.c->done, hipEventDisableTiming | hipEventBlockingSync));
    BfsCtlBlock &hb = lease.c->block();
    for (int64_t enq = 0;;) {
        const int batch = enq == 0 ? kFirstBatch : kLevelBatch;
        const XcdHint xh = xcd_hint(s);
        for (int k = 0; k < batch; ++k, ++enq) {
            const int lv = (int)(enq + 1);
            launch("bfs_level_kernel", bfs_level_kernel, dim3(kBfsGrid), dim3(kBfsThreads), 0, s, st, lv, bmode, blist,
                   bcount, L.nblocks, xh);
            launch("bfs_hubs_kernel", bfs_hubs_kernel, dim3(kBigGrid), dim3(kBfsThreads), 0, s, st, lv);
            if (int rc = launch_status("bfs level kernels")) return rc;
        }
        XD_HIP(hipMemcpyAsync(&hb, st.ctl, sizeof(hb), hipMemcpyDeviceToHost, s));
        XD_HIP(hipEventRecord(lease.c->done, s));
        const hipError_t q = wait_event(lease.c->done);
        if (q != hipSuccess) return hip_fail(q, "xd_bfs_csr: waiting for the control copy");
        // S_{lv-1} was published by the last level kernel; the step adds that level's totals
        const int lv = (int)enq;
        unsigned long long tv = 0, te = 0;
        for (int i = 0; i < kAccSlots; ++i) {
            tv += hb.acc[lv % 3].slot[i].verts;
            te += hb.acc[lv % 3].slot[i].edges;
        }
        h = ctl_step(hb.s[(lv - 1) % 2], tv, te, V);
        if (h.dir == kDone) break;
        if (enq > (int64_t)V + 1) return fail(XD_ERR_INCOMPLETE, "xd_bfs_csr: search did not finish");
    }
    if (stats) {
        stats->levels = h.depth;
        stats->topdown_steps = h.td_steps;
        stats->bottomup_steps = h.bu_steps;
        stats->reached_vertices = h.reached_v;
        stats->reached_edges = h.reached_e;
    }
    return XD_OK;
}

}  // extern "C"
