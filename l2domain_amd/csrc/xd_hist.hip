// Large-bin histogram: counts[k] = #{i : keys[i] == k} for k < num_bins (<= 2^24).
//
// Reference: applications/histogram/src/histogram256_sideaware.cu
//   add_word (20-25) / histogram256_chunked_kernel (51-85): per-warp LDS sub-histograms of
//     256 byte-bins over 4 KiB chunks, then per-block partials;
//   histogram256_persistent_kernel (87-134): chunks routed to the SM's L2 side;
//   merge_histogram256_kernel (136-157): sum of the per-block partials.
//
// MI355X design. 2^20 u32 counters (4 MiB) do not fit the 160 KB LDS of a CU, and global
// atomics on gfx950 run at a fixed ~27 Gatom/s chip-wide (~88 M/s on one hot address)
// wherever the line lives, so every key must be counted in LDS:
//   1. partition: each workgroup multi-splits a tile of 16384 keys into 32768-bin buckets
//      (bucket = key >> 15) and writes the 15-bit in-bucket offsets, grouped by bucket,
//      as u16 (tile-major), plus the tile's bucket offsets and bucket totals;
//   2. plan: apportions counting work items (bucket, tile range) in proportion to the
//      bucket totals; XCD-aware mode gives every XCD a contiguous range of buckets (bins
//      range-partitioned per XCD) and only that XCD's workgroups count them;
//   3. count: one workgroup per item keeps a 128 KB LDS histogram of its bucket, adds each
//      key with a ds_add (the wave's most common key is peeled into one add), and writes
//      the LDS histogram to its partial slot;
//   4. merge: counts = sum of the bucket's partial slots. XCD-aware mode fuses the merge
//      into the count pass: the last count workgroup of a bucket to finish (a ticket per
//      bucket) sums the bucket's slots, which its own XCD wrote and still holds in L2; the
//      merge kernel then only writes the empty buckets. Oblivious and rotated run the merge
//      kernel over every bucket.
#include <hip/hip_runtime.h>

#include "xd_common.hpp"

namespace xd {

constexpr int kHB = 15;
constexpr uint32_t kBucketBins = 1u << kHB;  // 32768 counters = 128 KB of LDS
constexpr int kTileKeys = 16384;
constexpr int kP1Threads = 1024;
constexpr int kP1Vec = kTileKeys / 4 / kP1Threads;  // uint4 loads per thread (4)
constexpr int kMaxBuckets = 512;                    // num_bins <= 2^24
constexpr int kP2Threads = 1024;
constexpr int kP2Waves = kP2Threads / kWave;
constexpr int kMergeThreads = 256;
constexpr int kMergeBins = 4096;  // bins per merge unit (16 per thread)
constexpr int kMergeUnitsPerBucket = kBucketBins / kMergeBins;
constexpr int kPlanThreads = kMaxBuckets;

struct HistItem {
    int bucket;  // -1: idle slot
    int t0, t1;  // tile range
    int pad;
};

struct HistBucket {
    int first;  // first item (= partial slot) of this bucket
    int count;  // items of this bucket (0: the bucket is empty)
    int xcd;
    int pad;
};

struct HistLayout {
    int nb, ntiles, per_xcd, nitems;
    size_t part, offs, tot, items, buckets, xcdr, bsync, partials, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static HistLayout hist_layout(size_t n, uint32_t num_bins) {
    HistLayout L{};
    L.nb = (int)((num_bins + kBucketBins - 1) / kBucketBins);
    if (L.nb < 1) L.nb = 1;
    L.ntiles = (int)((n + kTileKeys - 1) / kTileKeys);
    L.per_xcd = (L.nb + kNumXcd - 1) / kNumXcd + 8;
    if (L.per_xcd < 32) L.per_xcd = 32;
    L.nitems = L.per_xcd * kNumXcd;
    // Regions whose offsets depend only on num_bins come first, so a workspace sized for
    // more keys keeps its zeroed counters at the same place for every n.
    size_t o = 0;
    L.tot = o;
    o = align256(o + (size_t)kNumXcd * L.nb * sizeof(uint32_t));
    L.items = o;
    o = align256(o + (size_t)L.nitems * sizeof(HistItem));
    L.buckets = o;
    o = align256(o + (size_t)L.nb * sizeof(HistBucket));
    L.xcdr = o;
    o = align256(o + (size_t)kNumXcd * 2 * sizeof(int));
    L.bsync = o;  // per bucket: arrival counter and "written off its XCD" flag (zero between calls)
    o = align256(o + (size_t)2 * L.nb * sizeof(uint32_t));
    L.partials = o;
    o = align256(o + (size_t)L.nitems * kBucketBins * sizeof(uint32_t));
    L.offs = o;
    o = align256(o + (size_t)L.ntiles * (L.nb + 1) * sizeof(uint32_t));
    L.part = o;
    o = align256(o + (size_t)L.ntiles * kTileKeys * sizeof(uint16_t));
    L.total = o;
    return L;
}

__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        uint32_t t = __shfl_up(v, d, kWave);
        if (lane >= d) v += t;
    }
    return v;
}

// ---------------------------------------------------------------------------------------
// 1. partition
// ---------------------------------------------------------------------------------------
template <bool VEC>
__global__ void __launch_bounds__(kP1Threads)
hist_partition_kernel(const uint32_t *__restrict__ keys, size_t n, uint32_t num_bins, int nb,
                      uint16_t *__restrict__ part, uint32_t *__restrict__ offs, uint32_t *__restrict__ tot) {
    __shared__ uint32_t cnt[kMaxBuckets];
    __shared__ uint32_t base[kMaxBuckets + 1];
    __shared__ __attribute__((aligned(16))) uint16_t stage[kTileKeys];
    const int t = (int)blockIdx.x;
    const size_t k0 = (size_t)t * kTileKeys;
    const int tid = (int)threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    for (int i = tid; i < nb; i += kP1Threads) cnt[i] = 0;

    uint32_t kk[4 * kP1Vec];
    if (VEC && k0 + kTileKeys <= n) {
        const uint4 *kv = reinterpret_cast<const uint4 *>(keys + k0);
#pragma unroll
        for (int j = 0; j < kP1Vec; ++j) {
            uint4 v = kv[tid + j * kP1Threads];
            kk[4 * j] = v.x;
            kk[4 * j + 1] = v.y;
            kk[4 * j + 2] = v.z;
            kk[4 * j + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < kP1Vec; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                size_t idx = k0 + 4 * (size_t)(tid + j * kP1Threads) + c;
                kk[4 * j + c] = idx < n ? keys[idx] : 0xffffffffu;
            }
    }
    __syncthreads();

    // Slot of every key inside its bucket: a returning LDS add per key. (Same-bucket lanes
    // of a wave serialise in the LDS, which costs less than aggregating them in registers.)
    uint32_t pos[4 * kP1Vec];
#pragma unroll
    for (int j = 0; j < 4 * kP1Vec; ++j) {
        const uint32_t key = kk[j];
        pos[j] = key < num_bins ? atomicAdd(&cnt[key >> kHB], 1u) : 0u;
    }
    __syncthreads();

    if (wave == 0) {
        uint32_t carry = 0;
        for (int c0 = 0; c0 < nb; c0 += kWave) {
            const int i = c0 + lane;
            const uint32_t v = i < nb ? cnt[i] : 0u;
            const uint32_t incl = wave_incl_scan_u32(v);
            if (i < nb) base[i] = carry + incl - v;
            carry += (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
        }
        if (lane == 0) base[nb] = carry;
    }
    __syncthreads();

    uint32_t *my_offs = offs + (size_t)t * (nb + 1);
    for (int i = tid; i <= nb; i += kP1Threads) my_offs[i] = base[i];
    uint32_t *my_tot = tot + (size_t)(t % kNumXcd) * nb;
    for (int i = tid; i < nb; i += kP1Threads) {
        const uint32_t c = cnt[i];
        if (c) atomicAdd(&my_tot[i], c);
    }
#pragma unroll
    for (int j = 0; j < 4 * kP1Vec; ++j) {
        const uint32_t key = kk[j];
        if (key < num_bins) stage[base[key >> kHB] + pos[j]] = (uint16_t)(key & (kBucketBins - 1));
    }
    __syncthreads();

    const uint32_t total = base[nb];
    const uint32_t nvec = (total + 7) / 8;  // 8 u16 per 16-byte store
    const uint4 *src = reinterpret_cast<const uint4 *>(stage);
    uint4 *dst = reinterpret_cast<uint4 *>(part + k0);
    for (uint32_t i = (uint32_t)tid; i < nvec; i += kP1Threads) dst[i] = src[i];
}

// ---------------------------------------------------------------------------------------
// 2. plan (one workgroup; one thread per bucket)
// ---------------------------------------------------------------------------------------
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t *wsum, uint32_t *total) {
    const int tid = (int)threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const uint32_t incl = wave_incl_scan_u32(v);
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    if (tid == 0) {
        uint32_t c = 0;
        for (int w = 0; w < kPlanThreads / kWave; ++w) {
            uint32_t s = wsum[w];
            wsum[w] = c;
            c += s;
        }
        *total = c;
    }
    __syncthreads();
    const uint32_t r = wsum[wave] + incl - v;
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(kPlanThreads)
hist_plan_kernel(const uint32_t *__restrict__ tot, int nb, int ntiles, int per_xcd, int mode, HistItem *items,
                 HistBucket *buckets, int *xcd_range) {
    __shared__ uint32_t wsum[kPlanThreads / kWave];
    __shared__ uint32_t s_total, s_nnz_total;
    __shared__ uint32_t xnnz[kNumXcd];
    __shared__ uint32_t xload[kNumXcd];
    __shared__ uint32_t xfirst[kNumXcd];
    __shared__ int s_fallback;
    const int b = (int)threadIdx.x;
    const int nitems = per_xcd * kNumXcd;
    for (int i = b; i < nitems; i += kPlanThreads) items[i] = HistItem{-1, 0, 0, 0};
    if (b < kNumXcd) {
        xnnz[b] = 0;
        xload[b] = 0;
        xfirst[b] = 0xffffffffu;
    }
    if (b == 0) s_fallback = 0;

    uint32_t T = 0;
    if (b < nb)
        for (int x = 0; x < kNumXcd; ++x) T += tot[(size_t)x * nb + b];
    const uint32_t nz = (b < nb && T > 0) ? 1u : 0u;
    const uint32_t pre = block_excl_scan(T, wsum, &s_total);
    const uint32_t N = s_total;
    (void)block_excl_scan(nz, wsum, &s_nnz_total);
    const uint32_t nnz = s_nnz_total;

    if (mode == XD_MODE_OBLIVIOUS) {
        // One flat list: item g runs on workgroup g.
        uint32_t J = 0;
        if (nz) J = 1u + (uint32_t)(((unsigned long long)((uint32_t)nitems - min(nnz, (uint32_t)nitems)) * T) / (N ? N : 1u));
        uint32_t first = block_excl_scan(J, wsum, &s_total);
        // Totals always give sum(J) <= nitems; the clamp keeps every write inside the table.
        if (first > (uint32_t)nitems) first = (uint32_t)nitems;
        if (J > (uint32_t)nitems - first) J = (uint32_t)nitems - first;
        if (b < nb) {
            buckets[b] = HistBucket{(int)first, (int)J, -1, 0};
            for (uint32_t j = 0; j < J; ++j)
                items[first + j] = HistItem{b, (int)((unsigned long long)j * ntiles / J),
                                            (int)((unsigned long long)(j + 1) * ntiles / J), 0};
        }
        if (b < kNumXcd) {  // merge ranges: equal bucket counts
            xcd_range[2 * b] = (int)((long long)b * nb / kNumXcd);
            xcd_range[2 * b + 1] = (int)((long long)(b + 1) * nb / kNumXcd);
        }
        return;
    }

    // XCD-aware: contiguous bucket ranges, split where the load prefix crosses x * N / 8.
    int x = 0;
    if (b < nb) {
        x = N ? (int)(((unsigned long long)pre * kNumXcd) / N) : (int)((long long)b * kNumXcd / nb);
        if (x > kNumXcd - 1) x = kNumXcd - 1;
        if (nz) atomicAdd(&xnnz[x], 1u);
    }
    __syncthreads();
    if (b < kNumXcd && xnnz[b] > (uint32_t)per_xcd) s_fallback = 1;
    __syncthreads();
    if (s_fallback && b < nb) x = (int)((long long)b * kNumXcd / nb);
    if (b < nb) {
        atomicMin(&xfirst[x], (uint32_t)b);
        if (nz) atomicAdd(&xload[x], T);
    }
    __syncthreads();
    if (b < kNumXcd) xnnz[b] = 0;
    __syncthreads();
    if (b < nb && nz) atomicAdd(&xnnz[x], 1u);
    __syncthreads();
    uint32_t J = 0;
    if (nz) {
        const uint32_t L = xload[x];
        J = 1u + (uint32_t)(((unsigned long long)((uint32_t)per_xcd - min(xnnz[x], (uint32_t)per_xcd)) * T) / (L ? L : 1u));
    }
    // Buckets of one XCD are contiguous, so a global scan minus the scan value at the
    // XCD's first bucket gives the position inside that XCD's item list.
    const uint32_t gpre = block_excl_scan(J, wsum, &s_total);
    __shared__ uint32_t xbase[kNumXcd];
    if (b < nb && (uint32_t)b == xfirst[x]) xbase[x] = gpre;
    __syncthreads();
    if (b < nb) {
        uint32_t within = gpre - xbase[x];
        if (within > (uint32_t)per_xcd) within = (uint32_t)per_xcd;
        if (J > (uint32_t)per_xcd - within) J = (uint32_t)per_xcd - within;
        const uint32_t first = (uint32_t)(x * per_xcd) + within;
        buckets[b] = HistBucket{(int)first, (int)J, x, 0};
        for (uint32_t j = 0; j < J; ++j)
            items[first + j] = HistItem{b, (int)((unsigned long long)j * ntiles / J),
                                        (int)((unsigned long long)(j + 1) * ntiles / J), 0};
    }
    if (b < kNumXcd) {
        // Ranges: [first bucket of XCD b, first bucket of the next non-empty XCD).
        int b0 = (xfirst[b] == 0xffffffffu) ? nb : (int)xfirst[b];
        int b1 = nb;
        for (int y = b + 1; y < kNumXcd; ++y)
            if (xfirst[y] != 0xffffffffu) {
                b1 = (int)xfirst[y];
                break;
            }
        if (b0 > b1) b0 = b1;
        xcd_range[2 * b] = b0;
        xcd_range[2 * b + 1] = b1;
    }
}

// ---------------------------------------------------------------------------------------
// 3. count
// ---------------------------------------------------------------------------------------
constexpr uint32_t kTrash = kBucketBins;  // LDS slot that absorbs elements outside a run
#ifndef XD_HIST_RUNS_AHEAD
#define XD_HIST_RUNS_AHEAD 2
#endif
constexpr int kRunsAhead = XD_HIST_RUNS_AHEAD;  // runs loaded ahead of the one being counted

// Counts the 8 u16 keys of one 16-byte vector whose first element has index `e`, for the
// run [s0, e0). Keys equal to the wave's current hot key go to the per-lane register
// counter `hc` (the hot key of a Zipf bucket would otherwise make most lanes of a wave
// hit one LDS address); all others take one ds_add each.
__device__ __forceinline__ void count_vec(uint32_t *h, const uint4 &q, uint32_t e, uint32_t s0, uint32_t e0,
                                          uint32_t hot, uint32_t &hc) {
    if (e >= e0 || e + 8 <= s0) return;  // vector outside the run (most lanes' 2nd vector)
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const uint32_t len = e0 - s0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t key = (k & 1) ? (w[k >> 1] >> 16) : (w[k >> 1] & 0xffffu);
        key = (e + (uint32_t)k - s0 < len) ? key : kTrash;
        if (key == hot) ++hc;
        else atomicAdd(&h[key], 1u);
    }
}

__global__ void __launch_bounds__(kP2Threads)
hist_count_kernel(const uint16_t *__restrict__ part, const uint32_t *__restrict__ offs, int nb,
                  const HistItem *__restrict__ items, int per_xcd, uint32_t *__restrict__ partials, int mode,
                  unsigned rot, int fused, const HistBucket *__restrict__ buckets, uint32_t *__restrict__ bsync,
                  uint32_t num_bins, uint32_t *__restrict__ counts, bool counts16) {
    __shared__ __attribute__((aligned(16))) uint32_t h[kBucketBins + 4];
    const int g = (int)blockIdx.x;
    int item;
    if (mode == XD_MODE_OBLIVIOUS) {
        item = g;
    } else {
        XcdSlot s = xcd_slot(g, (int)gridDim.x, mode, rot);
        item = s.slice * per_xcd + s.rank;
    }
    const HistItem it = items[item];
    if (it.bucket < 0) return;
    const int tid = (int)threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    uint4 *h4 = reinterpret_cast<uint4 *>(h);
    for (int i = tid; i < (int)(kBucketBins / 4) + 1; i += kP2Threads) h4[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();

    const int b = it.bucket;
    uint32_t hot = kTrash + 1;  // no hot key yet
    uint32_t hc = 0;
    auto flush_hot = [&]() {
        const uint32_t tot_hot = wave_sum_u32(hc);
        if (lane == 0 && tot_hot) atomicAdd(&h[hot], tot_hot);
        hc = 0;
    };
    // Each wave walks the tiles t0 + wave, t0 + wave + 16, ...: lane i first fetches the run
    // bounds of 64 of them, then the wave counts run after run. A run is read as 16-byte
    // vectors (8 keys); the first two vectors per lane of the next kRunsAhead runs are in
    // flight while the current run is counted. Every load is issued unconditionally, with its
    // index clamped into the run (a run never leaves its tile) and the elements outside the
    // run discarded by count_vec: a load under a branch makes the compiler wait for every
    // load in flight where the branches join, which would empty the pipeline.
    for (int tb = it.t0 + wave; tb < it.t1; tb += kP2Waves * kWave) {
        const int tl = tb + lane * kP2Waves;
        const bool tok = tl < it.t1;
        const uint32_t *o = offs + (size_t)(tok ? tl : it.t1 - 1) * (nb + 1) + b;
        const uint32_t rs0 = o[0], re0 = o[1];
        const uint32_t rs = tok ? rs0 : 0u, re = tok ? re0 : 0u;
        const int ntl = min(kWave, (it.t1 - tb + kP2Waves - 1) / kP2Waves);
        // lanes past the end of a run re-read the run's last vector, a line already fetched
        auto load2 = [&](int i, uint4 &v0, uint4 &v1) {
            const uint32_t s0 = (uint32_t)__builtin_amdgcn_readlane((int)rs, i);
            const uint32_t e0 = (uint32_t)__builtin_amdgcn_readlane((int)re, i);
            const uint4 *run = reinterpret_cast<const uint4 *>(part + (size_t)(tb + i * kP2Waves) * kTileKeys);
            const uint32_t v = (s0 >> 3) + (uint32_t)lane;
            const uint32_t last = max((e0 + 7) >> 3, (s0 >> 3) + 1) - 1;  // < kTileVecs
            v0 = run[min(v, last)];
            v1 = run[min(v + (uint32_t)kWave, last)];
        };
        auto count_run = [&](int i, const uint4 &c0, const uint4 &c1) {
            const uint32_t s0 = (uint32_t)__builtin_amdgcn_readlane((int)rs, i);
            const uint32_t e0 = (uint32_t)__builtin_amdgcn_readlane((int)re, i);
            const uint32_t v = (s0 >> 3) + (uint32_t)lane;
            // Hot-key vote on the first key of every lane's first vector: keep the current
            // hot key while a quarter of the samples match it, else adopt the first sample if
            // a quarter of the samples match that one.
            const uint32_t e8 = 8 * v;
            const bool sv = e8 - s0 < e0 - s0;
            const uint32_t sk = c0.x & 0xffffu;
            if (__builtin_popcountll(__ballot(sv && sk == hot)) < kWave / 4) {
                const uint64_t svm = __ballot(sv);
                if (svm) {
                    const uint32_t cand = (uint32_t)__builtin_amdgcn_readlane((int)sk, __builtin_ctzll(svm));
                    if (__builtin_popcountll(__ballot(sv && sk == cand)) >= kWave / 4) {
                        flush_hot();
                        hot = cand;
                    }
                }
            }
            count_vec(h, c0, e8, s0, e0, hot, hc);
            count_vec(h, c1, 8 * (v + kWave), s0, e0, hot, hc);
            // long runs (the hot bucket): the remaining vectors, two per lane per trip, in a
            // loop whose trip count is the same for every lane
            const uint4 *run = reinterpret_cast<const uint4 *>(part + (size_t)(tb + i * kP2Waves) * kTileKeys);
            const uint32_t vend = (e0 + 7) >> 3;
            for (uint32_t u0 = (s0 >> 3) + 2 * kWave; u0 < vend; u0 += 2 * kWave) {
                const uint32_t u = u0 + (uint32_t)lane;
                const uint4 a0 = run[min(u, vend - 1)];
                const uint4 a1 = run[min(u + (uint32_t)kWave, vend - 1)];
                count_vec(h, a0, 8 * u, s0, e0, hot, hc);
                count_vec(h, a1, 8 * (u + kWave), s0, e0, hot, hc);
            }
        };
        // software pipeline over a ring of register buffers, statically indexed
        uint4 r0[kRunsAhead], r1[kRunsAhead];
#pragma unroll
        for (int j = 0; j < kRunsAhead; ++j) load2(min(j, ntl - 1), r0[j], r1[j]);
        int i0 = 0;
        for (; i0 + kRunsAhead <= ntl; i0 += kRunsAhead) {
#pragma unroll
            for (int j = 0; j < kRunsAhead; ++j) {
                const uint4 c0 = r0[j], c1 = r1[j];
                load2(min(i0 + j + kRunsAhead, ntl - 1), r0[j], r1[j]);
                count_run(i0 + j, c0, c1);
            }
        }
#pragma unroll
        for (int j = 0; j < kRunsAhead; ++j)
            if (i0 + j < ntl) count_run(i0 + j, r0[j], r1[j]);
    }
    if (hot < kTrash) flush_hot();
    __syncthreads();
    uint4 *dst = reinterpret_cast<uint4 *>(partials + (size_t)item * kBucketBins);
    for (int i = tid; i < (int)(kBucketBins / 4); i += kP2Threads) dst[i] = h4[i];
    if (!fused) return;

    // Fused merge (XCD-aware plans): every item of bucket b was planned on XCD item / per_xcd,
    // so the last of them to finish sums the bucket's partials out of that XCD's L2. A
    // workgroup that finds itself on another XCD (dispatch not round-robin) publishes its
    // partial with a device-scope release and marks the bucket, and the merger then
    // acquires before reading.
    __shared__ uint32_t s_last, s_foreign;
    const bool foreign = (int)hw_xcc_id() != item / per_xcd;
    if (foreign) __threadfence();
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have reached the L2
    __syncthreads();
    if (tid == 0) {
        uint32_t *cnt = bsync + 2 * b, *flag = cnt + 1;
        uint32_t f = 0;
        if (foreign) f = atomicOr(flag, 1u);
        asm volatile("" ::"v"(f));  // the flag is set before the ticket is taken
        const uint32_t t = atomicAdd(cnt, 1u);
        const HistBucket bk = buckets[b];
        s_last = t == (uint32_t)(bk.count - 1);
        s_foreign = 0;
        if (s_last) {
            atomicExch(cnt, 0u);
            s_foreign = atomicExch(flag, 0u);
        }
    }
    __syncthreads();
    if (!s_last) return;
    if (s_foreign || foreign) __threadfence();
    const HistBucket bk = buckets[b];
    const uint32_t bin0 = (uint32_t)b * kBucketBins;
    for (int v = tid; v < (int)(kBucketBins / 4); v += kP2Threads) {
        uint4 acc = h4[v];  // this workgroup's own partial, still in LDS
        for (int i = 0; i < bk.count; ++i) {
            const int slot = bk.first + i;
            if (slot == item) continue;
            const uint4 p = reinterpret_cast<const uint4 *>(partials + (size_t)slot * kBucketBins)[v];
            acc.x += p.x;
            acc.y += p.y;
            acc.z += p.z;
            acc.w += p.w;
        }
        const uint32_t k = bin0 + 4u * (uint32_t)v;
        if (counts16 && k + 3 < num_bins) {
            reinterpret_cast<uint4 *>(counts + k)[0] = acc;
        } else {
            if (k < num_bins) counts[k] = acc.x;
            if (k + 1 < num_bins) counts[k + 1] = acc.y;
            if (k + 2 < num_bins) counts[k + 2] = acc.z;
            if (k + 3 < num_bins) counts[k + 3] = acc.w;
        }
    }
}

// ---------------------------------------------------------------------------------------
// 4. merge
// ---------------------------------------------------------------------------------------
__device__ void merge_unit(int u, const uint32_t *__restrict__ partials, const HistBucket *__restrict__ buckets,
                           uint32_t num_bins, uint32_t *__restrict__ counts, bool counts16) {
    const int b = u / kMergeUnitsPerBucket;
    const int blk = u % kMergeUnitsPerBucket;
    const HistBucket bk = buckets[b];
    const uint32_t bin0 = (uint32_t)b * kBucketBins + (uint32_t)blk * kMergeBins;
    for (int v = (int)threadIdx.x; v < kMergeBins / 4; v += kMergeThreads) {
        uint4 acc = make_uint4(0, 0, 0, 0);
        for (int i = 0; i < bk.count; ++i) {
            const uint4 p = reinterpret_cast<const uint4 *>(partials + (size_t)(bk.first + i) * kBucketBins +
                                                             (size_t)blk * kMergeBins)[v];
            acc.x += p.x;
            acc.y += p.y;
            acc.z += p.z;
            acc.w += p.w;
        }
        const uint32_t k = bin0 + 4u * (uint32_t)v;
        if (counts16 && k + 3 < num_bins) {
            reinterpret_cast<uint4 *>(counts + k)[0] = acc;
        } else {
            if (k < num_bins) counts[k] = acc.x;
            if (k + 1 < num_bins) counts[k + 1] = acc.y;
            if (k + 2 < num_bins) counts[k + 2] = acc.z;
            if (k + 3 < num_bins) counts[k + 3] = acc.w;
        }
    }
}

__global__ void __launch_bounds__(kMergeThreads)
hist_merge_kernel(const uint32_t *__restrict__ partials, const HistBucket *__restrict__ buckets,
                  const int *__restrict__ xcd_range, int nb, uint32_t num_bins, uint32_t *__restrict__ counts,
                  bool counts16, uint32_t *__restrict__ tot, int mode, int only_empty) {
    const int g = (int)blockIdx.x;
    if (g == 0)
        for (int i = (int)threadIdx.x; i < kNumXcd * nb; i += kMergeThreads) tot[i] = 0;
    if (only_empty) {
        // fused plans merged every counted bucket in the count pass; write the empty ones
        for (int u = g; u < nb * kMergeUnitsPerBucket; u += (int)gridDim.x)
            if (buckets[u / kMergeUnitsPerBucket].count == 0)
                merge_unit(u, partials, buckets, num_bins, counts, counts16);
        return;
    }
    if (mode == XD_MODE_OBLIVIOUS) {
        for (int u = g; u < nb * kMergeUnitsPerBucket; u += (int)gridDim.x)
            merge_unit(u, partials, buckets, num_bins, counts, counts16);
    } else {
        // Buckets are merged on the XCD that counted them (aware), or on the XCD next to the
        // one that counted them (rotated: the count pass ran rotated by one).
        const XcdSlot s = xcd_slot(g, (int)gridDim.x, XD_MODE_AWARE, 0);
        const int x = s.slice;
        const int u0 = xcd_range[2 * x] * kMergeUnitsPerBucket;
        const int u1 = xcd_range[2 * x + 1] * kMergeUnitsPerBucket;
        for (int u = u0 + s.rank; u < u1; u += s.per_xcd) merge_unit(u, partials, buckets, num_bins, counts, counts16);
    }
}

}  // namespace xd

using namespace xd;

extern "C" {

size_t xd_hist_workspace_size(size_t n, uint32_t num_bins) {
    if (num_bins == 0 || num_bins > (1u << 24)) return 0;
    return hist_layout(n, num_bins).total;
}

int xd_hist_u32(const uint32_t *keys, size_t n, uint32_t *counts, uint32_t num_bins, int mode, void *workspace,
                size_t workspace_bytes, void *stream) {
    XD_REQUIRE(counts != nullptr, "xd_hist_u32: counts is NULL");
    XD_REQUIRE(n == 0 || keys != nullptr, "xd_hist_u32: keys is NULL");
    XD_REQUIRE(num_bins >= 1 && num_bins <= (1u << 24), "xd_hist_u32: num_bins must be in [1, 2^24]");
    XD_REQUIRE(n <= 0xffffffffull, "xd_hist_u32: n must be < 2^32 (u32 counters)");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "xd_hist_u32: bad mode");
    XD_REQUIRE((reinterpret_cast<uintptr_t>(keys) & 3u) == 0 && (reinterpret_cast<uintptr_t>(counts) & 3u) == 0,
               "xd_hist_u32: keys and counts must be 4-byte aligned");
    const HistLayout L = hist_layout(n, num_bins);
    if (workspace == nullptr || workspace_bytes < L.total || !aligned16(workspace))
        return fail(XD_ERR_WORKSPACE, "xd_hist_u32: workspace missing, misaligned or smaller than xd_hist_workspace_size()");
    hipStream_t s = (hipStream_t)stream;
    char *ws = static_cast<char *>(workspace);
    uint16_t *part = reinterpret_cast<uint16_t *>(ws + L.part);
    uint32_t *offs = reinterpret_cast<uint32_t *>(ws + L.offs);
    uint32_t *tot = reinterpret_cast<uint32_t *>(ws + L.tot);
    HistItem *items = reinterpret_cast<HistItem *>(ws + L.items);
    HistBucket *buckets = reinterpret_cast<HistBucket *>(ws + L.buckets);
    int *xcdr = reinterpret_cast<int *>(ws + L.xcdr);
    uint32_t *bsync = reinterpret_cast<uint32_t *>(ws + L.bsync);
    const int fused = mode == XD_MODE_AWARE ? 1 : 0;
    uint32_t *partials = reinterpret_cast<uint32_t *>(ws + L.partials);
    const unsigned rot = mode == XD_MODE_ROTATED ? next_rotation(1) % kNumXcd : 0u;
    const unsigned rot_eff = (mode == XD_MODE_ROTATED && rot == 0) ? 1u : rot;  // never the identity

    if (L.ntiles > 0) {
        KernelTimer kt("hist_partition", s);
        if (aligned16(keys))
            hipLaunchKernelGGL(hist_partition_kernel<true>, dim3(L.ntiles), dim3(kP1Threads), 0, s, keys, n, num_bins,
                               L.nb, part, offs, tot);
        else
            hipLaunchKernelGGL(hist_partition_kernel<false>, dim3(L.ntiles), dim3(kP1Threads), 0, s, keys, n,
                               num_bins, L.nb, part, offs, tot);
        if (int rc = launch_status("hist_partition_kernel")) return rc;
    }
    {
    KernelTimer kt("hist_plan", s);
    hipLaunchKernelGGL(hist_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, tot, L.nb, L.ntiles, L.per_xcd, mode, items,
                       buckets, xcdr);
    if (int rc = launch_status("hist_plan_kernel")) return rc;
    }
    {
    KernelTimer kt("hist_count", s);
    hipLaunchKernelGGL(hist_count_kernel, dim3(L.nitems), dim3(kP2Threads), 0, s, part, offs, L.nb, items, L.per_xcd,
                       partials, mode, rot_eff, fused, buckets, bsync, num_bins, counts, aligned16(counts));
    if (int rc = launch_status("hist_count_kernel")) return rc;
    }
    KernelTimer kt("hist_merge", s);
    const int merge_grid = kNumXcd * 64;
    hipLaunchKernelGGL(hist_merge_kernel, dim3(merge_grid), dim3(kMergeThreads), 0, s, partials, buckets, xcdr, L.nb,
                       num_bins, counts, aligned16(counts), tot, mode, fused);
    return launch_status("hist_merge_kernel");
}

}  // extern "C"
