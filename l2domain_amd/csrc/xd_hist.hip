// Large-bin histogram: counts[k] = #{i : keys[i] == k} for k < num_bins (<= 2^24).
//
// Reference: applications/histogram/src/histogram256_sideaware.cu
//   add_word (20-25) / histogram256_chunked_kernel (51-85): per-warp LDS sub-histograms of
//     256 byte-bins over 4 KiB chunks, then per-block partials;
//   histogram256_persistent_kernel (87-134): chunks routed to the SM's L2 side;
//   merge_histogram256_kernel (136-157): sum of the per-block partials.
//
// MI355X design. 2^20 u32 counters (4 MiB) do not fit the 160 KB LDS of a CU, and global
// atomics on gfx950 run at about 27 Gatom/s chip-wide (about 88 M/s on one hot address),
// so every key must be counted in LDS:
//   1. partition: each workgroup multi-splits a tile of kTileKeys keys into 32768-bin buckets
//      (bucket = key >> 15) and writes the 15-bit in-bucket offsets, grouped by bucket,
//      as u16 (tile-major), plus the tile's bucket offsets and bucket totals. XCD-aware
//      mode reads the keys as routed tiles: each I/O die's workgroups read only the 8 KiB
//      key chunks that die homes (the reference's side-aware chunks); rotated reads the far
//      chunks; oblivious reads contiguous tiles;
//   2. plan (at the start of every count workgroup, from the per-XCD bucket totals): deals
//      the counting work items (bucket, tile range) to the buckets in proportion to their
//      totals; XCD-aware mode lays the items out so that every XCD gets a contiguous range
//      of buckets (bins range-partitioned per XCD) and an equal share of keys, and only that
//      XCD's workgroups count them;
//   3. count: one workgroup per item keeps a 128 KB LDS histogram of its bucket, adds each
//      key with a ds_add (the wave's most common key is peeled into one add), and writes
//      the LDS histogram to its partial slot;
//   4. merge: counts = sum of the bucket's partial slots, eight partials in flight per
//      thread, units spread over the whole grid in every mode.
#include <hip/hip_runtime.h>


#include "xd_common.hpp"

namespace xd {

// 32768 counters = 128 KB of LDS per counting workgroup (16384-bin buckets, two workgroups
// per CU, counted no faster: 188 against 186 us at 2^28 keys, with a slower plan and merge).
constexpr int kHB = 15;
constexpr uint32_t kBucketBins = 1u << kHB;
// Keys per partition tile: whole 16-byte vectors per thread and whole 16 KiB pairs per
// routed tile. Longer tiles give the count pass longer runs (32768: count 176 us at 2^28
// keys against 208 us at 16384); 24576 measured fastest for the XCD-aware call.
constexpr int kTileKeys = 24576;
static_assert(kTileKeys % 4096 == 0 && kTileKeys < 65536, "tile shape (a tile's hot-key counts fit u16)");
// u16 slots per tile in the workspace: 128 bytes past the tile, so that the runs of tiles 16
// apart (those one count wave reads together) do not start at the same offset modulo 48 KiB.
// At 2^28 Zipf keys the count pass took 86.5 us with tiles at kTileKeys, 79.8 / 80.3 / 81.1 us
// at 64 / 128 / 256 slots more, and 84-86 us at 512 or more.
constexpr int kPartStride = kTileKeys + 64;
constexpr int kP1Threads = 1024;
constexpr int kP1Vec = kTileKeys / 4 / kP1Threads;  // uint4 loads per thread
constexpr int kMaxBuckets = 512;                    // num_bins <= 2^24
constexpr int kP2Threads = 1024;
constexpr int kP2Waves = kP2Threads / kWave;
constexpr int kMergeThreads = 256;
constexpr int kMergeBins = 1024;  // bins per merge unit (4 per thread)
constexpr int kMergeUnitsPerBucket = kBucketBins / kMergeBins;
constexpr uint32_t kSpareKey = (uint32_t)kMaxBuckets << kHB;  // above every valid key (num_bins <= 2^24)
constexpr uint32_t kColCounters = 2048;  // partition counters per tile (buckets x columns)
// Heavy hitter peeled in the partition: each tile's row of `offs` holds the nb + 1 bucket
// offsets, then {key, count} of the tile's peeled key (kNoKey: none). One key: a second
// compare per key took the kernel to 106 scalar registers and one workgroup per CU.
constexpr int kPeelWords = 2;
constexpr int kPeelCand = 8;       // candidates voted per tile: the first key of lanes 0..7 of wave 0
constexpr uint32_t kPeelMin = 8;   // ... peeled when at least 8 of the 256 samples match
constexpr uint32_t kNoKey = 0xffffffffu;
// Hot-key table: a sampling pass picks up to kHotSlots keys drawn at least kHotMin times
// among kHotSamples sampled keys; the partition counts them in LDS (one dense row of
// kHotSlots counters per tile) instead of writing their u16 offsets, and the count pass adds
// those rows into its bucket's histogram. A key's slot is direct-mapped (hot_slot(key)); a
// tile's row holds the slots' counters in key order (slot i at row position perm[i]), so the
// hot keys of one bucket hold a contiguous range of every row.
constexpr int kHotSlots = 256;
constexpr int kHotCopies = 8;  // partition: lane l counts a hot key in copy l % 8 of its counter (4: +6 us)
constexpr int kHotSamples = 8192;
constexpr int kHotBlocks = 32;               // samples: 32 runs of 256 consecutive keys, evenly spaced
constexpr int kHotTable = 16384;             // sampling pass: open-addressed LDS table (128 KB)
constexpr uint32_t kHotMin = 2;
constexpr size_t kHotMinKeys = size_t(1) << 20;  // smaller calls skip the sampling launch
// hot region of the workspace: tab[kHotSlots] (key or kNoKey), perm[kHotSlots] (row position
// of each slot), sorted[kHotSlots] (key at each row position), total[kHotSlots] (the count of
// the key at each row position, summed by the count pass), first[kMaxBuckets + 1]
constexpr int kHotTab = 0, kHotPerm = kHotSlots, kHotSorted = 2 * kHotSlots, kHotTotal = 3 * kHotSlots,
              kHotFirst = 4 * kHotSlots;
constexpr int kHotWords = 4 * kHotSlots + kMaxBuckets + 1;

struct HistBucket {
    int first;  // first item (= partial slot) of this bucket
    int count;  // items of this bucket (0: the bucket is empty)
};

struct HistLayout {
    int nb, ntiles, per_xcd, nitems;
    size_t part, offs, tot, buckets, partials, hot, hot_part, ones, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static HistLayout hist_layout(size_t n, uint32_t num_bins) {
    HistLayout L{};
    L.nb = (int)((num_bins + kBucketBins - 1) / kBucketBins);
    if (L.nb < 1) L.nb = 1;
    // Tile slots: contiguous calls use at most ceil(n / kTileKeys) + 1 (vector tiles and the
    // last n % 4 keys); routed calls at most ceil(pair keys / kTileKeys) + 2 (a short last
    // group cuts one short tile per die) plus two each for the keys before and after the pairs.
    L.ntiles = (int)((n + kTileKeys - 1) / kTileKeys) + 6;
    L.per_xcd = (L.nb + kNumXcd - 1) / kNumXcd + 8;
    if (L.per_xcd < 32) L.per_xcd = 32;
    L.nitems = L.per_xcd * kNumXcd;
    // Regions whose offsets depend only on num_bins come first, so a workspace sized for
    // more keys keeps its zeroed counters at the same place for every n.
    size_t o = 0;
    L.tot = o;
    o = align256(o + (size_t)kNumXcd * L.nb * sizeof(uint32_t));
    L.buckets = o;
    o = align256(o + (size_t)L.nb * sizeof(HistBucket));
    L.partials = o;
    o = align256(o + (size_t)L.nitems * kBucketBins * sizeof(uint32_t));
    L.offs = o;
    o = align256(o + (size_t)L.ntiles * (L.nb + 1 + kPeelWords) * sizeof(uint32_t));
    L.part = o;
    o = align256(o + (size_t)L.ntiles * kPartStride * sizeof(uint16_t));
    // hot-key table (kHotWords), then one row of kHotSlots u16 counters per tile (a tile holds
    // fewer than 2^16 keys)
    L.hot = o;
    o = align256(o + (size_t)kHotWords * sizeof(uint32_t));
    L.hot_part = o;
    o = align256(o + (size_t)L.ntiles * kHotSlots * sizeof(uint16_t));
    // an 8 KiB chunk of all-ones keys (written by the sampling pass)
    L.ones = o;
    o = align256(o + kHomeChunk);
    L.total = o;
    return L;
}

// A 16-byte non-temporal load, for data read exactly once: the partition's key stream and
// the count pass's runs (at 2^28 keys, aware: partition 272 -> 242 us, count 165 -> 179 us
// with only the key stream non-temporal, 179 -> 169-179 us with both).
__device__ __forceinline__ uint4 load_stream(const uint4 *p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

// A 16-byte non-temporal store, for the partition's runs: 0.5 GiB at 2^28 keys, read once by
// the count pass a pass later, never from cache. At 2^28 Zipf keys, aware: partition 208.3 ->
// 207.1 us and count 68.6 -> 65.6 us against ordinary stores (the count pass no longer meets
// the write-backs of the runs' dirty lines); contiguous tiles: 216.4 -> 220.1 and 70.1 ->
// 64.9 us.
__device__ __forceinline__ void store_stream(uint4 *p, const uint4 &v) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(v4u{v.x, v.y, v.z, v.w}, reinterpret_cast<v4u *>(p));
}

// ---------------------------------------------------------------------------------------
// 0. hot keys (one workgroup): which keys the partition counts in LDS
// ---------------------------------------------------------------------------------------
// A key's slot: its low bits (one VALU op: the partition is bound by VALU issue, where a
// multiplicative hash's 32-bit multiply ran at a quarter of the rate). Consecutive hot keys
// get distinct slots; keys equal in their low 8 bits share one, the most sampled winning it.
__device__ __forceinline__ uint32_t hot_slot(uint32_t key) { return key & (kHotSlots - 1); }

// Samples kHotSamples keys (kHotBlocks evenly spaced runs of consecutive keys: one page
// each, where single keys spread over the whole array cost a translation miss apiece), counts
// them in an open-addressed LDS table, and gives each direct-mapped slot the most sampled key
// that maps to it (at least kHotMin samples; ties to the larger key, so the table is a
// function of the keys alone). Which keys are hot changes where they are counted, never the
// counts. Needs n >= kHotSamples.
__global__ void __launch_bounds__(1024) hist_hot_kernel(const uint32_t *__restrict__ keys, size_t n, uint32_t num_bins,
                                                        int nb, uint32_t *__restrict__ hot, uint32_t *__restrict__ ones) {
    constexpr int kPer = kHotSamples / 1024;
    constexpr int kRun = kHotSamples / kHotBlocks;
    static_assert(1024 == 4 * kHotSlots, "the rank loop runs four threads per slot");
    __shared__ __attribute__((aligned(16))) uint32_t tk[kHotTable], tc[kHotTable];
    __shared__ unsigned long long best[kHotSlots];
    __shared__ __attribute__((aligned(16))) uint32_t skey[kHotSlots];
    __shared__ uint32_t ssorted[kHotSlots], s_rank[kHotSlots];
    __shared__ uint32_t s_empty[kHotSlots / kWave], s_valid;
    const int tid = (int)threadIdx.x;
    uint32_t smp[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = tid + k * 1024;
        smp[k] = keys[(size_t)(i / kRun) * (n / kHotBlocks) + (size_t)(i % kRun)];
    }
    for (int i = tid; i < kHotTable / 4; i += 1024) {
        reinterpret_cast<uint4 *>(tk)[i] = make_uint4(kNoKey, kNoKey, kNoKey, kNoKey);
        reinterpret_cast<uint4 *>(tc)[i] = make_uint4(0, 0, 0, 0);
    }
    if (tid < kHotSlots) best[tid] = 0ull;
    // the lean partition's stand-in for vectors past the end of a routed group
    reinterpret_cast<uint2 *>(ones)[tid] = make_uint2(0xffffffffu, 0xffffffffu);
    __syncthreads();
    // First probes of all kPer samples issued together (one LDS round trip for the lot; the
    // compare-and-swap claims an empty entry or returns its key), then the rare ones that met
    // another key walk on one by one. kHotSamples < kHotTable: a free or matching entry is
    // always found.
    uint32_t hh[kPer], cur[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        hh[k] = (smp[k] * 0x85EBCA6Bu) >> (32 - 14);
        cur[k] = smp[k] < num_bins ? atomicCAS(&tk[hh[k]], kNoKey, smp[k]) : smp[k];
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t key = smp[k];
        if (key >= num_bins) continue;
        uint32_t h = hh[k], c = cur[k];
        for (int probe = 0; probe < kHotTable && !(c == kNoKey || c == key); ++probe) {
            h = (h + 1) & (kHotTable - 1);
            c = atomicCAS(&tk[h], kNoKey, key);
        }
        atomicAdd(&tc[h], 1u);
    }
    __syncthreads();
    for (int i = tid; i < kHotTable / 4; i += 1024) {
        const uint4 k4 = reinterpret_cast<const uint4 *>(tk)[i], c4 = reinterpret_cast<const uint4 *>(tc)[i];
        const uint32_t kw[4] = {k4.x, k4.y, k4.z, k4.w}, cw[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (kw[c] != kNoKey && cw[c] >= kHotMin) atomicMax(&best[hot_slot(kw[c])], ((unsigned long long)cw[c] << 32) | kw[c]);
    }
    __syncthreads();
    if (tid < kHotSlots) skey[tid] = best[tid] ? (uint32_t)best[tid] : kNoKey;
    __syncthreads();
    // row position of slot i: the rank of its key among the valid keys (distinct; kNoKey sorts
    // last), empty slots after them in slot order (their place from the waves' ballots)
    // (four threads per slot, a quarter of the entries each)
    if (tid < kHotSlots) {
        const int lane = tid % kWave, wave = tid / kWave;
        const uint64_t empty = __ballot(skey[tid] == kNoKey);
        if (lane == 0) s_empty[wave] = (uint32_t)__builtin_popcountll(empty);
        s_rank[tid] = 0;
    }
    __syncthreads();
    {
        const int slot = tid % kHotSlots, part = tid / kHotSlots;
        const uint32_t key = skey[slot];
        uint32_t below = 0;
        const uint4 *s4 = reinterpret_cast<const uint4 *>(skey) + part * (kHotSlots / 16);
#pragma unroll
        for (int q = 0; q < kHotSlots / 16; ++q) {
            const uint4 v = s4[q];
            below += (v.x < key ? 1u : 0u) + (v.y < key ? 1u : 0u) + (v.z < key ? 1u : 0u) + (v.w < key ? 1u : 0u);
        }
        if (below) atomicAdd(&s_rank[slot], below);
    }
    __syncthreads();
    if (tid < kHotSlots) {
        const uint32_t key = skey[tid];
        const int lane = tid % kWave, wave = tid / kWave;
        uint32_t nempty = 0, empty_before = 0;
        for (int w = 0; w < kHotSlots / kWave; ++w) {
            nempty += s_empty[w];
            empty_before += w < wave ? s_empty[w] : 0u;
        }
        const uint64_t empty = __ballot(key == kNoKey);
        empty_before += (uint32_t)__builtin_popcountll(empty & ((1ull << lane) - 1));
        const uint32_t nvalid = kHotSlots - nempty;
        const uint32_t pos = key != kNoKey ? s_rank[tid] : nvalid + empty_before;
        hot[kHotTab + tid] = key;
        hot[kHotPerm + tid] = pos;
        hot[kHotSorted + pos] = key;
        hot[kHotTotal + tid] = 0u;
        ssorted[pos] = key;
        if (tid == 0) s_valid = nvalid;
    }
    __syncthreads();
    // first[b]: the row position of bucket b's first key (a binary search over the sorted keys)
    for (int b = tid; b <= nb; b += 1024) {
        uint32_t lo = 0, hi = s_valid;
        while (lo < hi) {
            const uint32_t mid = (lo + hi) / 2;
            if ((ssorted[mid] >> kHB) < (uint32_t)b) lo = mid + 1;
            else hi = mid;
        }
        hot[kHotFirst + b] = lo;
    }
}

// ---------------------------------------------------------------------------------------
// 1. partition
// ---------------------------------------------------------------------------------------
// Key sources of a partition workgroup.
enum PartKind { kPartFull = 0, kPartRange = 1, kPartRouted = 2 };
constexpr int kRouteGroupPairs = kTileKeys / 2048;  // 16 KiB pairs per routed tile pair

struct PartSrc {
    const uint32_t *keys;  // the call's keys (key 0)
    size_t r0, r1;         // full / range: keys [r0, r1), tile k of the launch at r0 + k * kTileKeys
                           // (full: keys + r0 16-byte aligned, r1 - r0 a non-zero multiple of 4)
    int tile0;             // full / range: tile index of the launch's first tile
    int groups;            // routed: groups of up to kRouteGroupPairs pairs, two tiles each
    uint64_t pair_first;   // routed: first 16 KiB pair (address / 16 KiB) of the first group
    uint64_t npairs;       // routed: pairs in all groups (the last group may be short)
    int mode;              // routed: XD_MODE_AWARE (near chunks) or XD_MODE_ROTATED (far chunks)
    HomeMap home;          // routed
    XcdHint xh;            // routed: workgroup -> XCD placement
};

// PACK (at most kPackBuckets buckets, full and routed kinds): each counter column takes one
// lane of each of the 16 waves, so a key's slot inside its column is below 16 * (keys per
// thread) and shares the key's register (key or the spare 2^20 in bits 0-20, slot from bit
// 21): the live state across the scan is then one register per key.
constexpr int kPackBuckets = kColCounters / kWave;
constexpr uint32_t kPackSpare = (uint32_t)kPackBuckets << kHB;
constexpr int kPackShift = 21;
static_assert(kPackSpare == (1u << (kPackShift - 1)), "packed keys and the spare fit below the slot bits");
static_assert((kPackSpare >> kHB) * kWave == kColCounters, "the packed spare key's counter row is the spare row");
static_assert(kP1Threads / kWave * 4 * kP1Vec * (kWave * kPackBuckets / kColCounters) <= (1 << (32 - kPackShift)),
              "packed slots overflow");

template <int KIND, bool PACK>
__device__ __forceinline__ void partition_tile(PartSrc src, uint32_t num_bins, int nb, uint16_t *__restrict__ part,
                                               uint32_t *__restrict__ offs, uint32_t *__restrict__ tot,
                                               const uint32_t *__restrict__ hot, uint16_t *__restrict__ hot_part) {
    // Every bucket's counter is split into S columns, column = lane % S (S = 64 for up to
    // 32 buckets), laid out col[b * S + s]: the lanes of one LDS add never share an address,
    // so a wave's 64 adds do not serialise on a popular bucket. col[kColCounters + s] and
    // stage[kTileKeys] are spares: the full and routed kinds replace a key outside
    // [0, num_bins) by kSpareKey, whose add and store land there, so no key needs a branch.
    __shared__ uint32_t col[kColCounters + kWave];
    __shared__ uint32_t wsum[kP1Threads / kWave];
    __shared__ uint32_t s_total;
    __shared__ uint32_t s_hot, s_hotc;
    __shared__ __attribute__((aligned(16))) uint16_t stage[kTileKeys + 8];
    constexpr bool VEC = KIND != kPartRange;
    const int g = (int)blockIdx.x;
    int t;
    uint32_t want = 0;
    int grp = 0;
    if (KIND == kPartRouted) {
        // Routed: group i's pairs each hold one 8 KiB chunk on either I/O die; tile 2i + d
        // is the group's chunks homed on die d, read by a workgroup of die d (aware) or of
        // the other die (rotated). The grid holds at least `groups` workgroups per die.
        report_xcd(src.xh);
        grp = die_rank(g, src.xh);
        if (grp >= src.groups) return;
        want = src.mode == XD_MODE_AWARE ? wg_die(g, src.xh) : (wg_die(g, src.xh) ^ 1u);
        t = 2 * grp + (int)want;
    } else {
        t = src.tile0 + g;
    }
    const int tid = (int)threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    int S = kWave;
    while (S > 1 && nb * S > (int)kColCounters) S >>= 1;
    const int ncol = nb * S;
    const uint32_t my_col = (uint32_t)(lane & (S - 1));
    for (int i = tid; i < (int)kColCounters + kWave; i += kP1Threads) col[i] = 0;

    // Full / routed: tiles of 16-byte vectors; a vector past the end of the range is loaded
    // clamped to the last one and its keys become spares, so no load sits under a branch
    // (the launcher sends unaligned keys and the last n % 4 keys to the range kind, whose
    // per-key loads would otherwise set these kinds' register count). The out-of-range mask
    // is hidden from the compiler: seeing a masked vector's value unused, it would load the
    // other vectors' words one by one under branches, each join waiting for every load.
    uint32_t kk[4 * kP1Vec];
    constexpr uint32_t spare = PACK ? kPackSpare : kSpareKey;
    auto keep = [&](int j, uint4 v, bool ok) {
        uint32_t m = ok ? 0u : 0xffffffffu;  // out of range: every word reads as 0xffffffff
        asm volatile("" : "+v"(m));
        const uint32_t x = v.x | m, y = v.y | m, z = v.z | m, w = v.w | m;
        kk[4 * j] = x < num_bins ? x : spare;
        kk[4 * j + 1] = y < num_bins ? y : spare;
        kk[4 * j + 2] = z < num_bins ? z : spare;
        kk[4 * j + 3] = w < num_bins ? w : spare;
    };
    if (KIND == kPartFull) {
        const uint4 *kv = reinterpret_cast<const uint4 *>(src.keys + src.r0);
        const size_t nvec = (src.r1 - src.r0) / 4;
        const size_t v0 = (size_t)g * (kTileKeys / 4);
#pragma unroll
        for (int j = 0; j < kP1Vec; ++j) {
            const size_t v = v0 + (size_t)(tid + j * kP1Threads);
            const bool ok = v < nvec;
            keep(j, load_stream(&kv[ok ? v : nvec - 1]), ok);
        }
    } else if (KIND == kPartRouted) {
        // The group spans at most kRouteGroupPairs * 16 KiB <= 2 MiB, so at most two map
        // pages: the even chunk of a pair has address bit 13 clear, so its home is its page's
        // attribute and the odd chunk is homed on the other die.
        const uint64_t A = reinterpret_cast<uint64_t>(src.keys);
        const uint64_t P0 = src.pair_first + (uint64_t)grp * kRouteGroupPairs;
        const uint64_t np = min((uint64_t)kRouteGroupPairs, src.npairs - (uint64_t)grp * kRouteGroupPairs);
        const uint64_t pg_lo = (P0 * 16384) / kHomePage;
        const uint64_t pg_hi = ((P0 + np) * 16384 - 1) / kHomePage;
        uint32_t h_lo, h_hi;
        if (src.home.attr) {
            h_lo = src.home.attr[pg_lo - src.home.page0];
            h_hi = src.home.attr[pg_hi - src.home.page0];
        } else {
            h_lo = home_of(pg_lo * kHomePage, src.home.mask);
            h_hi = home_of(pg_hi * kHomePage, src.home.mask);
        }
        const uint4 *kv = reinterpret_cast<const uint4 *>(src.keys);
#pragma unroll
        for (int j = 0; j < kP1Vec; ++j) {
            const int vi = tid + j * kP1Threads;  // vector of the tile: 512 per 8 KiB chunk
            const bool ok = (uint64_t)(vi >> 9) < np;
            const uint64_t P = P0 + (ok ? (uint64_t)(vi >> 9) : np - 1);
            const uint32_t h0 = (P * 16384) / kHomePage == pg_lo ? h_lo : h_hi;
            const uint64_t chunk = 2 * P + (h0 ^ want);
            keep(j, load_stream(&kv[(chunk * kHomeChunk - A) / 16 + (uint64_t)(vi & 511)]), ok);
        }
    } else {
        const size_t k0 = src.r0 + (size_t)g * kTileKeys;
#pragma unroll
        for (int j = 0; j < kP1Vec; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                size_t idx = k0 + 4 * (size_t)(tid + j * kP1Threads) + c;
                kk[4 * j + c] = idx < src.r1 ? src.keys[idx] : 0xffffffffu;
            }
    }
    // Heavy hitter: wave 0 votes the tile's most frequent key among kPeelCand candidates on
    // 256 samples (the first four keys of each lane); every thread then counts that key in a
    // register and makes it a spare, so it is neither staged nor written: under a skewed
    // stream it is a large share of the u16 offsets the count pass would read back. The
    // tile's {key, count} goes after its bucket offsets; the count pass adds it.
    if (VEC && wave == 0) {
        uint32_t b1 = kNoKey, c1 = 0;
        // (calls with a hot-key table run the lean kinds, which peel nothing)
#pragma unroll 1
        for (int j = 0; j < kPeelCand; ++j) {
            const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)kk[0], j);
            const uint32_t m = (kk[0] == c ? 1u : 0u) + (kk[1] == c ? 1u : 0u) + (kk[2] == c ? 1u : 0u) +
                               (kk[3] == c ? 1u : 0u);
            const uint32_t n = wave_sum_u32(m);
            if (c != spare && n > c1) {  // wave-uniform
                b1 = c;
                c1 = n;
            }
        }
        if (lane == 0) {
            s_hot = c1 >= kPeelMin ? b1 : kNoKey;
            s_hotc = 0;
        }
    }
    __syncthreads();
    uint32_t h1 = kNoKey;
    if (VEC) {
        h1 = s_hot;
        if (h1 != kNoKey) {  // (uniform)
            uint32_t n1 = 0;
#pragma unroll
            for (int j = 0; j < 4 * kP1Vec; ++j) {
                const bool m1 = kk[j] == h1;
                n1 += m1 ? 1u : 0u;
                kk[j] = m1 ? spare : kk[j];
            }
            n1 = wave_sum_u32(n1);
            if (lane == 0 && n1) atomicAdd(&s_hotc, n1);
        }
    }

    // Counter index of a key: its bucket's row, this lane's column (a spare key's row is past
    // the table, so the clamp sends it to this lane's spare counter). Packed (at most
    // kPackBuckets buckets, so S = kWave): the spare key kPackSpare is bucket kPackBuckets,
    // whose row is exactly the spare counters, so no clamp is needed.
    auto slot_of = [&](uint32_t key) -> uint32_t {
        if (PACK) return ((key >> kHB) * (uint32_t)kWave) | my_col;
        return min((key >> kHB) * (uint32_t)S + my_col, kColCounters + my_col);
    };

    // Slot of every key inside its column: a returning LDS add. Unpacked, slots stay below
    // kTileKeys <= 2^16, so two share a register.
    uint32_t pos2[PACK ? 1 : 2 * kP1Vec];
#pragma unroll
    for (int j = 0; j < 4 * kP1Vec; j += 2) {
        const uint32_t a = kk[j], b = kk[j + 1];
        uint32_t pa = 0, pb = 0;
        if (VEC) {
            pa = atomicAdd(&col[slot_of(a)], 1u);
            pb = atomicAdd(&col[slot_of(b)], 1u);
        } else {
            if (a < num_bins) pa = atomicAdd(&col[slot_of(a)], 1u);
            if (b < num_bins) pb = atomicAdd(&col[slot_of(b)], 1u);
        }
        if (PACK) {
            kk[j] = a | (pa << kPackShift);
            kk[j + 1] = b | (pb << kPackShift);
        } else {
            pos2[j / 2] = pa | (pb << 16);
        }
    }
    // Redefine the keys so the scatter recomputes their LDS addresses instead of keeping them
    // live across the scan.
#pragma unroll
    for (int j = 0; j < 4 * kP1Vec; ++j) asm volatile("" : "+v"(kk[j]));
    __syncthreads();

    // Exclusive scan of the ncol <= kColCounters counters in (bucket, column) order, two per
    // thread; afterwards col[b * S] is where bucket b starts inside the tile.
    const int i0 = 2 * tid;
    const uint32_t c0 = i0 < ncol ? col[i0] : 0u;
    const uint32_t c1 = i0 + 1 < ncol ? col[i0 + 1] : 0u;
    const uint32_t v = c0 + c1;
    const uint32_t incl = wave_incl_scan_u32(v);
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        const uint32_t w = lane < kP1Threads / kWave ? wsum[lane] : 0u;
        const uint32_t wi = wave_incl_scan_u32(w);
        if (lane < kP1Threads / kWave) wsum[lane] = wi - w;
        if (lane == kP1Threads / kWave - 1) s_total = wi;
    }
    __syncthreads();
    {
        const uint32_t e = wsum[wave] + incl - v;
        if (i0 < ncol) col[i0] = e;
        if (i0 + 1 < ncol) col[i0 + 1] = e + c0;
    }
    if (tid < kWave) col[kColCounters + tid] = kTileKeys;  // spare slots land on stage[kTileKeys]
    __syncthreads();

    uint32_t *my_offs = offs + (size_t)t * (nb + 1 + kPeelWords);
    uint32_t *my_tot = tot + (size_t)(t % kNumXcd) * nb;
#pragma unroll
    for (int j = 0; j < 4 * kP1Vec; ++j) {
        const uint32_t key = PACK ? kk[j] & ((1u << kPackShift) - 1) : kk[j];
        const uint32_t pos = PACK ? kk[j] >> kPackShift : (pos2[j / 2] >> (16 * (j & 1))) & 0xffffu;
        const uint16_t low = (uint16_t)(key & (kBucketBins - 1));
        if (VEC)
            stage[min(col[slot_of(key)] + pos, (uint32_t)kTileKeys)] = low;
        else if (key < num_bins)
            stage[col[slot_of(key)] + pos] = low;
    }
    __syncthreads();
    const uint32_t tile_total = s_total;
    for (int b = tid; b < nb; b += kP1Threads) {
        const uint32_t start = col[b * S];
        const uint32_t end = b + 1 < nb ? col[(b + 1) * S] : tile_total;
        my_offs[b] = start;
        if (end > start) atomicAdd(&my_tot[b], end - start);
    }
    if (tid == 0) {
        my_offs[nb] = tile_total;
        my_offs[nb + 1] = h1;  // s_hotc is final: every wave added before the last barriers
        my_offs[nb + 2] = VEC ? s_hotc : 0u;
        // a bucket whose keys were all peeled still needs a counting item, which the plan
        // deals only to buckets with a non-zero total: one unit per peeling tile is enough
        if (VEC && h1 != kNoKey && s_hotc) atomicAdd(&my_tot[h1 >> kHB], 1u);
    }
    // The range kind runs beside the lean kinds in calls with a hot-key table (the keys before
    // and after the vector tiles): its tiles add no hot counts, so their rows are zero, as the
    // count pass sums the rows of every tile. (The other generic kinds run without a table.)
    if (KIND == kPartRange && hot != nullptr && tid < kHotSlots) hot_part[(size_t)t * kHotSlots + tid] = 0;

    const uint32_t nvec = (tile_total + 7) / 8;  // 8 u16 per 16-byte store
    const uint4 *from = reinterpret_cast<const uint4 *>(stage);
    uint4 *dst = reinterpret_cast<uint4 *>(part + (size_t)t * kPartStride);
    for (uint32_t i = (uint32_t)tid; i < nvec; i += kP1Threads) store_stream(&dst[i], from[i]);
}

// Two workgroups of 16 waves share a CU only while a wave holds at most 80 scalar registers
// in all (measured: the routed packed kind at 82 ran at half the resident waves, 408 against
// 286 us at 2^28 keys, though the compiler's occupancy estimate said 8 waves per SIMD), so
// the packed and lean kinds are capped (78 requested gives 76 in all; 74 gave 72 but spilled
// half again as many scalars to vector lanes); the unpacked ones stay within 80 uncapped, and
// a cap would cost them a vector register past 64.
constexpr int kPartPackedSgprs = 78;

template <int KIND>
__global__ void __launch_bounds__(kP1Threads) __attribute__((amdgpu_num_sgpr(kPartPackedSgprs)))
hist_partition_packed_kernel(PartSrc src, uint32_t num_bins, int nb, uint16_t *__restrict__ part,
                             uint32_t *__restrict__ offs, uint32_t *__restrict__ tot, const uint32_t *__restrict__ hot,
                             uint16_t *__restrict__ hot_part) {
    partition_tile<KIND, true>(src, num_bins, nb, part, offs, tot, hot, hot_part);
}

template <int KIND>
__global__ void __launch_bounds__(kP1Threads)
hist_partition_kernel(PartSrc src, uint32_t num_bins, int nb, uint16_t *__restrict__ part, uint32_t *__restrict__ offs,
                      uint32_t *__restrict__ tot, const uint32_t *__restrict__ hot, uint16_t *__restrict__ hot_part) {
    partition_tile<KIND, false>(src, num_bins, nb, part, offs, tot, hot, hot_part);
}

// ---------------------------------------------------------------------------------------
// 1b. lean partition: calls with a hot-key table into at most kPackBuckets buckets
// ---------------------------------------------------------------------------------------
// The packed multi-split of partition_tile with the per-key work cut to what the split needs.
// The generic kinds spend about 30 VALU instructions and 5 LDS instructions a key; the LDS
// pipe then bounds the pass (dropping only the stage stores from a timing copy saved 31 us
// of 236 at 2^28 keys; the key loads alone take 183 us).
//  * a wave's 64 key vectors are consecutive (in a routed tile, inside one 8 KiB chunk), so
//    their addresses are wave-uniform and computed with scalar instructions; a vector past
//    the end of a routed group is loaded from an 8 KiB chunk of all-ones keys in the
//    workspace instead, so no key carries a range flag;
//  * one min() guards the range: bound = nb << kHB, so a key at or above it becomes `bound`,
//    whose counter row (row nb) is the spare row; a key in [num_bins, bound) is split like any
//    key of the last bucket, counted past num_bins by the count pass and dropped by the merge
//    (which writes bins below num_bins only);
//  * one returning LDS add per key: a hot key adds to its hot counter (lane % 8's copy), any
//    other key to its counter column, and the hot key's returned value is dropped: it
//    becomes a spare at slot `lane` of the spare row (the stage's trash);
//  * a key's slot in its column is packed at bit kLeanShift, one above the key's bit 20, so
//    x >> (kLeanShift - 1) is twice the slot: the stage byte address in one more op;
//  * the stage has room past kTileKeys for every spare position, so the scatter needs no
//    clamp, and it stores the packed register's low half as it is: bits 0-14 the in-bucket
//    offset, bit 15 the bucket's low bit, which the count pass masks off in the same
//    instruction that extracts the u16.
constexpr int kLeanRows = kPackBuckets + 1;                    // bucket rows, then the spare row
constexpr int kLeanCopyStride = kHotSlots + 1;                 // copies of one slot in different banks
constexpr int kLeanColumnKeys = kP1Threads / kWave * 4 * kP1Vec;  // keys one counter column can take
constexpr int kLeanStage = kTileKeys + kLeanColumnKeys;
static_assert(kLeanStage % 8 == 0, "the stage is copied out in 16-byte vectors");
static_assert(kLeanColumnKeys >= kWave, "a hot key's trash slot (its lane) is a spare position");
constexpr int kLeanShift = 22;  // keys <= kPackSpare = 2^20: bit 21 stays clear
static_assert(kPackSpare < (1u << (kLeanShift - 1)), "bit kLeanShift - 1 of a packed key is clear");
static_assert(kLeanColumnKeys <= (1 << (32 - kLeanShift)), "packed slots overflow");
static_assert(kLeanRows * kWave * 4 <= (0x3f00 | 0xff) + 1, "row offsets fit the 6-bit row field");

struct LeanLds {
    uint32_t col[kLeanRows * kWave];                // counter (row, lane), then each column's start
    uint32_t cnt[kHotCopies * kLeanCopyStride];     // hot counters: copy c of slot i at c * stride + i
    uint32_t tab[kHotSlots];                        // the hot-key table
    uint32_t wsum[kP1Threads / kWave];
    uint32_t total;
    uint32_t pad_[3];
    uint16_t stage[kLeanStage];
};
static_assert(offsetof(LeanLds, col) == 0, "counter byte offsets are offsets into the struct");
static_assert(offsetof(LeanLds, stage) % 16 == 0, "stage copied out with 16-byte loads");

template <int KIND>
__global__ void __launch_bounds__(kP1Threads) __attribute__((amdgpu_num_sgpr(kPartPackedSgprs)))
hist_partition_lean_kernel(PartSrc src, uint32_t bound, int nb, uint16_t *__restrict__ part,
                           uint32_t *__restrict__ offs, uint32_t *__restrict__ tot, const uint32_t *__restrict__ hot,
                           uint16_t *__restrict__ hot_part, const uint32_t *__restrict__ ones) {
    __shared__ __attribute__((aligned(16))) LeanLds S;
    const int g = (int)blockIdx.x;
    const int tid = (int)threadIdx.x;
    const int lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    int t;
    uint32_t want = 0;
    int grp = 0;
    if (KIND == kPartRouted) {
        // as partition_tile: tile 2i + d is group i's chunks homed on die d
        report_xcd(src.xh);
        grp = die_rank(g, src.xh);
        if (grp >= src.groups) return;
        want = src.mode == XD_MODE_AWARE ? wg_die(g, src.xh) : (wg_die(g, src.xh) ^ 1u);
        t = 2 * grp + (int)want;
    } else {
        t = src.tile0 + g;
    }

    // the table words first: the first barrier waits for them, and the counter is in order
    uint32_t my_perm = 0, my_tab = 0;
    if (tid < kHotSlots) {
        my_tab = hot[kHotTab + tid];
        my_perm = hot[kHotPerm + tid];
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t kk[4 * kP1Vec];
    auto put = [&](int j, const uint4 &v) {
        kk[4 * j] = v.x;
        kk[4 * j + 1] = v.y;
        kk[4 * j + 2] = v.z;
        kk[4 * j + 3] = v.w;
    };
    if (KIND == kPartFull) {
        // keys + r0 is 16-byte aligned; only the launch's last tile can be partial
        const uint4 *kv = reinterpret_cast<const uint4 *>(src.keys + src.r0) + (size_t)g * (kTileKeys / 4);
        const size_t left = (src.r1 - src.r0) / 4 - (size_t)g * (kTileKeys / 4);  // vectors from this tile on
        if (left >= (size_t)(kTileKeys / 4)) {
#pragma unroll
            for (int j = 0; j < kP1Vec; ++j) put(j, load_stream(kv + tid + j * kP1Threads));
        } else {
            // (uniform branch) a vector past the end reads the all-ones chunk, whose keys the
            // guard turns into spares
#pragma unroll
            for (int j = 0; j < kP1Vec; ++j) {
                const uint32_t v = (uint32_t)(tid + j * kP1Threads);
                put(j, load_stream(v < left ? kv + v : reinterpret_cast<const uint4 *>(ones) + ((uint32_t)tid & 511u)));
            }
        }
    } else {
        // Routed: vector tid + j * kP1Threads of the tile is vector tid % 512 of the chunk of
        // pair 2j + tid / 512 of the group; tid / 512 = wave / 8, so the chunk is wave-uniform.
        // The group spans at most kRouteGroupPairs * 16 KiB <= 2 MiB, so at most two map pages:
        // the even chunk of a pair has address bit 13 clear, so its home is its page's.
        const uint64_t A = reinterpret_cast<uint64_t>(src.keys);
        const uint64_t P0 = src.pair_first + (uint64_t)grp * kRouteGroupPairs;
        const uint32_t np = (uint32_t)min((uint64_t)kRouteGroupPairs, src.npairs - (uint64_t)grp * kRouteGroupPairs);
        const uint64_t pg_lo = (P0 * 16384) / kHomePage;
        const uint64_t pg_hi = ((P0 + np) * 16384 - 1) / kHomePage;
        uint32_t h_lo, h_hi;
        if (src.home.attr) {
            h_lo = __builtin_amdgcn_readfirstlane((uint32_t)src.home.attr[pg_lo - src.home.page0]);
            h_hi = __builtin_amdgcn_readfirstlane((uint32_t)src.home.attr[pg_hi - src.home.page0]);
        } else {
            h_lo = home_of(pg_lo * kHomePage, src.home.mask);
            h_hi = home_of(pg_hi * kHomePage, src.home.mask);
        }
        const uint32_t lv = (uint32_t)tid & 511u;
#pragma unroll
        for (int j = 0; j < kP1Vec; ++j) {
            const uint32_t pi = (uint32_t)(2 * j + wave / 8);
            const uint64_t P = P0 + min(pi, np - 1u);
            const uint32_t h0 = (P * 16384) / kHomePage == pg_lo ? h_lo : h_hi;
            // (chunk addresses as offsets from the keys pointer: a global pointer, not flat)
            const uint32_t *chunk = src.keys + ((2 * P + (h0 ^ want)) * kHomeChunk - A) / 4;
            const uint32_t *base = pi < np ? chunk : ones;
            put(j, load_stream(reinterpret_cast<const uint4 *>(base) + lv));
        }
    }

    // counters zeroed and the table copied in after the loads are issued
    for (int i = tid; i < kLeanRows * kWave; i += kP1Threads) S.col[i] = 0;
    for (int i = tid; i < kHotCopies * kLeanCopyStride; i += kP1Threads) S.cnt[i] = 0;
    if (tid < kHotSlots) S.tab[tid] = my_tab;
    // the counters and the table are in LDS before any wave reads them; the keys are clamped
    // batch by batch below, so a batch waits only for its own loads
    __syncthreads();

    // One returning add per key (byte offsets into S): a hot key's counter copy, else the key's
    // counter column (row key >> kHB, at most the spare row, column = lane). Table keys are
    // below num_bins <= bound and empty entries are all ones, so a spare never matches.
    const uint32_t lanebyte = (uint32_t)lane * 4u;
    const uint32_t hotbase =
        (uint32_t)offsetof(LeanLds, cnt) + (uint32_t)(lane & (kHotCopies - 1)) * kLeanCopyStride * 4u;
    const uint32_t hotspare = bound | ((uint32_t)lane << kLeanShift);  // trash slot `lane` of the spare row
    char *const sb = reinterpret_cast<char *>(&S);
    auto col_off = [&](uint32_t x) { return ((x >> (kHB - 8)) & 0x3f00u) | lanebyte; };
    constexpr int kBatch = 2 * kP1Vec;
#pragma unroll
    for (int j0 = 0; j0 < 4 * kP1Vec; j0 += kBatch) {
        uint32_t e[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) kk[j0 + j] = min(kk[j0 + j], bound);
#pragma unroll
        for (int j = 0; j < kBatch; ++j) e[j] = S.tab[hot_slot(kk[j0 + j])];
        // the batch's offsets, then its adds back to back, then the packing (a hot offset is at
        // or above offsetof(cnt), every column offset below it)
        uint32_t off[kBatch], pos[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint32_t k = kk[j0 + j];
            // both offsets computed, then one select (the compiler otherwise branches per key)
            uint32_t ho = hotbase + 4u * hot_slot(k), co = col_off(k);
            asm("" : "+v"(ho), "+v"(co));
            off[j] = e[j] == k ? ho : co;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) pos[j] = atomicAdd(reinterpret_cast<uint32_t *>(sb + off[j]), 1u);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint32_t k = kk[j0 + j];
            kk[j0 + j] = off[j] >= (uint32_t)offsetof(LeanLds, cnt) ? hotspare : (k | (pos[j] << kLeanShift));
        }
    }
#pragma unroll
    for (int j = 0; j < 4 * kP1Vec; ++j) asm volatile("" : "+v"(kk[j]));
    __syncthreads();

    // exclusive scan of the nb * 64 counters in (bucket, column) order, two per thread
    const int ncol = nb * kWave;
    const int i0 = 2 * tid;
    const uint32_t c0 = i0 < ncol ? S.col[i0] : 0u;
    const uint32_t c1 = i0 + 1 < ncol ? S.col[i0 + 1] : 0u;
    const uint32_t v = c0 + c1;
    const uint32_t incl = wave_incl_scan_u32(v);
    if (lane == kWave - 1) S.wsum[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        const uint32_t w = lane < kP1Threads / kWave ? S.wsum[lane] : 0u;
        const uint32_t wi = wave_incl_scan_u32(w);
        if (lane < kP1Threads / kWave) S.wsum[lane] = wi - w;
        if (lane == kP1Threads / kWave - 1) S.total = wi;
    }
    __syncthreads();
    {
        const uint32_t e = S.wsum[wave] + incl - v;
        if (i0 < ncol) S.col[i0] = e;
        if (i0 + 1 < ncol) S.col[i0 + 1] = e + c0;
    }
    if (tid < kWave) S.col[nb * kWave + tid] = kTileKeys;  // the spare row's keys land past kTileKeys
    __syncthreads();

    // Scatter in batches: the column starts first, then the stores, hot keys' left out (their
    // trash stores shared dwords and cost bank cycles: 6.8 against 4.4 cycles per wave store
    // in a bank simulation of Zipf tiles)
#pragma unroll
    for (int j0 = 0; j0 < 4 * kP1Vec; j0 += kBatch) {
        uint32_t start[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) start[j] = *reinterpret_cast<const uint32_t *>(sb + col_off(kk[j0 + j]));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint32_t x = kk[j0 + j];
            const uint32_t byte = 2u * start[j] + (x >> (kLeanShift - 1));  // 2 (start + slot)
            if (x != hotspare) *reinterpret_cast<uint16_t *>(reinterpret_cast<char *>(S.stage) + byte) = (uint16_t)x;
        }
    }
    __syncthreads();

    const uint32_t tile_total = S.total;
    uint32_t *my_offs = offs + (size_t)t * (nb + 1 + kPeelWords);
    uint32_t *my_tot = tot + (size_t)(t % kNumXcd) * nb;
    for (int b = tid; b < nb; b += kP1Threads) {
        const uint32_t start = S.col[b * kWave];
        const uint32_t end = b + 1 < nb ? S.col[(b + 1) * kWave] : tile_total;
        my_offs[b] = start;
        if (end > start) atomicAdd(&my_tot[b], end - start);
    }
    if (tid == 0) {
        my_offs[nb] = tile_total;
        my_offs[nb + 1] = kNoKey;  // nothing peeled
        my_offs[nb + 2] = 0u;
    }
    if (tid < kHotSlots) {
        uint32_t c = 0;
#pragma unroll
        for (int k = 0; k < kHotCopies; ++k) c += S.cnt[k * kLeanCopyStride + tid];
        hot_part[(size_t)t * kHotSlots + my_perm] = (uint16_t)c;  // c <= kTileKeys < 2^16
    }
    const uint32_t nvec = (tile_total + 7) / 8;
    const uint4 *from = reinterpret_cast<const uint4 *>(S.stage);
    uint4 *dst = reinterpret_cast<uint4 *>(part + (size_t)t * kPartStride);
    for (uint32_t i = (uint32_t)tid; i < nvec; i += kP1Threads) store_stream(&dst[i], from[i]);
}

// ---------------------------------------------------------------------------------------
// 2. plan (run by every count workgroup: one thread per bucket)
// ---------------------------------------------------------------------------------------
template <int THREADS>
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t *wsum, uint32_t *total) {
    constexpr int W = THREADS / kWave;
    static_assert(W <= kWave, "one wave scans the wave sums");
    const int tid = (int)threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const uint32_t incl = wave_incl_scan_u32(v);
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        const uint32_t w = lane < W ? wsum[lane] : 0u;
        const uint32_t wi = wave_incl_scan_u32(w);
        if (lane < W) wsum[lane] = wi - w;
        if (lane == W - 1) *total = wi;
    }
    __syncthreads();
    const uint32_t r = wsum[wave] + incl - v;
    __syncthreads();
    return r;
}

struct Deal {
    uint32_t first, count;  // item slots [first, first + count) of the calling thread's bucket
};

// Thread b < nb gets bucket b's item slots (every thread of the block must call it). The slots
// are dealt to the buckets in bucket order, in proportion to their keys: bucket b starts at
// slot nzpre + floor(pre * R / N), R = slots beyond one per non-empty bucket, and the slots
// end exactly at nitems (the clamps only guard the table).
template <int THREADS>
__device__ Deal deal_items(const uint32_t *__restrict__ tot, int nb, int nitems, uint32_t *wsum) {
    __shared__ uint32_t s_total, s_nnz;
    const int b = (int)threadIdx.x;
    uint32_t T = 0;
    if (b < nb)
        for (int x = 0; x < kNumXcd; ++x) T += tot[(size_t)x * nb + b];
    const uint32_t nz = (b < nb && T > 0) ? 1u : 0u;
    const uint32_t pre = block_excl_scan<THREADS>(T, wsum, &s_total);
    const uint32_t N = s_total;
    const uint32_t nzpre = block_excl_scan<THREADS>(nz, wsum, &s_nnz);
    const uint32_t nnz = s_nnz;
    const unsigned long long R = (unsigned long long)nitems - min(nnz, (uint32_t)nitems);
    const uint32_t Nd = N ? N : 1u;
    uint32_t first = nzpre + (uint32_t)(((unsigned long long)pre * R) / Nd);
    uint32_t J = nz ? 1u + (uint32_t)(((unsigned long long)(pre + T) * R) / Nd - ((unsigned long long)pre * R) / Nd) : 0u;
    if (first > (uint32_t)nitems) first = (uint32_t)nitems;
    if (J > (uint32_t)nitems - first) J = (uint32_t)nitems - first;
    return Deal{first, J};
}

// ---------------------------------------------------------------------------------------
// 3. count
// ---------------------------------------------------------------------------------------
constexpr uint32_t kTrash = kBucketBins;  // first LDS slot past the bins (hot-key sentinel above it)
constexpr uint32_t kLaneTrash = kBucketBins + 4;  // lane l's private slot kLaneTrash + l absorbs its dropped keys
constexpr uint32_t kCountSlots = kLaneTrash + kWave;

// Counts the 8 u16 keys of one 16-byte vector whose first element has index `e`, for the
// run [s0, e0). Keys equal to the wave's two current hot keys go to the per-lane register
// counters `hc` and `hc2` (the hot keys of a Zipf bucket would otherwise make many lanes of
// a wave hit one LDS address). Every key takes one ds_add, with no branch: keys outside the
// run and hot keys are added to the lane's private trash slot `trash`, so the adds of one
// instruction never meet on a dropped key's address.
// (VOTE false: no register keys, for calls whose hot-key table took the popular keys out)
template <bool VOTE>
__device__ __forceinline__ void count_vec(uint32_t *h, const uint4 &q, uint32_t e, uint32_t s0, uint32_t e0,
                                          uint32_t hot, uint32_t hot2, uint32_t &hc, uint32_t &hc2,
                                          uint32_t trash) {
    if (e >= e0 || e + 8 <= s0) return;  // vector outside the run (most lanes' 2nd vector)
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const uint32_t len = e0 - s0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        // (15 bits: the lean partition leaves its bucket's low bit in bit 15)
        uint32_t key = (k & 1) ? ((w[k >> 1] >> 16) & (kBucketBins - 1)) : (w[k >> 1] & (kBucketBins - 1));
        key = (e + (uint32_t)k - s0 < len) ? key : trash;
        if (VOTE) {
            const bool h1 = key == hot, h2 = key == hot2;  // a trash slot is never a hot key
            hc += h1 ? 1u : 0u;
            hc2 += h2 ? 1u : 0u;
            atomicAdd(&h[(h1 | h2) ? trash : key], 1u);
        } else {
            atomicAdd(&h[key], 1u);
        }
    }
}

__global__ void __launch_bounds__(kP2Threads)
hist_count_kernel(const uint16_t *__restrict__ part, const uint32_t *__restrict__ offs, int nb, int ntiles,
                  const uint32_t *__restrict__ tot, int per_xcd, uint32_t *__restrict__ partials,
                  HistBucket *__restrict__ buckets, int mode, unsigned rot, uint32_t *__restrict__ hot_tab,
                  const uint16_t *__restrict__ hot_part, XcdHint xh) {
    __shared__ __attribute__((aligned(16))) uint32_t h[kCountSlots];
    __shared__ uint32_t wsum[kP2Waves];
    __shared__ int s_item[3];  // bucket (-1: idle slot), t0, t1
    __shared__ uint32_t s_hot[kP2Threads / (kHotSlots / 2) * kHotSlots];
    const int g = (int)blockIdx.x;
    const int tid = (int)threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    int slot;
    if (mode == XD_MODE_OBLIVIOUS) {
        slot = g;
    } else {
        XcdSlot s = xcd_slot(g, (int)gridDim.x, mode, rot, xh);
        slot = s.slice * per_xcd + s.rank;
    }
    if (tid == 0) s_item[0] = -1;
    const int nitems = per_xcd * kNumXcd;
    const Deal d = deal_items<kP2Threads>(tot, nb, nitems, wsum);  // synchronises the block
    if (tid < nb && d.count > 0 && (uint32_t)slot >= d.first && (uint32_t)slot < d.first + d.count) {
        const uint32_t j = (uint32_t)slot - d.first;
        s_item[0] = tid;
        s_item[1] = (int)((unsigned long long)j * ntiles / d.count);
        s_item[2] = (int)((unsigned long long)(j + 1) * ntiles / d.count);
    }
    if (g == 0 && tid < nb) buckets[tid] = HistBucket{(int)d.first, (int)d.count};  // the merge pass's view
    uint4 *h4 = reinterpret_cast<uint4 *>(h);
    for (int i = tid; i < (int)(kCountSlots / 4); i += kP2Threads) h4[i] = make_uint4(0, 0, 0, 0);
    // The hot-table counters: workgroup g sums the rows of tiles [g ntiles / G, (g + 1) ntiles
    // / G) (G = the grid, whatever its bucket: each thread reads one 32-bit word, two row
    // positions, of every 8th row, eight loads in flight) and adds them to the positions'
    // totals, which the merge adds to the keys' bins. (Summing each bucket's keys over its
    // items' tile ranges read one or two lines of every row per item, and took 11.5 us of the
    // 64 a median item ran at 2^28 Zipf keys.)
    if (hot_tab != nullptr) {
        const int G = (int)gridDim.x;
        const int ta = (int)((long long)g * ntiles / G), tz = (int)((long long)(g + 1) * ntiles / G);
        constexpr int W = kHotSlots / 2, Q = kP2Threads / W, U = 8;  // words per row, row streams
        const int w = tid % W, q = tid / W;
        const uint32_t *rows = reinterpret_cast<const uint32_t *>(hot_part);
        uint32_t lo = 0, hi = 0;
        for (int tt = ta + q; tt < tz; tt += U * Q) {
            uint32_t v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = rows[(size_t)min(tt + u * Q, tz - 1) * W + w];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t vv = tt + u * Q < tz ? v[u] : 0u;
                lo += vv & 0xffffu;
                hi += vv >> 16;
            }
        }
        s_hot[q * kHotSlots + 2 * w] = lo;
        s_hot[q * kHotSlots + 2 * w + 1] = hi;
        __syncthreads();
        if (tid < kHotSlots) {
            uint32_t sum = 0;
#pragma unroll
            for (int k = 0; k < Q; ++k) sum += s_hot[k * kHotSlots + tid];
            if (sum) atomicAdd(hot_tab + kHotTotal + tid, sum);
        }
    }
    __syncthreads();
    const int b = s_item[0];
    if (b < 0) return;  // an idle slot (uniform over the block)
    struct {
        int t0, t1;
    } const it{s_item[1], s_item[2]};
    // The heavy hitters the partition peeled from this item's tiles, where they fall in this
    // bucket: every tile's {key, count} is added by the one item of its key's bucket whose
    // tile range holds the tile.
    // (calls with a hot-key table peel nothing)
    for (int tt = it.t0 + tid; hot_tab == nullptr && tt < it.t1; tt += kP2Threads) {
        const uint32_t *pw = offs + (size_t)tt * (nb + 1 + kPeelWords) + nb + 1;
        const uint32_t k1 = pw[0], n1 = pw[1];
        if (k1 != kNoKey && (int)(k1 >> kHB) == b && n1) atomicAdd(&h[k1 & (kBucketBins - 1)], n1);
    }
    uint32_t hot = kTrash + 1, hot2 = kTrash + 2;  // no hot keys yet (never equal, never a key)
    uint32_t hc = 0, hc2 = 0;
    auto flush_hot2 = [&]() {
        const uint32_t tot_hot = wave_sum_u32(hc2);
        if (lane == 0 && tot_hot) atomicAdd(&h[hot2], tot_hot);
        hc2 = 0;
    };
    auto flush_hot = [&]() {
        const uint32_t tot_hot = wave_sum_u32(hc);
        if (lane == 0 && tot_hot) atomicAdd(&h[hot], tot_hot);
        hc = 0;
    };
    // Each wave walks the tiles t0 + wave, t0 + wave + 16, ...: lane i fetches the bounds of
    // the bucket's run in 64 of them, and the wave counts the concatenation of those runs as
    // a stream of 16-byte vectors (8 keys), vector G + lane on lane `lane`, so every lane has
    // a vector whatever the run lengths. A run's vectors start at the exclusive prefix of the
    // vector counts; the runs holding vectors [G, G + 64) form a short window found with two
    // ballots, and a uniform walk over it gives each lane its run. The next 128 vectors are
    // loaded while the current 128 are counted. Every load is issued unconditionally (past
    // the stream a lane re-reads the last vector and counts nothing): a load under a branch
    // makes the compiler wait for every load in flight where the branches join.
    for (int tb = it.t0 + wave; tb < it.t1; tb += kP2Waves * kWave) {
        const int tl = tb + lane * kP2Waves;
        const bool tok = tl < it.t1;
        const uint32_t *o = offs + (size_t)(tok ? tl : it.t1 - 1) * (nb + 1 + kPeelWords) + b;
        const uint32_t rs0 = o[0], re0 = o[1];
        const uint32_t rs = tok ? rs0 : 0u, re = tok ? re0 : 0u;
        const uint32_t nvec = re > rs ? ((re + 7) >> 3) - (rs >> 3) : 0u;
        const uint32_t incl = wave_incl_scan_u32(nvec);
        const uint32_t excl = incl - nvec;
        const uint32_t T = (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
        if (T == 0) continue;
        // vector G + lane of the stream: q, the key index of its first element in its tile (e8;
        // past the stream: the run's end, so nothing is counted) and its run's bounds
        auto fetch = [&](uint32_t G, uint4 &q, uint32_t &e8, uint32_t &s0, uint32_t &e0) {
            const uint32_t g = G + (uint32_t)lane;
            const uint32_t gc = min(g, T - 1);
            const uint32_t Gq = min(G, T - 1), Gz = min(G + (uint32_t)kWave - 1, T - 1);
            const int jlo = __builtin_ctzll(__ballot(incl > Gq));
            const int jhi = __builtin_ctzll(__ballot(incl > Gz));
            int jj = jlo;
            uint32_t ex = 0, ss = 0, ee = 0;
            for (int jr = jlo; jr <= jhi; ++jr) {
                const uint32_t exj = (uint32_t)__builtin_amdgcn_readlane((int)excl, jr);
                const uint32_t rsj = (uint32_t)__builtin_amdgcn_readlane((int)rs, jr);
                const uint32_t rej = (uint32_t)__builtin_amdgcn_readlane((int)re, jr);
                const bool in = gc >= exj;  // the last such run holds the vector (empty runs share
                jj = in ? jr : jj;          // their successor's start and lose to it)
                ex = in ? exj : ex;
                ss = in ? rsj : ss;
                ee = in ? rej : ee;
            }
            const uint32_t v = (ss >> 3) + (gc - ex);
            const uint4 *run = reinterpret_cast<const uint4 *>(part + (size_t)(tb + jj * kP2Waves) * kPartStride);
            q = load_stream(&run[v]);  // read once
            e8 = g < T ? 8 * v : ee;
            s0 = ss;
            e0 = ee;
        };
        uint4 qa, qb;
        uint32_t ea, eb, sa, sb, xa, xb;
        fetch(0, qa, ea, sa, xa);
        fetch(kWave, qb, eb, sb, xb);
        for (uint32_t G = 0; G < T; G += 2 * kWave) {
            uint4 na, nb2;
            uint32_t fa, fb, ta, tb2, ya, yb;
            fetch(G + 2 * kWave, na, fa, ta, ya);
            fetch(G + 3 * kWave, nb2, fb, tb2, yb);
            // Hot-key votes on the first key of every lane's first vector: keep the current
            // hot key while a quarter of the samples match it, else adopt the first sample if
            // a quarter of the samples match that one; the second hot key likewise among the
            // other samples, at an eighth. (The votes are wave-uniform.)
            // (skipped after a hot-key table took the popular keys out of the runs: the votes
            // then rarely adopt a key and cost 7 us of the 105 at 2^28 Zipf keys)
            const bool sv = ea - sa < xa - sa;
            const uint32_t sk = qa.x & (kBucketBins - 1);
            if (hot_tab == nullptr) {
            if (__builtin_popcountll(__ballot(sv && sk == hot)) < kWave / 4) {
                const uint64_t svm = __ballot(sv);
                if (svm) {
                    const uint32_t cand = (uint32_t)__builtin_amdgcn_readlane((int)sk, __builtin_ctzll(svm));
                    if (__builtin_popcountll(__ballot(sv && sk == cand)) >= kWave / 4) {
                        flush_hot();
                        if (cand == hot2) {
                            flush_hot2();
                            hot2 = kTrash + 2;
                        }
                        hot = cand;
                    }
                }
            }
            if (__builtin_popcountll(__ballot(sv && sk == hot2)) < kWave / 8) {
                const uint64_t svm = __ballot(sv && sk != hot);
                if (svm) {
                    const uint32_t cand = (uint32_t)__builtin_amdgcn_readlane((int)sk, __builtin_ctzll(svm));
                    if (__builtin_popcountll(__ballot(sv && sk == cand)) >= kWave / 8) {
                        flush_hot2();
                        hot2 = cand;
                    }
                }
            }
            }
            if (hot_tab == nullptr) {
                count_vec<true>(h, qa, ea, sa, xa, hot, hot2, hc, hc2, kLaneTrash + (uint32_t)lane);
                count_vec<true>(h, qb, eb, sb, xb, hot, hot2, hc, hc2, kLaneTrash + (uint32_t)lane);
            } else {
                count_vec<false>(h, qa, ea, sa, xa, hot, hot2, hc, hc2, kLaneTrash + (uint32_t)lane);
                count_vec<false>(h, qb, eb, sb, xb, hot, hot2, hc, hc2, kLaneTrash + (uint32_t)lane);
            }
            qa = na;
            qb = nb2;
            ea = fa;
            eb = fb;
            sa = ta;
            sb = tb2;
            xa = ya;
            xb = yb;
        }
    }
    if (hot < kTrash) flush_hot();
    if (hot2 < kTrash) flush_hot2();
    __syncthreads();
    uint4 *dst = reinterpret_cast<uint4 *>(partials + (size_t)slot * kBucketBins);
    for (int i = tid; i < (int)(kBucketBins / 4); i += kP2Threads) dst[i] = h4[i];
}

// ---------------------------------------------------------------------------------------
// 4. merge
// ---------------------------------------------------------------------------------------
__device__ void merge_unit(int u, const uint32_t *__restrict__ partials, const HistBucket *__restrict__ buckets,
                           uint32_t num_bins, uint32_t *__restrict__ counts, bool counts16,
                           const uint32_t *__restrict__ hot) {
    const int b = u / kMergeUnitsPerBucket;
    const int blk = u % kMergeUnitsPerBucket;
    const HistBucket bk = buckets[b];
    const uint32_t bin0 = (uint32_t)b * kBucketBins + (uint32_t)blk * kMergeBins;
    for (int v = (int)threadIdx.x; v < kMergeBins / 4; v += kMergeThreads) {
        uint4 acc = make_uint4(0, 0, 0, 0);
        const uint4 *col = reinterpret_cast<const uint4 *>(partials + (size_t)bk.first * kBucketBins +
                                                           (size_t)blk * kMergeBins) + v;
        // eight partials in flight per thread: the pass is bound by load latency otherwise
#pragma unroll 8
        for (int i = 0; i < bk.count; ++i) {
            const uint4 p = col[(size_t)i * (kBucketBins / 4)];
            acc.x += p.x;
            acc.y += p.y;
            acc.z += p.z;
            acc.w += p.w;
        }
        const uint32_t k = bin0 + 4u * (uint32_t)v;
        if (hot != nullptr) {
            // the hot-table keys among bins [k, k + 4): the bucket's keys are sorted ascending
            const uint32_t lo = hot[kHotFirst + b], hi = hot[kHotFirst + b + 1];
            for (uint32_t j = lo; j < hi; ++j) {
                const uint32_t key = hot[kHotSorted + j];
                if (key >= k + 4) break;
                if (key >= k) {
                    const uint32_t c = hot[kHotTotal + j];
                    acc.x += key == k ? c : 0u;
                    acc.y += key == k + 1 ? c : 0u;
                    acc.z += key == k + 2 ? c : 0u;
                    acc.w += key == k + 3 ? c : 0u;
                }
            }
        }
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
hist_merge_kernel(const uint32_t *__restrict__ partials, const HistBucket *__restrict__ buckets, int nb,
                  uint32_t num_bins, uint32_t *__restrict__ counts, bool counts16, uint32_t *__restrict__ tot,
                  const uint32_t *__restrict__ hot) {
    const int g = (int)blockIdx.x;
    if (g == 0)
        for (int i = (int)threadIdx.x; i < kNumXcd * nb; i += kMergeThreads) tot[i] = 0;
    // Units over the whole grid in every mode: merging each bucket on the XCD that counted it
    // (its partials in that XCD's L2) measured slower (aware 11.1-11.7 us against 9.5 us),
    // since an XCD whose range is one hot bucket has few units for its 128 workgroups.
    for (int u = g; u < nb * kMergeUnitsPerBucket; u += (int)gridDim.x)
        merge_unit(u, partials, buckets, num_bins, counts, counts16, hot);
}

}  // namespace xd

using namespace xd;

extern "C" {

size_t xd_hist_workspace_size(size_t n, uint32_t num_bins) {
    if (num_bins == 0 || num_bins > (1u << 24)) return 0;
    return hist_layout(n, num_bins).total;
}

int xd_hist_u32(const uint32_t *keys, size_t n, uint32_t *counts, uint32_t num_bins, int mode,
                const uint8_t *home_attr, void *workspace, size_t workspace_bytes, void *stream) {
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
    const XcdHint xh = xcd_hint(s);
    char *ws = static_cast<char *>(workspace);
    uint16_t *part = reinterpret_cast<uint16_t *>(ws + L.part);
    uint32_t *offs = reinterpret_cast<uint32_t *>(ws + L.offs);
    uint32_t *tot = reinterpret_cast<uint32_t *>(ws + L.tot);
    HistBucket *buckets = reinterpret_cast<HistBucket *>(ws + L.buckets);
    uint32_t *partials = reinterpret_cast<uint32_t *>(ws + L.partials);
    const unsigned rot = mode == XD_MODE_ROTATED ? next_rotation(1) % kNumXcd : 0u;
    const unsigned rot_eff = (mode == XD_MODE_ROTATED && rot == 0) ? 1u : rot;  // never the identity

    // Plan every partition launch before enqueuing any, so that a shape the workspace cannot
    // hold is refused with nothing written. XCD-aware and rotated calls read the 16 KiB pairs
    // inside the keys as routed tiles (each group of up to kRouteGroupPairs pairs gives one
    // tile per I/O die); the keys before the first and after the last pair, and oblivious
    // calls, go in contiguous tiles (one workgroup per tile).
    const bool pack = L.nb <= kPackBuckets;
    struct PartLaunch {
        int kind;     // kPartFull / kPartRange / kPartRouted
        PartSrc ps;
        unsigned grid;
    };
    PartLaunch plan[5];
    int nplan = 0, ntl = 0;
    const HomeMap home{home_attr, reinterpret_cast<uint64_t>(keys) / kHomePage, home_mask()};
    auto contiguous = [&](size_t r0, size_t r1) {  // tiles of keys [r0, r1)
        // vector tiles over the whole 16-byte vectors, then the last (r1 - r0) % 4 keys
        const size_t vend = aligned16(keys + r0) ? r0 + (r1 - r0) / 4 * 4 : r0;
        if (vend > r0) {
            const size_t nt = (vend - r0 + kTileKeys - 1) / kTileKeys;
            plan[nplan++] = PartLaunch{kPartFull, PartSrc{keys, r0, vend, ntl, 0, 0, 0, 0, home, XcdHint{0u, nullptr}}, (unsigned)nt};
            ntl += (int)nt;
        }
        if (vend < r1) {
            const size_t nt = (r1 - vend + kTileKeys - 1) / kTileKeys;
            plan[nplan++] = PartLaunch{kPartRange, PartSrc{keys, vend, r1, ntl, 0, 0, 0, 0, home, XcdHint{0u, nullptr}}, (unsigned)nt};
            ntl += (int)nt;
        }
    };
    if (n > 0) {
        const uint64_t A = reinterpret_cast<uint64_t>(keys);
        const uint64_t pfirst = (A + 16383) / 16384, pend = (A + 4 * (uint64_t)n) / 16384;
        // (the routed kind reads 16-byte vectors counted from key 0: keys must be 16-byte aligned)
        const uint64_t npairs = (mode != XD_MODE_OBLIVIOUS && aligned16(keys) && pend > pfirst) ? pend - pfirst : 0;
        if (npairs == 0) {
            contiguous(0, n);
        } else {
            const uint64_t groups = (npairs + kRouteGroupPairs - 1) / kRouteGroupPairs;
            const size_t head = (size_t)(pfirst * 16384 - A) / 4;
            const size_t tail0 = head + (size_t)npairs * 4096;
            const unsigned grid = (unsigned)((groups + kNumXcd / 2 - 1) / (kNumXcd / 2) * kNumXcd);
            plan[nplan++] = PartLaunch{kPartRouted, PartSrc{keys, 0, 0, 0, (int)groups, pfirst, npairs, mode, home, xh}, grid};
            ntl = 2 * (int)groups;
            if (head > 0) contiguous(0, head);
            if (tail0 < n) contiguous(tail0, n);
        }
    }
    if (ntl > L.ntiles) return fail(XD_ERR_WORKSPACE, "xd_hist_u32: tile count exceeds the workspace layout");

    // From the first launch on, an error return leaves the workspace's bucket totals
    // non-zero: the caller must zero-fill the workspace again before its next use.
    // Hot-key table: for calls of at least kHotMinKeys keys into at most kPackBuckets buckets
    // (the packed partition: the unpacked one has no registers left for the lookups).
    uint32_t *hot = nullptr;
    uint16_t *hot_part = reinterpret_cast<uint16_t *>(ws + L.hot_part);
    if (n >= kHotMinKeys && pack) {
        hot = reinterpret_cast<uint32_t *>(ws + L.hot);
        launch("hist_hot_kernel", hist_hot_kernel, dim3(1), dim3(1024), 0, s, keys, n, num_bins, L.nb, hot,
               reinterpret_cast<uint32_t *>(ws + L.ones));
        if (int rc = launch_status("hist_hot_kernel")) return rc;
    }
    using PartKernel = void (*)(PartSrc, uint32_t, int, uint16_t *, uint32_t *, uint32_t *, const uint32_t *, uint16_t *);
    using LeanKernel =
        void (*)(PartSrc, uint32_t, int, uint16_t *, uint32_t *, uint32_t *, const uint32_t *, uint16_t *, const uint32_t *);
    for (int k = 0; k < nplan; ++k) {
        const PartLaunch &pl = plan[k];
        if (hot != nullptr && pl.kind != kPartRange) {
            // the lean kinds: a hot-key table and at most kPackBuckets buckets
            const LeanKernel lk =
                pl.kind == kPartRouted ? hist_partition_lean_kernel<kPartRouted> : hist_partition_lean_kernel<kPartFull>;
            launch("hist_partition_kernel", lk, dim3(pl.grid), dim3(kP1Threads), 0, s, pl.ps, (uint32_t)L.nb << kHB,
                   L.nb, part, offs, tot, (const uint32_t *)hot, hot_part, (const uint32_t *)(ws + L.ones));
            if (int rc = launch_status("hist_partition_kernel")) return rc;
            continue;
        }
        PartKernel kern;
        if (pl.kind == kPartRouted)
            kern = pack ? hist_partition_packed_kernel<kPartRouted> : hist_partition_kernel<kPartRouted>;
        else if (pl.kind == kPartFull)
            kern = pack ? hist_partition_packed_kernel<kPartFull> : hist_partition_kernel<kPartFull>;
        else
            kern = hist_partition_kernel<kPartRange>;
        launch("hist_partition_kernel", kern, dim3(pl.grid), dim3(kP1Threads), 0, s, pl.ps, num_bins, L.nb, part, offs,
               tot, hot, hot_part);
        if (int rc = launch_status("hist_partition_kernel")) return rc;
    }
    launch("hist_count_kernel", hist_count_kernel, dim3(L.nitems), dim3(kP2Threads), 0, s, part, offs, L.nb, ntl, tot,
           L.per_xcd, partials, buckets, mode, rot_eff, hot, hot_part, xh);
    if (int rc = launch_status("hist_count_kernel")) return rc;
    // one workgroup per merge unit, up to 4096
    const int merge_grid = std::min(std::max(L.nb * kMergeUnitsPerBucket, kNumXcd * 64), 4096);
    launch("hist_merge_kernel", hist_merge_kernel, dim3(merge_grid), dim3(kMergeThreads), 0, s, partials, buckets, L.nb,
           num_bins, counts, aligned16(counts), tot, (const uint32_t *)hot);
    return launch_status("hist_merge_kernel");
}

}  // extern "C"
