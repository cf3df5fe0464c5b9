// Bulk build of the u64 open-addressing table: the table's previous contents are replaced by
// n (key, value) pairs, with every slot written once by a plain store and no atomic on the
// table except for a few spilled pairs.
//
// Reference: applications/hash/src/hash_probe_dep.cu builds its table on the CPU (226-241),
// inserting the keys one after another with linear probing; probe_chain_one (46-64) is the
// lookup the table must answer. The GPU insert (xd_hash_insert_u64) claims each slot with a
// compare-and-swap that gfx950 executes at the memory side, about 16 G claims/s on a 2 GiB
// table whichever die issues them. A table built from scratch needs no claims in memory:
//   0. clear: zero the partition cursors;
//   1. split A: each workgroup reads a tile of 4096 pairs, splits it in LDS by the high
//      digit of the pair's range (a range = 4096 slots = 64 KiB) and appends each digit's
//      run to that digit's region for its XCD slot (one memory-side add per run on the
//      region's cursor; runs of one region come from one XCD, whose L2 joins their
//      boundary lines);
//   2. split B: every region of step 1, tile by tile, split by the low digit into one region
//      per range;
//   3. build: one workgroup per range inserts the range's pairs into a 4096-slot table in
//      LDS (64-bit LDS compare-and-swap, linear probing inside runs of adjacent slots) and
//      writes the whole range with 16-byte stores, EMPTY slots included; a pair whose probe
//      reaches the end of its run is a spill;
//   4. fix-up: spills, and pairs that found their region full in steps 1-2, are inserted into
//      the built table with the compare-and-swap insert. Every slot from a spill's home to
//      the end of its run is occupied, so it lands where a serial insert could have put it;
//      lookups see the same keys and values as after the serial build.
// Ranges and placement:
//   oblivious: range r = slots [4096 r, 4096 r + 4096) (one run), workgroup r builds it;
//   aware:     range 2 rho + d = the eight 8 KiB chunks homed on I/O die d among the sixteen
//              chunks of 128 KiB region rho (each 16 KiB pair of chunks has one chunk on each
//              die); runs are the 512-slot chunks; a workgroup on die d builds it, so the
//              2 GiB of table stores are near;
//   rotated:   the same ranges built on the other die.
#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>

#include "xd_hash.hpp"

namespace xd {

constexpr int kLgRange = 12;
constexpr uint32_t kRange = 1u << kLgRange;  // slots per range: 64 KiB of LDS
constexpr uint32_t kChunkSlots = (uint32_t)(kHomeChunk / sizeof(Slot));  // 512
constexpr int kSplitThreads = 1024;
constexpr int kSplitPer = 4;  // pairs per thread
constexpr uint32_t kSplitTile = kSplitThreads * kSplitPer;
constexpr int kMaxDigitBits = 9;
constexpr int kBuildThreads = 1024;  // 2 workgroups per CU (LDS-bound); build kernel 721 us at 512 threads, 612 here
constexpr int kBuildPer = kRange / kBuildThreads;  // slots written per thread
constexpr int kBuildLoad = 4;                       // pairs in flight per thread
constexpr uint32_t kSpillPerRange = 32;  // expected ~0.25 per run end (two per aware range)
constexpr int kMinLgSlots = 15;          // 8 ranges: one per XCD slot of a grid
constexpr int kMaxLgSlots = 30;          // two digits of at most 9 bits
constexpr uint64_t kMinPairsPerRange = 64;  // fewer pairs per range (load factor < 1/64): clear + insert
constexpr int kBuildLdsPages = 4096;     // tables up to 8 GiB stage their page map in LDS
constexpr int kFixThreads = 256;
static_assert(kChunkSlots * 8 == kRange, "an aware range is one chunk of each of 8 pairs");
static_assert((1 << kMaxDigitBits) <= kSplitThreads, "one digit counter per split thread");

struct BuildGeom {
    uint64_t mask;  // slots - 1
    uint64_t base;  // table address
    int die;        // 1: ranges are die halves of 128 KiB regions (home modes, aligned table)
    HomeMap home;
};

// Range of home slot h (the die bit is the range's lowest bit in die mode).
__device__ __forceinline__ uint32_t range_of(const BuildGeom &g, const StagedHome &sh, uint64_t h) {
    if (!g.die) return (uint32_t)(h >> kLgRange);
    return (uint32_t)((h >> (kLgRange + 1)) << 1) | sh(g.base + h * sizeof(Slot));
}

// Position of home slot h in its range's LDS table.
__device__ __forceinline__ uint32_t local_of(const BuildGeom &g, uint64_t h) {
    if (!g.die) return (uint32_t)(h & (kRange - 1));
    return (uint32_t)(((h >> 10) & 7u) << 9) | (uint32_t)(h & (kChunkSlots - 1));
}

struct SplitSrc {
    // split A: the caller's arrays
    const uint64_t *keys, *vals;
    uint64_t n;
    int vec;  // keys and vals 16-byte aligned
    // split B: the regions of split A
    const Slot *reg;
    const uint32_t *cur;
    uint64_t cap;
    uint32_t tpr;  // tiles per region
};

struct SplitDst {
    Slot *out;
    uint32_t *cur;
    uint64_t cap;
    Slot *ovf;
    uint32_t *ovf_cnt;
    uint64_t ovf_cap;
};

__device__ __forceinline__ Slot load_pair_nt(const Slot *p) {
    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return Slot{(uint64_t)t.x | ((uint64_t)t.y << 32), (uint64_t)t.z | ((uint64_t)t.w << 32)};
}

__device__ __forceinline__ void store_pair(Slot *p, const Slot &s) {
    *reinterpret_cast<uint4 *>(p) = make_uint4((uint32_t)s.key, (uint32_t)(s.key >> 32), (uint32_t)s.val,
                                               (uint32_t)(s.val >> 32));
}

// The table is written once here and read back only by later lookups: non-temporal stores
// (build kernel 612 -> 589 us at 2^27 slots). The split regions, which the next pass reads,
// keep ordinary stores (non-temporal ones made each split pass 100 us slower).
__device__ __forceinline__ void store_pair_nt(Slot *p, const Slot &s) {
    const u32x4 v = {(uint32_t)s.key, (uint32_t)(s.key >> 32), (uint32_t)s.val, (uint32_t)(s.val >> 32)};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(p));
}

__device__ __forceinline__ void to_overflow(const SplitDst &d, const Slot &s) {
    const uint32_t k = atomicAdd(d.ovf_cnt, 1u);
    if (k < d.ovf_cap) store_pair(&d.ovf[k], s);
}

// Exclusive scan of one value per thread over a kSplitThreads block; *total = the sum.
__device__ __forceinline__ uint32_t split_scan(uint32_t v, uint32_t *wsum, uint32_t *total) {
    constexpr int W = kSplitThreads / kWave;
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
    return wsum[wave] + incl - v;
}

// Split pass. FROM_REGIONS = false (split A): tile g of the caller's pairs, digit = the
// range's high bits (range >> shift), output region digit * 8 + (g mod 8). true (split B):
// tile g % tpr of region g / tpr of split A, digit = the range's low `nbits` bits, output
// region = the range.
template <bool FROM_REGIONS>
__global__ void __launch_bounds__(kSplitThreads)
hb_split_kernel(SplitSrc src, BuildGeom g, int shift, int nbits, SplitDst dst) {
    __shared__ __attribute__((aligned(16))) Slot stage[kSplitTile];
    __shared__ uint32_t cnt[1 << kMaxDigitBits];
    __shared__ uint32_t off[1 << kMaxDigitBits];
    __shared__ uint32_t gbase[1 << kMaxDigitBits];
    __shared__ uint32_t wsum[kSplitThreads / kWave];
    __shared__ uint32_t s_total;
    __shared__ uint8_t lattr[kBuildLdsPages];
    const int tid = (int)threadIdx.x;
    const uint32_t nd = 1u << nbits;
    uint64_t t0 = 0, avail = 0;
    uint32_t reg = 0;
    if (FROM_REGIONS) {
        reg = blockIdx.x / src.tpr;
        t0 = (uint64_t)(blockIdx.x % src.tpr) * kSplitTile;
        const uint64_t c = min((uint64_t)src.cur[reg], src.cap);
        if (t0 >= c) return;  // uniform over the block, before any barrier
        avail = c - t0;
    }
    for (uint32_t i = (uint32_t)tid; i < nd; i += kSplitThreads) cnt[i] = 0;
    const StagedHome sh = stage_home_nosync(g.home, g.base, (g.mask + 1) * sizeof(Slot), lattr, kBuildLdsPages, g.die);

    // Pair c of this thread: split A, lane-contiguous 16-byte vectors (pairs 2 tid + {0, 1} of
    // each half tile); split B, pair tid + c * kSplitThreads of the tile.
    Slot r[kSplitPer];
    bool ok[kSplitPer];
    if (!FROM_REGIONS) {
        const uint64_t tile0 = (uint64_t)blockIdx.x * kSplitTile;
#pragma unroll
        for (int h = 0; h < kSplitPer / 2; ++h) {
            const uint64_t i = tile0 + (uint64_t)h * (2 * kSplitThreads) + 2u * (uint64_t)tid;
            ok[2 * h] = i < src.n;
            ok[2 * h + 1] = i + 1 < src.n;
            if (src.vec && i + 2 <= src.n) {
                const u32x4 k = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src.keys + i));
                const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src.vals + i));
                r[2 * h] = Slot{(uint64_t)k.x | ((uint64_t)k.y << 32), (uint64_t)v.x | ((uint64_t)v.y << 32)};
                r[2 * h + 1] = Slot{(uint64_t)k.z | ((uint64_t)k.w << 32), (uint64_t)v.z | ((uint64_t)v.w << 32)};
            } else {
                r[2 * h] = ok[2 * h] ? Slot{src.keys[i], src.vals[i]} : Slot{kEmpty, 0};
                r[2 * h + 1] = ok[2 * h + 1] ? Slot{src.keys[i + 1], src.vals[i + 1]} : Slot{kEmpty, 0};
            }
        }
    } else {
        const Slot *in = src.reg + (uint64_t)reg * src.cap + t0;
#pragma unroll
        for (int c = 0; c < kSplitPer; ++c) {
            const uint64_t i = (uint64_t)tid + (uint64_t)c * kSplitThreads;
            ok[c] = i < avail;
            r[c] = load_pair_nt(&in[ok[c] ? i : 0]);
        }
    }
    uint32_t dig[kSplitPer];
    __syncthreads();  // counters cleared, page map staged
#pragma unroll
    for (int c = 0; c < kSplitPer; ++c) {
        dig[c] = nd;  // not counted: past the input or an EMPTY key (never stored)
        if (ok[c] && r[c].key != kEmpty)
            dig[c] = (range_of(g, sh, mix64(r[c].key) & g.mask) >> shift) & (nd - 1u);
    }
    uint32_t rank[kSplitPer];
#pragma unroll
    for (int c = 0; c < kSplitPer; ++c) rank[c] = dig[c] < nd ? atomicAdd(&cnt[dig[c]], 1u) : 0u;
    __syncthreads();
    const uint32_t v = (uint32_t)tid < nd ? cnt[tid] : 0u;
    const uint32_t e = split_scan(v, wsum, &s_total);
    // output region of digit d: split A, per digit and XCD slot; split B, the range
    const uint32_t xs = blockIdx.x % kNumXcd;
    auto region_of = [&](uint32_t d) -> uint64_t {
        return FROM_REGIONS ? (((uint64_t)(reg / kNumXcd) << nbits) | d) : ((uint64_t)d * kNumXcd + xs);
    };
    if ((uint32_t)tid < nd) {
        off[tid] = e;
        if (v > 0) gbase[tid] = atomicAdd(&dst.cur[region_of((uint32_t)tid)], v);
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kSplitPer; ++c)
        if (dig[c] < nd) stage[off[dig[c]] + rank[c]] = r[c];
    __syncthreads();
    const uint32_t total = s_total;
    for (uint32_t i = (uint32_t)tid; i < total; i += kSplitThreads) {
        const Slot s = stage[i];
        const uint32_t d = (range_of(g, sh, mix64(s.key) & g.mask) >> shift) & (nd - 1u);
        const uint64_t pos = (uint64_t)gbase[d] + (i - off[d]);
        if (pos < dst.cap)
            store_pair(&dst.out[region_of(d) * dst.cap + pos], s);
        else
            to_overflow(dst, s);
    }
}

// Build pass: one workgroup per range (see the file comment for the placement).
__global__ void __launch_bounds__(kBuildThreads)
hb_build_kernel(BuildGeom g, int mode, const Slot *__restrict__ reg, const uint32_t *__restrict__ cur, uint64_t cap,
                Slot *__restrict__ table, Slot *__restrict__ spill, uint32_t *__restrict__ spill_cnt, SplitDst ovf,
                XcdHint xh) {
    __shared__ __attribute__((aligned(16))) Slot tab[kRange];
    report_xcd(xh);
    __shared__ uint32_t s_nsp;
    __shared__ uint8_t lattr[kBuildLdsPages];
    const int tid = (int)threadIdx.x;
    const int b = (int)blockIdx.x;
    uint32_t r;
    if (!g.die) {
        r = (uint32_t)b;
    } else {
        const uint32_t die = wg_die(b, xh);
        const uint32_t want = mode == XD_MODE_AWARE ? die : (die ^ 1u);
        const uint32_t rank = (uint32_t)die_rank(b, xh);
        r = 2u * rank + want;
    }
    for (uint32_t j = (uint32_t)tid; j < kRange; j += kBuildThreads) tab[j] = Slot{kEmpty, 0};
    if (tid == 0) s_nsp = 0;
    const StagedHome sh = stage_home_nosync(g.home, g.base, (g.mask + 1) * sizeof(Slot), lattr, kBuildLdsPages, g.die);
    const uint64_t count = min((uint64_t)cur[r], cap);
    const Slot *in = reg + (uint64_t)r * cap;
    __syncthreads();

    for (uint64_t p0 = 0; p0 < count; p0 += (uint64_t)kBuildLoad * kBuildThreads) {
        Slot q[kBuildLoad];
#pragma unroll
        for (int k = 0; k < kBuildLoad; ++k) {
            const uint64_t i = p0 + (uint64_t)tid + (uint64_t)k * kBuildThreads;
            q[k] = load_pair_nt(&in[i < count ? i : 0]);
        }
#pragma unroll
        for (int k = 0; k < kBuildLoad; ++k) {
            const uint64_t i = p0 + (uint64_t)tid + (uint64_t)k * kBuildThreads;
            if (i >= count) continue;
            const uint64_t key = q[k].key;
            uint32_t loc = local_of(g, mix64(key) & g.mask);
            const uint32_t end = g.die ? ((loc | (kChunkSlots - 1)) + 1) : kRange;
            for (;;) {
                if (loc == end) {  // the run is full from the home slot on: a spill
                    const uint32_t j = atomicAdd(&s_nsp, 1u);
                    if (j < kSpillPerRange)
                        store_pair(&spill[(uint64_t)r * kSpillPerRange + j], q[k]);
                    else
                        to_overflow(ovf, q[k]);
                    break;
                }
                const uint64_t old = atomicCAS(reinterpret_cast<unsigned long long *>(&tab[loc].key),
                                               (unsigned long long)kEmpty, (unsigned long long)key);
                if (old == kEmpty || old == key) {
                    tab[loc].val = q[k].val;
                    break;
                }
                ++loc;
            }
        }
    }
    __syncthreads();
    // Write-out: pass k stores local slots kBuildThreads k .. kBuildThreads (k + 1) - 1, whole 8 KiB chunks.
#pragma unroll
    for (int k = 0; k < kBuildPer; ++k) {
        const uint32_t j = (uint32_t)tid + (uint32_t)k * kBuildThreads;
        uint64_t slot;
        if (!g.die) {
            slot = (uint64_t)r * kRange + j;
        } else {
            const uint64_t even = (uint64_t)(r >> 1) * (2 * kRange) + (uint64_t)(j >> 9) * (2 * kChunkSlots);
            const uint32_t he = sh(g.base + even * sizeof(Slot));
            slot = even + (he == (r & 1u) ? 0 : kChunkSlots) + (j & (kChunkSlots - 1));
        }
        store_pair_nt(&table[slot], tab[j]);
    }
    if (tid == 0) spill_cnt[r] = s_nsp;
}

// Fix-up: items [0, nr * kSpillPerRange) are the ranges' spill slots (item i valid when
// i mod kSpillPerRange < the range's spill count), items beyond are the overflow list.
__global__ void __launch_bounds__(kFixThreads)
hb_fixup_kernel(Slot *table, uint64_t mask, uint32_t nr, const Slot *__restrict__ spill,
                const uint32_t *__restrict__ spill_cnt, const Slot *__restrict__ ovf, const uint32_t *__restrict__ ovf_cnt,
                uint64_t ovf_cap, uint64_t max_probe, unsigned long long *failed) {
    const uint64_t nsp = (uint64_t)nr * kSpillPerRange;
    const uint64_t items = nsp + min((uint64_t)*ovf_cnt, ovf_cap);
    const uint64_t stride = (uint64_t)gridDim.x * kFixThreads;
    for (uint64_t i = (uint64_t)blockIdx.x * kFixThreads + threadIdx.x; i < items; i += stride) {
        Slot s;
        if (i < nsp) {
            const uint32_t rr = (uint32_t)(i / kSpillPerRange);
            if ((uint32_t)(i % kSpillPerRange) >= spill_cnt[rr]) continue;
            s = spill[i];
        } else {
            s = ovf[i - nsp];
        }
        if (!slot_insert(table, mask, mix64(s.key) & mask, s.key, s.val, max_probe) && failed) atomicAdd(failed, 1ull);
    }
}

__global__ void __launch_bounds__(256) hb_clear_kernel(uint32_t *w, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) w[i] = 0;
}

// ---------------------------------------------------------------------------------------
// Workspace layout
// ---------------------------------------------------------------------------------------
struct BuildLayout {
    bool bulk;        // false: the shape is built by clearing and the compare-and-swap insert
    int dA, dB;       // digit bits of split A and split B
    uint32_t nr, na;  // ranges; regions of split A (2^dA digits x 8 XCD slots)
    uint64_t capA, capB, tprA;
    size_t curA, curB, ovf_cnt, spill_cnt, regA, regB, spill, ovf, total;
};

static uint64_t region_cap(uint64_t n, uint64_t regions) {
    const double mean = (double)((n + regions - 1) / regions);
    // mean + 1/32 + six standard deviations of a binomial count: a region overflows only for
    // skewed input, and its excess then takes the fix-up path
    const uint64_t c = (uint64_t)(mean + mean / 32.0 + 6.0 * sqrt(mean) + 64.0);
    return (c + 3) & ~(uint64_t)3;
}

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

static BuildLayout build_layout(uint64_t n, uint64_t slots) {
    BuildLayout L{};
    int lg = 0;
    while ((1ull << lg) < slots) ++lg;
    L.bulk = n > 0 && n < (1ull << 32) && lg >= kMinLgSlots && lg <= kMaxLgSlots && (1ull << lg) == slots;
    // at least kMinPairsPerRange pairs per range on average: below that the regions' floor
    // (64 + 1/32 + six deviations each) would size the workspace instead of n, and clearing
    // plus inserting so few keys costs no more than the build's whole-table stores
    L.bulk = L.bulk && n >= (uint64_t)kMinPairsPerRange << (lg - kLgRange);
    if (!L.bulk) return L;
    const int nrb = lg - kLgRange;
    L.dB = nrb / 2;
    L.dA = nrb - L.dB;
    L.nr = 1u << nrb;
    L.na = (1u << L.dA) * kNumXcd;
    L.capA = region_cap(n, L.na);
    L.capB = region_cap(n, L.nr);
    L.tprA = (L.capA + kSplitTile - 1) / kSplitTile;
    size_t o = 0;
    L.curA = o;  // the three counter blocks are cleared together
    o += (size_t)L.na * 4;
    L.curB = o;
    o += (size_t)L.nr * 4;
    L.ovf_cnt = o;
    o = al256(o + 4);
    L.spill_cnt = o;
    o = al256(o + (size_t)L.nr * 4);
    L.regA = o;
    o = al256(o + (size_t)L.na * L.capA * sizeof(Slot));
    L.regB = o;
    o = al256(o + (size_t)L.nr * L.capB * sizeof(Slot));
    L.spill = o;
    o = al256(o + (size_t)L.nr * kSpillPerRange * sizeof(Slot));
    L.ovf = o;
    o = al256(o + (size_t)n * sizeof(Slot));
    L.total = o;
    return L;
}

}  // namespace xd

using namespace xd;

extern "C" {

size_t xd_hash_build_workspace_size(uint64_t n, uint64_t slots) { return build_layout(n, slots).total; }

int xd_hash_build_u64(void *table, uint64_t slots, const uint64_t *keys, const uint64_t *vals, uint64_t n, int mode,
                      const uint8_t *home_attr, void *workspace, size_t workspace_bytes, unsigned long long *failed,
                      void *stream) {
    XD_REQUIRE(table != nullptr && aligned16(table), "xd_hash_build_u64: table must be non-NULL and 16-byte aligned");
    XD_REQUIRE(slots >= 1 && (slots & (slots - 1)) == 0, "xd_hash_build_u64: slots must be a power of two");
    XD_REQUIRE(n == 0 || (keys != nullptr && vals != nullptr), "xd_hash_build_u64: NULL keys/vals");
    XD_REQUIRE(n < (1ull << 32), "xd_hash_build_u64: n must be < 2^32 per call");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "xd_hash_build_u64: bad mode");
    XD_REQUIRE((reinterpret_cast<uintptr_t>(keys) & 7u) == 0 && (reinterpret_cast<uintptr_t>(vals) & 7u) == 0,
               "xd_hash_build_u64: keys and vals must be 8-byte aligned");
    const BuildLayout L = build_layout(n, slots);
    if (!L.bulk) {  // no pairs, or a table outside [2^15, 2^30] slots
        if (int rc = xd_hash_init(table, slots, stream)) return rc;
        return xd_hash_insert_u64(table, slots, keys, vals, n, mode, home_attr, failed, stream);
    }
    if (workspace == nullptr || workspace_bytes < L.total || !aligned16(workspace))
        return fail(XD_ERR_WORKSPACE,
                    "xd_hash_build_u64: workspace missing, misaligned or smaller than xd_hash_build_workspace_size()");
    hipStream_t s = (hipStream_t)stream;
    char *ws = static_cast<char *>(workspace);
    uint32_t *curA = reinterpret_cast<uint32_t *>(ws + L.curA);
    uint32_t *curB = reinterpret_cast<uint32_t *>(ws + L.curB);
    uint32_t *ovf_cnt = reinterpret_cast<uint32_t *>(ws + L.ovf_cnt);
    uint32_t *spill_cnt = reinterpret_cast<uint32_t *>(ws + L.spill_cnt);
    Slot *regA = reinterpret_cast<Slot *>(ws + L.regA);
    Slot *regB = reinterpret_cast<Slot *>(ws + L.regB);
    Slot *spill = reinterpret_cast<Slot *>(ws + L.spill);
    Slot *ovf = reinterpret_cast<Slot *>(ws + L.ovf);
    const uint64_t base = reinterpret_cast<uint64_t>(table);
    BuildGeom g;
    g.mask = slots - 1;
    g.base = base;
    // Die ranges need whole 16 KiB pairs of chunks at every 128 KiB region, and one chunk of
    // each pair on either die: true with a page map (the home flips with bit 13 inside a page)
    // and with an address mask that holds bit 13. Under another mask both chunks of a pair
    // can share a die, and the two would be built into one LDS run, so such calls take the
    // contiguous ranges.
    const bool pairs_split = home_attr != nullptr || (home_mask() & kHomeChunk) != 0;
    g.die = (mode != XD_MODE_OBLIVIOUS && base % (2 * kHomeChunk) == 0 && pairs_split) ? 1 : 0;
    g.home = HomeMap{home_attr, base / kHomePage, home_mask()};

    const uint64_t nclear = (uint64_t)L.na + L.nr + 1;
    launch("hb_clear_kernel", hb_clear_kernel, dim3((unsigned)std::min<uint64_t>((nclear + 255) / 256, 1024)),
           dim3(256), 0, s, curA, nclear);
    if (int rc = launch_status("hb_clear_kernel")) return rc;

    const SplitDst dA{regA, curA, L.capA, ovf, ovf_cnt, n};
    SplitSrc in{};
    in.keys = keys;
    in.vals = vals;
    in.n = n;
    in.vec = aligned16(keys) && aligned16(vals);
    launch("hb_split_kernel", hb_split_kernel<false>, dim3((unsigned)((n + kSplitTile - 1) / kSplitTile)),
           dim3(kSplitThreads), 0, s, in, g, L.dB, L.dA, dA);
    if (int rc = launch_status("hb_split_kernel")) return rc;

    const SplitDst dB{regB, curB, L.capB, ovf, ovf_cnt, n};
    SplitSrc mid{};
    mid.reg = regA;
    mid.cur = curA;
    mid.cap = L.capA;
    mid.tpr = (uint32_t)L.tprA;
    launch("hb_split_kernel", hb_split_kernel<true>, dim3((unsigned)(L.na * L.tprA)), dim3(kSplitThreads), 0, s, mid, g,
           0, L.dB, dB);
    if (int rc = launch_status("hb_split_kernel")) return rc;

    launch("hb_build_kernel", hb_build_kernel, dim3(L.nr), dim3(kBuildThreads), 0, s, g, mode,
           static_cast<const Slot *>(regB), static_cast<const uint32_t *>(curB), L.capB, static_cast<Slot *>(table), spill,
           spill_cnt, dB, xcd_hint(s));
    if (int rc = launch_status("hb_build_kernel")) return rc;

    const uint64_t max_probe = slots < kMaxProbe ? slots : kMaxProbe;
    launch("hb_fixup_kernel", hb_fixup_kernel, dim3(1024), dim3(kFixThreads), 0, s, static_cast<Slot *>(table), slots - 1,
           L.nr, static_cast<const Slot *>(spill), static_cast<const uint32_t *>(spill_cnt),
           static_cast<const Slot *>(ovf), static_cast<const uint32_t *>(ovf_cnt), (uint64_t)n, max_probe, failed);
    return launch_status("hb_fixup_kernel");
}

}  // extern "C"
