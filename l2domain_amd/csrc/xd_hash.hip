// Open-addressing linear-probe hash table of uint64 keys and uint64 values.
//
// Reference: applications/hash/src/hash_probe_dep.cu
//   Entry{int key; int next}, EMPTY_KEY = -1 (14-21); probe_chain_one (46-64): slot =
//   mix32(key) & mask, linear probing until the key or EMPTY; probe_dep_base (66-83) walks
//   queries in launch order (locality-oblivious); probe_dep_sa (85-116) takes per-side query
//   lists routed on the host (244-270) so that each SM probes slots homed on its L2 side.
//   The reference builds the table on the CPU (226-241); here insertion is on the GPU.
//
// MI355X design. A slot is 16 bytes {key, value}; EMPTY = 0xFFFF'FFFF'FFFF'FFFF; the home
// slot is mix64(key) & (slots - 1) and probing walks forward with wrap-around. Insert claims
// a slot with a 64-bit compare-and-swap on the key (executed at the memory side on gfx950)
// and then stores the value; a lookup reads one 16-byte slot per probe. Placement:
//   oblivious: keys in input order over a plain grid;
//   aware:     every workgroup reads the whole input but handles only the keys whose home
//              slot lies in memory homed on its own I/O die (the slot's address picks the
//              die, so this partitions the buckets by hash bits), so every probe is a near
//              access and no routing pass or output scatter is needed;
//   rotated:   the swapped control: each die handles the keys homed on the other die.
#include <hip/hip_runtime.h>

#include "xd_hash.hpp"

namespace xd {

constexpr int kHashThreads = 256;

__global__ void __launch_bounds__(256) hash_init_kernel(Slot *table, uint64_t slots) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < slots; i += stride)
        table[i] = Slot{kEmpty, 0};
}

// Work walk. Every wave takes 64-item chunks of the input: chunk c = first + k * stride.
// Oblivious: the chunks of the whole grid in order. Home modes: the waves of each die walk
// all chunks (each die sees every item) and keep only the items whose home slot lies on the
// wanted die; the kept items (index and key) are compacted into a per-wave LDS queue and
// probed 64 at a time, so that no lane idles through a probe loop.
struct Walk {
    uint64_t first, stride;  // in 64-item chunks
    uint32_t want;           // die whose items this wave takes (home modes)
};

__device__ __forceinline__ Walk make_walk(int mode, const XcdHint &xh) {
    report_xcd(xh);
    Walk w;
    const int b = (int)blockIdx.x;
    const int wave = (int)threadIdx.x / kWave;
    constexpr int kWavesPerWg = kHashThreads / kWave;
    if (mode == XD_MODE_OBLIVIOUS) {
        w.first = (uint64_t)b * kWavesPerWg + wave;
        w.stride = (uint64_t)gridDim.x * kWavesPerWg;
        w.want = 0;
    } else {
        const int per_die = (int)gridDim.x / 2;
        const int rank = die_rank(b, xh);
        w.first = (uint64_t)rank * kWavesPerWg + wave;
        w.stride = (uint64_t)per_die * kWavesPerWg;
        const uint32_t die = wg_die(b, xh);
        w.want = (mode == XD_MODE_AWARE) ? die : (die ^ 1u);
    }
    return w;
}

// Home of a slot address with the table's page map staged in LDS (a 2 GiB table has 1024
// pages), so the ownership test of the home modes costs no global load.
constexpr int kLdsPages = 4096;  // tables up to 8 GiB; larger ones read the map from memory

typedef StagedHome SlotHome;

// Stages the page map of [base, base + bytes) into `lds` when it fits; every thread calls it.
__device__ __forceinline__ SlotHome stage_home(const HomeMap &h, uint64_t base, uint64_t bytes, uint8_t *lds,
                                               bool filter) {
    const SlotHome sh = stage_home_nosync(h, base, bytes, lds, kLdsPages, filter);
    __syncthreads();
    return sh;
}

// Runs body(item, key) for every item this wave owns, always on a full wave except for the
// last batch. key_of(i) is read one chunk ahead; in the home modes keep(key) decides
// ownership. The kept items' indices and keys are compacted into the wave's LDS queue, so
// that body() never reads an item's key a second time.
template <typename KeyOf, typename Keep, typename Body>
__device__ __forceinline__ void for_each_owned(const Walk &w, uint64_t n, bool filter, uint32_t *qidx, uint64_t *qkey,
                                               KeyOf key_of, Keep keep, Body body) {
    const int lane = lane_id();
    uint32_t fill = 0;  // wave-uniform
    uint64_t c = w.first;
    uint64_t key = 0;
    if (c * kWave + (uint64_t)lane < n) key = key_of(c * kWave + (uint64_t)lane);
    for (; c * kWave < n; c += w.stride) {
        const uint64_t i = c * kWave + (uint64_t)lane;
        const uint64_t inext = (c + w.stride) * kWave + (uint64_t)lane;
        uint64_t knext = 0;
        if (inext < n) knext = key_of(inext);
        const bool mine = i < n && (!filter || keep(key));
        const uint64_t m = __ballot(mine);
        if (mine) {
            const uint32_t at = fill + mask_rank(m);
            qidx[at] = (uint32_t)i;
            qkey[at] = key;
        }
        key = knext;
        fill += (uint32_t)__builtin_popcountll(m);
        __builtin_amdgcn_wave_barrier();
        if (fill >= (uint32_t)kWave) {
            const uint32_t item = qidx[lane];
            const uint64_t ikey = qkey[lane];
            const uint32_t spill = qidx[kWave + lane];
            const uint64_t skey = qkey[kWave + lane];
            body((uint64_t)item, ikey);
            fill -= kWave;
            if ((uint32_t)lane < fill) {
                qidx[lane] = spill;
                qkey[lane] = skey;
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
    if ((uint32_t)lane < fill) body((uint64_t)qidx[lane], qkey[lane]);
}

__global__ void __launch_bounds__(kHashThreads)
hash_insert_kernel(Slot *__restrict__ table, uint64_t mask, const uint64_t *__restrict__ keys,
                   const uint64_t *__restrict__ vals, uint64_t n, int mode, HomeMap home,
                   unsigned long long *__restrict__ failed, XcdHint xh) {
    __shared__ uint32_t qidx[kHashThreads / kWave][2 * kWave];
    __shared__ uint64_t qkey[kHashThreads / kWave][2 * kWave];
    __shared__ uint8_t lattr[kLdsPages];
    const Walk w = make_walk(mode, xh);
    const bool filter = mode != XD_MODE_OBLIVIOUS;
    const uint64_t base = reinterpret_cast<uint64_t>(table);
    const SlotHome sh = stage_home(home, base, (mask + 1) * sizeof(Slot), lattr, filter);
    const uint64_t max_probe = mask + 1 < kMaxProbe ? mask + 1 : kMaxProbe;
    auto key_of = [&](uint64_t i) { return keys[i]; };
    auto keep = [&](uint64_t key) { return sh(base + (mix64(key) & mask) * sizeof(Slot)) == w.want; };
    auto body = [&](uint64_t i, uint64_t key) {
        if (key == kEmpty) return;
        if (!slot_insert(table, mask, mix64(key) & mask, key, vals[i], max_probe) && failed) atomicAdd(failed, 1ull);
    };
    for_each_owned(w, n, filter, qidx[threadIdx.x / kWave], qkey[threadIdx.x / kWave], key_of, keep, body);
}

__global__ void __launch_bounds__(kHashThreads)
hash_lookup_kernel(const Slot *__restrict__ table, uint64_t mask, const uint64_t *__restrict__ queries, uint64_t n,
                   int mode, HomeMap home, uint64_t *__restrict__ vals_out, uint8_t *__restrict__ found_out,
                   XcdHint xh) {
    __shared__ uint32_t qidx[kHashThreads / kWave][2 * kWave];
    __shared__ uint64_t qkey[kHashThreads / kWave][2 * kWave];
    __shared__ uint8_t lattr[kLdsPages];
    const Walk w = make_walk(mode, xh);
    const bool filter = mode != XD_MODE_OBLIVIOUS;
    const uint64_t base = reinterpret_cast<uint64_t>(table);
    const SlotHome sh = stage_home(home, base, (mask + 1) * sizeof(Slot), lattr, filter);
    const uint64_t max_probe = mask + 1 < kMaxProbe ? mask + 1 : kMaxProbe;
    auto key_of = [&](uint64_t i) { return queries[i]; };
    auto keep = [&](uint64_t q) { return sh(base + (mix64(q) & mask) * sizeof(Slot)) == w.want; };
    auto body = [&](uint64_t i, uint64_t q) {
        uint64_t s = mix64(q) & mask;
        uint64_t v = 0;
        uint8_t f = 0;
        if (q != kEmpty) {
            for (uint64_t step = 0; step < max_probe; ++step) {
                // the whole 16-byte slot in one load: reading the value after a key match
                // would send a second request for the same line
                const uint4 e = reinterpret_cast<const uint4 *>(table)[s];
                asm volatile("" ::"v"(e.z), "v"(e.w));  // keeps the value in the same load
                const uint64_t ek = (uint64_t)e.x | ((uint64_t)e.y << 32);
                if (ek == q) {
                    v = (uint64_t)e.z | ((uint64_t)e.w << 32);
                    f = 1;
                    break;
                }
                if (ek == kEmpty) break;
                s = (s + 1) & mask;
            }
        }
        vals_out[i] = v;
        found_out[i] = f;
    };
    for_each_owned(w, n, filter, qidx[threadIdx.x / kWave], qkey[threadIdx.x / kWave], key_of, keep, body);
}

// ---------------------------------------------------------------------------------------
// The reference's dependent-probe workload (hash_probe_dep.cu): 8-byte entries {int key;
// int next}, EMPTY key -1, home slot mix32(key) & mask, linear probing; a query follows its
// key's `next` chain for chain_len probes and returns (sum of found slots, -1 for a miss) ^
// final key. The aware mode routes each query to the die that homes its first slot.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t mix32d(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// probe_chain_one (HASH.cu:46-64): the found slot or -1, and the key's successor (the key
// itself when it is absent).
__device__ __forceinline__ int32_t dep_probe_one(const int2 *__restrict__ table, uint32_t mask, int32_t key,
                                                 int32_t &next) {
    uint32_t slot = mix32d((uint32_t)key) & mask;
    bool found = false;
    int32_t nk = key;
    for (uint64_t step = 0; step <= (uint64_t)mask; ++step) {
        // one 8-byte load per entry: fetching the successor separately after a match would
        // send a second request for the same line
        const uint64_t e = reinterpret_cast<const uint64_t *>(table)[slot];
        const int32_t ek = (int32_t)(uint32_t)e;
        if (ek == key) {
            found = true;
            nk = (int32_t)(uint32_t)(e >> 32);
            break;
        }
        if (ek == -1) break;
        slot = (slot + 1) & mask;
    }
    next = nk;
    return found ? (int32_t)slot : -1;
}

__global__ void __launch_bounds__(kHashThreads)
dep_probe_kernel(const int2 *__restrict__ table, uint32_t mask, const int32_t *__restrict__ queries, uint64_t n,
                 int chain_len, int32_t *__restrict__ out, int mode, HomeMap home, XcdHint xh) {
    __shared__ uint32_t qidx[kHashThreads / kWave][2 * kWave];
    __shared__ uint64_t qkey[kHashThreads / kWave][2 * kWave];
    __shared__ uint8_t lattr[kLdsPages];
    const Walk w = make_walk(mode, xh);
    const bool filter = mode != XD_MODE_OBLIVIOUS;
    const uint64_t base = reinterpret_cast<uint64_t>(table);
    const SlotHome sh = stage_home(home, base, ((uint64_t)mask + 1) * sizeof(int2), lattr, filter);
    auto key_of = [&](uint64_t i) { return (uint64_t)(uint32_t)queries[i]; };
    auto keep = [&](uint64_t key) {
        return sh(base + (uint64_t)(mix32d((uint32_t)key) & mask) * sizeof(int2)) == w.want;
    };
    auto body = [&](uint64_t i, uint64_t qkey32) {
        int32_t key = (int32_t)(uint32_t)qkey32;
        uint32_t acc = 0;  // wraps like the reference's int accumulator
        for (int it = 0; it < chain_len; ++it) {
            int32_t nk;
            acc += (uint32_t)dep_probe_one(table, mask, key, nk);
            key = nk;
        }
        out[i] = (int32_t)(acc ^ (uint32_t)key);
    };
    for_each_owned(w, n, filter, qidx[threadIdx.x / kWave], qkey[threadIdx.x / kWave], key_of, keep, body);
}

// Routed dependent probe: the reference's per-side query lists (HASH.cu:244-270, built on the
// host there, outside the timed region) built on the device by an order-preserving partition
// of the queries by the die homing their first slot; probe_dep_sa (:85-116) is then a probe
// in which die d consumes list d (aware) or list 1 - d (rotated) and scatters out[qid].
// Route buffer: {uint64 n0, uint64 n} | per-block die-1 counts (their exclusive prefix after
// the scan) | int2 entries {key, qid}: die-0 list [0, n0), die-1 list [n0, n), each in query
// order.
constexpr int kRouteBlock = 4096;  // queries per partition block
constexpr int kRoutePer = kRouteBlock / kHashThreads;
constexpr int kScanThreads = 1024;

struct RouteLayout {
    size_t bcnt, entries, total;
    uint64_t nblocks;
};

static RouteLayout route_layout(uint64_t n) {
    RouteLayout L;
    L.nblocks = (n + kRouteBlock - 1) / kRouteBlock;
    L.bcnt = 256;
    L.entries = (L.bcnt + 4 * L.nblocks + 255) & ~(size_t)255;
    L.total = L.entries + 8 * n;
    return L;
}

__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t *red) {
    v = wave_sum_u32(v);
    const int wave = (int)threadIdx.x / kWave;
    if (lane_id() == 0) red[wave] = v;
    __syncthreads();
    uint32_t t = 0;
    for (int w = 0; w < (int)blockDim.x / kWave; ++w) t += red[w];
    __syncthreads();
    return t;
}

__global__ void __launch_bounds__(kHashThreads)
route_count_kernel(uint32_t mask, const int32_t *__restrict__ queries, uint64_t n, HomeMap home, uint64_t base,
                   uint32_t *__restrict__ bcnt) {
    __shared__ uint8_t lattr[kLdsPages];
    __shared__ uint32_t red[kHashThreads / kWave];
    const SlotHome sh = stage_home(home, base, ((uint64_t)mask + 1) * sizeof(int2), lattr, true);
    const uint64_t i0 = (uint64_t)blockIdx.x * kRouteBlock;
    uint32_t c1 = 0;
#pragma unroll
    for (int j = 0; j < kRoutePer; ++j) {
        const uint64_t i = i0 + (uint64_t)j * kHashThreads + threadIdx.x;
        if (i < n) c1 += sh(base + (uint64_t)(mix32d((uint32_t)queries[i]) & mask) * sizeof(int2));
    }
    const uint32_t t = block_sum_u32(c1, red);
    if (threadIdx.x == 0) bcnt[blockIdx.x] = t;
}

// One workgroup: exclusive prefix of the per-block die-1 counts, in place; header = {n0, n}.
__global__ void __launch_bounds__(kScanThreads) route_scan_kernel(uint32_t *bcnt, uint64_t nblocks, uint64_t n,
                                                                 unsigned long long *header) {
    __shared__ uint32_t wsum[kScanThreads / kWave];
    __shared__ uint64_t carry_s;
    if (threadIdx.x == 0) carry_s = 0;
    __syncthreads();
    const int lane = lane_id(), wave = (int)threadIdx.x / kWave;
    for (uint64_t c0 = 0; c0 < nblocks; c0 += kScanThreads) {
        const uint64_t i = c0 + threadIdx.x;
        const uint32_t v = i < nblocks ? bcnt[i] : 0u;
        uint32_t incl = v;  // inclusive scan inside the wave
        for (int off = 1; off < kWave; off <<= 1) {
            const uint32_t o = __shfl_up(incl, off);
            if (lane >= off) incl += o;
        }
        if (lane == kWave - 1) wsum[wave] = incl;
        __syncthreads();
        uint32_t before = 0, total = 0;
        for (int w = 0; w < kScanThreads / kWave; ++w) {
            if (w < wave) before += wsum[w];
            total += wsum[w];
        }
        const uint64_t carry = carry_s;
        if (i < nblocks) bcnt[i] = (uint32_t)(carry + before + incl - v);
        __syncthreads();
        if (threadIdx.x == 0) carry_s = carry + total;
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        header[0] = n - carry_s;
        header[1] = n;
    }
}

__global__ void __launch_bounds__(kHashThreads)
route_scatter_kernel(uint32_t mask, const int32_t *__restrict__ queries, uint64_t n, HomeMap home, uint64_t base,
                     const uint32_t *__restrict__ bcnt, const unsigned long long *__restrict__ header,
                     int2 *__restrict__ entries) {
    __shared__ uint8_t lattr[kLdsPages];
    __shared__ uint32_t w0[kHashThreads / kWave], w1[kHashThreads / kWave];
    const SlotHome sh = stage_home(home, base, ((uint64_t)mask + 1) * sizeof(int2), lattr, true);
    const uint64_t b = blockIdx.x, i0 = b * kRouteBlock;
    const uint64_t n0 = header[0];
    const uint64_t off1 = bcnt[b], off0 = i0 - off1;
    const int lane = lane_id(), wave = (int)threadIdx.x / kWave;
    const uint64_t lt = (1ull << lane) - 1ull;
    uint64_t r0 = 0, r1 = 0;  // entries of each list written by the earlier slabs of this block
    for (int j = 0; j < kRoutePer; ++j) {
        const uint64_t i = i0 + (uint64_t)j * kHashThreads + threadIdx.x;
        const bool valid = i < n;
        const int32_t key = valid ? queries[i] : 0;
        const uint32_t d = valid ? sh(base + (uint64_t)(mix32d((uint32_t)key) & mask) * sizeof(int2)) : 0u;
        const uint64_t m1 = __ballot(valid && d == 1u), m0 = __ballot(valid && d == 0u);
        if (lane == 0) {
            w0[wave] = (uint32_t)__builtin_popcountll(m0);
            w1[wave] = (uint32_t)__builtin_popcountll(m1);
        }
        __syncthreads();
        uint32_t p0 = 0, p1 = 0, t0 = 0, t1 = 0;
        for (int w = 0; w < kHashThreads / kWave; ++w) {
            if (w < wave) {
                p0 += w0[w];
                p1 += w1[w];
            }
            t0 += w0[w];
            t1 += w1[w];
        }
        if (valid) {
            const uint64_t pos = d ? n0 + off1 + r1 + p1 + (uint64_t)__builtin_popcountll(m1 & lt)
                                   : off0 + r0 + p0 + (uint64_t)__builtin_popcountll(m0 & lt);
            entries[pos] = make_int2(key, (int32_t)i);
        }
        r0 += t0;
        r1 += t1;
        __syncthreads();
    }
}

__global__ void __launch_bounds__(kHashThreads)
dep_probe_routed_kernel(const int2 *__restrict__ table, uint32_t mask, const int2 *__restrict__ entries,
                        const unsigned long long *__restrict__ header, int chain_len, int32_t *__restrict__ out,
                        int mode, XcdHint xh) {
    report_xcd(xh);
    const uint64_t n0 = header[0], n = header[1];
    const int b = (int)blockIdx.x;
    uint64_t first, end, rank, nwg;
    if (mode == XD_MODE_OBLIVIOUS) {
        first = 0;
        end = n;
        rank = (uint64_t)b;
        nwg = gridDim.x;
    } else {
        const uint32_t die = wg_die(b, xh);
        const uint32_t list = (mode == XD_MODE_AWARE) ? die : (die ^ 1u);
        first = list ? n0 : 0;
        end = list ? n : n0;
        rank = (uint64_t)die_rank(b, xh);
        nwg = gridDim.x / 2;
    }
    for (uint64_t idx = first + rank * kHashThreads + threadIdx.x; idx < end; idx += nwg * kHashThreads) {
        const int2 e = entries[idx];
        int32_t key = e.x;
        uint32_t acc = 0;  // wraps like the reference's int accumulator
        for (int it = 0; it < chain_len; ++it) {
            int32_t nk;
            acc += (uint32_t)dep_probe_one(table, mask, key, nk);
            key = nk;
        }
        out[e.y] = (int32_t)(acc ^ (uint32_t)key);
    }
}

// Seeded inputs (device): key i = splitmix64(seed, i) (distinct for distinct i),
// value i = splitmix64(seed ^ 0x5BD1E9955BD1E995, i); query j is a hit for even j
// (key splitmix64(qseed, j) mod n_keys) and a miss for odd j (key n_keys + j/2, from the
// disjoint index range above the inserted keys).
__device__ __forceinline__ uint64_t sm64(uint64_t seed, uint64_t i) { return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ull); }

__global__ void __launch_bounds__(256) gen_hash_kv_kernel(uint64_t *keys, uint64_t *vals, uint64_t n, uint64_t seed) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        keys[i] = sm64(seed, i);
        if (vals) vals[i] = sm64(seed ^ 0x5BD1E9955BD1E995ull, i);
    }
}

__global__ void __launch_bounds__(256) gen_hash_queries_kernel(uint64_t *q, uint64_t n, uint64_t n_keys, uint64_t seed,
                                                               uint64_t qseed) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t j = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += stride) {
        const uint64_t idx = (j & 1) ? n_keys + (j >> 1) : sm64(qseed, j) % n_keys;
        q[j] = sm64(seed, idx);
    }
}

static unsigned grid_for(uint64_t n, unsigned cap) {
    uint64_t g = (n + 255) / 256;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

static int check_table(const void *table, uint64_t slots) {
    XD_REQUIRE(table != nullptr && aligned16(table), "hash: table must be non-NULL and 16-byte aligned");
    XD_REQUIRE(slots >= 1 && (slots & (slots - 1)) == 0, "hash: slots must be a power of two");
    return XD_OK;
}

// Grid for the probing kernels: a multiple of 8 so that every XCD gets the same number of
// workgroups (workgroup i runs on XCD i mod 8), at most `cap` workgroups (waves then walk
// several 64-item chunks).
constexpr uint64_t kWalkCap = 256 * 16;  // insert and routed probes: 16 workgroups per CU
static unsigned probe_grid(uint64_t n, uint64_t cap = kWalkCap) {
    uint64_t g = (n + kHashThreads - 1) / kHashThreads;
    if (g > cap) g = cap;
    g = (g + kNumXcd - 1) / kNumXcd * kNumXcd;
    return (unsigned)g;
}

// Lookups and dependent probes: oblivious calls give every wave one chunk and let the
// dispatcher refill the CUs; the home modes, whose waves walk every chunk and keep about
// half, cap the grid at 2^16 workgroups (each stages the table's page map in LDS). At 2^26
// lookups into 2^27 slots, kernel µs oblivious / aware: 2202 / 2451 with 4096 workgroups,
// 2207 / 2414 at 2^14, 2141 / 2285 at 2^16, 2090 / 2378 at one chunk per wave (aware 2315 at
// 2^15 and 2310 at 2^17); the reference's dependent probe (8 M queries) 552 / 407 against
// 535 / 396 at 2^16 or one chunk per wave.
// (2^23 workgroups keep the dispatch's work-item count, a 32-bit field, at 2^31.)
static unsigned lookup_grid(uint64_t n, int mode) {
    return probe_grid(n, mode == XD_MODE_OBLIVIOUS ? (1ull << 23) : (1ull << 16));
}

}  // namespace xd

using namespace xd;

extern "C" {

size_t xd_hash_table_bytes(uint64_t slots) { return (size_t)slots * sizeof(Slot); }

int xd_hash_init(void *table, uint64_t slots, void *stream) {
    if (int rc = check_table(table, slots)) return rc;
    launch("hash_init_kernel", hash_init_kernel, dim3(grid_for(slots, 8192)), dim3(256), 0, (hipStream_t)stream,
                       static_cast<Slot *>(table), slots);
    return launch_status("hash_init_kernel");
}

int xd_hash_insert_u64(void *table, uint64_t slots, const uint64_t *keys, const uint64_t *vals, uint64_t n, int mode,
                       const uint8_t *home_attr, unsigned long long *failed, void *stream) {
    if (int rc = check_table(table, slots)) return rc;
    XD_REQUIRE(n == 0 || (keys != nullptr && vals != nullptr), "xd_hash_insert_u64: NULL keys/vals");
    XD_REQUIRE(n < (1ull << 32), "xd_hash_insert_u64: n must be < 2^32 per call");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "xd_hash_insert_u64: bad mode");
    if (n == 0) return XD_OK;
    launch("hash_insert_kernel", hash_insert_kernel, dim3(probe_grid(n)), dim3(kHashThreads), 0, (hipStream_t)stream,
                       static_cast<Slot *>(table), slots - 1, keys, vals, n, mode,
                       HomeMap{home_attr, reinterpret_cast<uint64_t>(table) / kHomePage, home_mask()}, failed,
                       xcd_hint((hipStream_t)stream));
    return launch_status("hash_insert_kernel");
}

int xd_hash_lookup_u64(const void *table, uint64_t slots, const uint64_t *queries, uint64_t n, uint64_t *vals_out,
                       uint8_t *found_out, int mode, const uint8_t *home_attr, void *stream) {
    if (int rc = check_table(table, slots)) return rc;
    XD_REQUIRE(n == 0 || (queries != nullptr && vals_out != nullptr && found_out != nullptr),
               "xd_hash_lookup_u64: NULL queries/outputs");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "xd_hash_lookup_u64: bad mode");
    XD_REQUIRE(n < (1ull << 32), "xd_hash_lookup_u64: n must be < 2^32 per call");
    if (n == 0) return XD_OK;
    launch("hash_lookup_kernel", hash_lookup_kernel, dim3(lookup_grid(n, mode)), dim3(kHashThreads), 0, (hipStream_t)stream,
                       static_cast<const Slot *>(table), slots - 1, queries, n, mode,
                       HomeMap{home_attr, reinterpret_cast<uint64_t>(table) / kHomePage, home_mask()}, vals_out,
                       found_out, xcd_hint((hipStream_t)stream));
    return launch_status("hash_lookup_kernel");
}

int xd_dep_probe(const void *table, uint64_t slots, const int32_t *queries, uint64_t n, int chain_len, int32_t *out,
                 int mode, const uint8_t *home_attr, void *stream) {
    XD_REQUIRE(table != nullptr && (reinterpret_cast<uintptr_t>(table) & 7u) == 0, "xd_dep_probe: table must be 8-byte aligned");
    XD_REQUIRE(slots >= 2 && (slots & (slots - 1)) == 0 && slots <= (1ull << 32), "xd_dep_probe: slots must be a power of two <= 2^32");
    XD_REQUIRE(n == 0 || (queries != nullptr && out != nullptr), "xd_dep_probe: NULL queries/out");
    XD_REQUIRE(n < (1ull << 32), "xd_dep_probe: n must be < 2^32");
    XD_REQUIRE(chain_len >= 1 && chain_len <= 4096, "xd_dep_probe: chain_len must be in [1, 4096]");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "xd_dep_probe: bad mode");
    if (n == 0) return XD_OK;
    launch("dep_probe_kernel", dep_probe_kernel, dim3(lookup_grid(n, mode)), dim3(kHashThreads), 0, (hipStream_t)stream,
                       static_cast<const int2 *>(table), (uint32_t)(slots - 1), queries, n, chain_len, out, mode,
                       HomeMap{home_attr, reinterpret_cast<uint64_t>(table) / kHomePage, home_mask()},
                       xcd_hint((hipStream_t)stream));
    return launch_status("dep_probe_kernel");
}

size_t xd_dep_route_bytes(uint64_t n) { return route_layout(n).total; }

int xd_dep_route(const void *table, uint64_t slots, const int32_t *queries, uint64_t n, const uint8_t *home_attr,
                 void *route, size_t route_bytes, void *stream) {
    XD_REQUIRE(table != nullptr && (reinterpret_cast<uintptr_t>(table) & 7u) == 0, "xd_dep_route: table must be 8-byte aligned");
    XD_REQUIRE(slots >= 2 && (slots & (slots - 1)) == 0 && slots <= (1ull << 32), "xd_dep_route: slots must be a power of two <= 2^32");
    XD_REQUIRE(n < (1ull << 31), "xd_dep_route: n must be < 2^31 (int query ids)");
    XD_REQUIRE(n == 0 || queries != nullptr, "xd_dep_route: NULL queries");
    const RouteLayout L = route_layout(n);
    if (route == nullptr || route_bytes < L.total || !aligned16(route))
        return fail(XD_ERR_WORKSPACE, "xd_dep_route: route buffer missing, misaligned or smaller than xd_dep_route_bytes()");
    hipStream_t s = (hipStream_t)stream;
    char *r = static_cast<char *>(route);
    unsigned long long *header = reinterpret_cast<unsigned long long *>(r);
    uint32_t *bcnt = reinterpret_cast<uint32_t *>(r + L.bcnt);
    const uint64_t base = reinterpret_cast<uint64_t>(table);
    const HomeMap home{home_attr, base / kHomePage, home_mask()};
    if (n > 0) {
        launch("route_count_kernel", route_count_kernel, dim3((unsigned)L.nblocks), dim3(kHashThreads), 0, s,
                           (uint32_t)(slots - 1), queries, n, home, base, bcnt);
        if (int rc = launch_status("route_count_kernel")) return rc;
    }
    launch("route_scan_kernel", route_scan_kernel, dim3(1), dim3(kScanThreads), 0, s, bcnt, L.nblocks, n, header);
    if (int rc = launch_status("route_scan_kernel")) return rc;
    if (n == 0) return XD_OK;
    launch("route_scatter_kernel", route_scatter_kernel, dim3((unsigned)L.nblocks), dim3(kHashThreads), 0, s,
                       (uint32_t)(slots - 1), queries, n, home, base, bcnt, header,
                       reinterpret_cast<int2 *>(r + L.entries));
    return launch_status("route_scatter_kernel");
}

int xd_dep_probe_routed(const void *table, uint64_t slots, const void *route, uint64_t n, int chain_len, int32_t *out,
                        int mode, void *stream) {
    XD_REQUIRE(table != nullptr && (reinterpret_cast<uintptr_t>(table) & 7u) == 0, "xd_dep_probe_routed: table must be 8-byte aligned");
    XD_REQUIRE(slots >= 2 && (slots & (slots - 1)) == 0 && slots <= (1ull << 32), "xd_dep_probe_routed: slots must be a power of two <= 2^32");
    XD_REQUIRE(n < (1ull << 31), "xd_dep_probe_routed: n must be < 2^31");
    XD_REQUIRE(route != nullptr && aligned16(route) && (n == 0 || out != nullptr), "xd_dep_probe_routed: NULL route/out");
    XD_REQUIRE(chain_len >= 1 && chain_len <= 4096, "xd_dep_probe_routed: chain_len must be in [1, 4096]");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "xd_dep_probe_routed: bad mode");
    if (n == 0) return XD_OK;
    const RouteLayout L = route_layout(n);
    const char *r = static_cast<const char *>(route);
    launch("dep_probe_routed_kernel", dep_probe_routed_kernel, dim3(probe_grid(n)), dim3(kHashThreads), 0, (hipStream_t)stream,
                       static_cast<const int2 *>(table), (uint32_t)(slots - 1),
                       reinterpret_cast<const int2 *>(r + L.entries), reinterpret_cast<const unsigned long long *>(r),
                       chain_len, out, mode, xcd_hint((hipStream_t)stream));
    return launch_status("dep_probe_routed_kernel");
}

int xd_gen_hash_kv(uint64_t *keys, uint64_t *vals, uint64_t n, uint64_t seed, void *stream) {
    XD_REQUIRE(n == 0 || keys != nullptr, "xd_gen_hash_kv: NULL keys");
    if (n == 0) return XD_OK;
    launch("gen_hash_kv_kernel", gen_hash_kv_kernel, dim3(grid_for(n, 8192)), dim3(256), 0, (hipStream_t)stream, keys, vals, n,
                       seed);
    return launch_status("gen_hash_kv_kernel");
}

int xd_gen_hash_queries(uint64_t *queries, uint64_t n, uint64_t n_keys, uint64_t seed, uint64_t qseed, void *stream) {
    XD_REQUIRE(n == 0 || queries != nullptr, "xd_gen_hash_queries: NULL queries");
    XD_REQUIRE(n_keys > 0, "xd_gen_hash_queries: n_keys must be positive");
    if (n == 0) return XD_OK;
    launch("gen_hash_queries_kernel", gen_hash_queries_kernel, dim3(grid_for(n, 8192)), dim3(256), 0, (hipStream_t)stream, queries, n,
                       n_keys, seed, qseed);
    return launch_status("gen_hash_queries_kernel");
}

}  // extern "C"
