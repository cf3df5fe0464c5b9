// Host side of the reference's dependent-probe hash workload, reproduced as an input mode
// (applications/hash/src/hash_probe_dep.cu:118-270): 32-bit keys with a `next` key each,
// two hot pools whose home slots lie on opposite sides (here: I/O dies, from the measured
// home map of the table) chained into cycles, cold keys that point to themselves, a table
// built serially on the CPU in shuffled order, and a query stream that alternates the two
// hot pools for hot_pct percent of the queries. The reference draws its randomness from
// std::mt19937 and std::uniform_int_distribution (implementation-defined); every draw here
// is xd_rand64(seed, i) so any implementation regenerates the same workload.
#include <stdint.h>
#include <string.h>

#include <vector>

#include "xdom.h"

namespace {

inline uint32_t mix32(uint32_t x) {  // lowbias32, the slot function of HASH.cu:29-36
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// Die homing entry `slot` of an 8-byte-entry table at device address `base`.
inline uint32_t slot_home(uint64_t base, uint64_t slot, const uint8_t *attr, uint64_t mask_bits) {
    const uint64_t a = base + slot * 8;
    if (attr) return (uint32_t)(((a >> 13) & 1u) ^ attr[(a >> 21) - (base >> 21)]);
    return (uint32_t)(__builtin_popcountll(a & mask_bits) & 1);
}

}  // namespace

extern "C" {

int xd_dep_make_keys(uint64_t table_addr, uint64_t slots, const uint8_t *home_attr_host, int32_t K, int32_t H,
                     int32_t *keys, int32_t *nexts) {
    if (slots < 2 || (slots & (slots - 1)) || K <= 0 || H <= 0 || 2LL * H > K || (uint64_t)K >= slots || !keys ||
        !nexts)
        return XD_ERR_INVALID_ARG;
    const uint32_t mask = (uint32_t)(slots - 1);
    const uint64_t mbits = xd_home_mask();
    std::vector<int32_t> hot0, hot1;
    hot0.reserve((size_t)H);
    hot1.reserve((size_t)H);
    int64_t cand = 1;  // odd keys, ascending (HASH.cu:197-209)
    while ((int32_t)hot0.size() < H || (int32_t)hot1.size() < H) {
        if (cand > INT32_MAX) return XD_ERR_UNSUPPORTED;
        const int32_t key = (int32_t)cand;
        cand += 2;
        const uint32_t side = slot_home(table_addr, mix32((uint32_t)key) & mask, home_attr_host, mbits);
        if (side == 0 && (int32_t)hot0.size() < H) hot0.push_back(key);
        else if (side == 1 && (int32_t)hot1.size() < H) hot1.push_back(key);
    }
    int32_t n = 0;
    for (int32_t i = 0; i < H; ++i, ++n) {
        keys[n] = hot0[i];
        nexts[n] = hot0[(i + 1) % H];
    }
    for (int32_t i = 0; i < H; ++i, ++n) {
        keys[n] = hot1[i];
        nexts[n] = hot1[(i + 1) % H];
    }
    for (; n < K; ++n) {
        if (cand > INT32_MAX) return XD_ERR_UNSUPPORTED;
        keys[n] = (int32_t)cand;
        nexts[n] = (int32_t)cand;  // a cold key is its own successor: its chain stays put
        cand += 2;
    }
    return XD_OK;
}

int xd_dep_build(int32_t *table, uint64_t slots, const int32_t *keys, const int32_t *nexts, int32_t K, uint64_t seed) {
    if (!table || !keys || !nexts || slots < 2 || (slots & (slots - 1)) || K <= 0 || (uint64_t)K >= slots)
        return XD_ERR_INVALID_ARG;
    const uint32_t mask = (uint32_t)(slots - 1);
    for (uint64_t s = 0; s < slots; ++s) {
        table[2 * s] = -1;  // EMPTY_KEY
        table[2 * s + 1] = 0;
    }
    std::vector<int32_t> perm((size_t)K);
    for (int32_t i = 0; i < K; ++i) perm[(size_t)i] = i;
    for (int64_t i = K - 1; i > 0; --i) {  // Fisher-Yates, j = rand64(seed, i) mod (i + 1)
        const int64_t j = (int64_t)(xd_rand64(seed, (uint64_t)i) % (uint64_t)(i + 1));
        const int32_t t = perm[(size_t)i];
        perm[(size_t)i] = perm[(size_t)j];
        perm[(size_t)j] = t;
    }
    for (int32_t p : perm) {  // serial insertion, HASH.cu:232-241
        uint32_t slot = mix32((uint32_t)keys[p]) & mask;
        while (table[2 * (size_t)slot] != -1) slot = (slot + 1) & mask;
        table[2 * (size_t)slot] = keys[p];
        table[2 * (size_t)slot + 1] = nexts[p];
    }
    return XD_OK;
}

int xd_dep_queries(int32_t *queries, int32_t Q, const int32_t *keys, int32_t K, int32_t H, int32_t hot_pct,
                   uint64_t seed) {
    if (!queries || !keys || Q <= 0 || K <= 0 || H <= 0 || 2LL * H > K || hot_pct < 0 || hot_pct > 100)
        return XD_ERR_INVALID_ARG;
    const int64_t hot = (int64_t)Q * hot_pct / 100;
    for (int64_t i = 0; i < Q; ++i) {
        const uint64_t r = xd_rand64(seed, (uint64_t)i);
        if (i < hot) queries[i] = keys[(size_t)((i & 1) ? H : 0) + (size_t)(r % (uint64_t)H)];  // pools alternate
        else queries[i] = keys[(size_t)(r % (uint64_t)K)];
    }
    return XD_OK;
}

}  // extern "C"
