// The u64 open-addressing table shared by the insert/lookup kernels (xd_hash.hip) and the
// bulk build (xd_hash_build.hip): 16-byte slots {key, value}, EMPTY = all ones, home slot
// mix64(key) & (slots - 1), linear probing with wrap-around.
#pragma once

#include <hip/hip_runtime.h>

#include "xd_common.hpp"

namespace xd {

constexpr uint64_t kEmpty = ~0ull;
constexpr uint64_t kMaxProbe = 1ull << 16;

struct __attribute__((aligned(16))) Slot {
    uint64_t key;
    uint64_t val;
};

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Inserts (key, val) into the table in global memory, probing from slot s: a plain
// (possibly stale) read of the key pre-checks each slot -- a slot's key only ever changes
// from EMPTY to a key, so a stale read can only show EMPTY for a taken slot, and the
// compare-and-swap then returns the real owner -- so only slots that look free pay for the
// memory-side atomic. An existing equal key gets the new value. Returns false when no slot
// was found within max_probe probes.
__device__ __forceinline__ bool slot_insert(Slot *table, uint64_t mask, uint64_t s, uint64_t key, uint64_t val,
                                            uint64_t max_probe) {
    for (uint64_t step = 0; step < max_probe; ++step) {
        unsigned long long *kp = reinterpret_cast<unsigned long long *>(&table[s].key);
        const uint64_t cur = __hip_atomic_load(kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        uint64_t owner = cur;
        if (cur == kEmpty) owner = atomicCAS(kp, (unsigned long long)kEmpty, (unsigned long long)key);
        if (owner == kEmpty || owner == key) {
            table[s].val = val;
            return true;
        }
        s = (s + 1) & mask;
    }
    return false;
}

}  // namespace xd
