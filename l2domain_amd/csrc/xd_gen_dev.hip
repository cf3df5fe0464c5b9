// Device-side seeded generators for the large integer inputs (Zipf histogram keys).
// Integer-only: the result does not depend on device math libraries, so the host oracle
// regenerates exactly the same keys from the same seed and threshold table.
#include <hip/hip_runtime.h>

#include "xd_common.hpp"

namespace xd {

__device__ __forceinline__ uint64_t d_splitmix64(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void __launch_bounds__(256) gen_zipf_keys_kernel(uint32_t *__restrict__ keys, size_t n,
                                                            const uint64_t *__restrict__ t, uint32_t num_bins,
                                                            uint64_t seed, int scramble) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const bool pow2 = (num_bins & (num_bins - 1)) == 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t u = d_splitmix64(seed, i);
        uint32_t lo = 0, hi = num_bins - 1;  // least k with u < t[k]; num_bins-1 if none
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (u < t[mid]) hi = mid;
            else lo = mid + 1;
        }
        uint32_t k = lo;
        if (scramble && pow2) k = (uint32_t)(((uint64_t)(k + 1) * 0x9E3779B1ull) & (num_bins - 1));
        keys[i] = k;
    }
}

}  // namespace xd

using namespace xd;

extern "C" int xd_gen_zipf_keys(uint32_t *keys, size_t n, const uint64_t *thresholds, uint32_t num_bins,
                                uint64_t seed, int scramble, void *stream) {
    XD_REQUIRE(num_bins >= 1, "xd_gen_zipf_keys: num_bins must be >= 1");
    XD_REQUIRE(n == 0 || (keys != nullptr && thresholds != nullptr), "xd_gen_zipf_keys: NULL pointer");
    if (n == 0) return XD_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    launch("gen_zipf_keys_kernel", gen_zipf_keys_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, keys, n,
                       thresholds, num_bins, seed, scramble);
    return launch_status("gen_zipf_keys_kernel");
}
