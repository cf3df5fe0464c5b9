// Architecture probes: XDom-PChase (same-XCD vs cross-XCD hit latency of a pointer chase)
// and MaskProbe (the address bits that move a line between the two I/O dies).
//
// Reference: utility/latopt.cuh k_peer_pchase (354-406) and peer_pchase; architecture/src/
// architecture_probe.cu run_figure_2 (572-596: leader/follower chase of 2048 elements at a
// 128-byte stride, four traces), measure_offsets / derive_active_bits / run_mask_probe
// (417-458, 495-523, 644-670: per-bit latency curves seen from the two sides, active bits
// where the near/far relation flips against the base address).
//
// MI355X design. The reference pins a leader and a follower to two SMs and hands over with
// a flag in global memory. Here the leader and the follower are workgroups placed on chosen
// XCDs (workgroup i is dispatched to XCD i mod 8, and each role is claimed with a CAS by the
// first workgroup whose HW_REG_XCC_ID matches), and the handover is a kernel boundary:
// the leader's launch finishes before the follower's starts, and L2 contents survive the
// boundary, so no workgroup ever waits on another. Latencies are s_memtime deltas around
// one dependent load (or one returning memory-side atomic), kept in LDS until the chase ends.
#include <hip/hip_runtime.h>

#include "xd_common.hpp"

namespace xd {

constexpr int kMaxChase = 8192;  // elements per trace (LDS: 4 bytes each)

__global__ void chase_init_kernel(uint64_t *chain, int numel, int stride_words) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < numel) {
        const int nxt = (i + 1) % numel;
        chain[(size_t)i * stride_words] = reinterpret_cast<uint64_t>(chain + (size_t)nxt * stride_words);
    }
}

__global__ void probe_clear_kernel(uint32_t *w, int n) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) w[i] = 0u;
}

// One timed dependent load: returns the cycles between issue and arrival, and the loaded
// pointer in `next`.
__device__ __forceinline__ uint32_t timed_load(const uint64_t *p, uint64_t &next) {
    uint64_t t0, t1, v;
    asm volatile(
        "s_waitcnt vmcnt(0) lgkmcnt(0)\n\t"
        "s_memtime %0\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "global_load_dwordx2 %2, %3, off\n\t"
        "s_waitcnt vmcnt(0)\n\t"
        "s_memtime %1\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        : "=&s"(t0), "=&s"(t1), "=&v"(v)
        : "v"(p)
        : "memory");
    next = v;
    return (uint32_t)(t1 - t0);
}

// One timed returning memory-side atomic (fetch-add of 0: the data is unchanged).
__device__ __forceinline__ uint32_t timed_fetch_add0(uint32_t *p) {
    uint64_t t0, t1;
    uint32_t v;
    asm volatile(
        "s_waitcnt vmcnt(0) lgkmcnt(0)\n\t"
        "s_memtime %0\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "global_atomic_add %2, %3, %4, off sc0\n\t"
        "s_waitcnt vmcnt(0)\n\t"
        "s_memtime %1\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        : "=&s"(t0), "=&s"(t1), "=&v"(v)
        : "v"(p), "v"(0u)
        : "memory");
    return (uint32_t)(t1 - t0) + (v & 0u);
}

// True in exactly one workgroup: the first one found running on XCD `xcd` (claim word
// `claim` must be zero before the launch). Also records the XCC id of the winner.
__device__ __forceinline__ bool claim_role(int xcd, uint32_t *claim, uint32_t *who) {
    __shared__ int won;
    if (threadIdx.x == 0) {
        won = 0;
        if ((int)hw_xcc_id() == xcd && atomicCAS(claim, 0u, 1u) == 0u) {
            won = 1;
            *who = hw_xcc_id();
        }
    }
    __syncthreads();
    return won != 0;
}

// Two chases of the chain by the workgroup that claims XCD `xcd`: lat[0..n) is the first
// (the lines come from wherever they are), lat[n..2n) the second (the lines are now in this
// XCD's L2).
__global__ void __launch_bounds__(64) pchase_role_kernel(const uint64_t *chain, int numel, int xcd, uint32_t *lat,
                                                         uint32_t *claim, uint32_t *who) {
    __shared__ uint32_t sl[kMaxChase];
    if (!claim_role(xcd, claim, who)) return;
    for (int pass = 0; pass < 2; ++pass) {
        if (threadIdx.x == 0) {
            const uint64_t *p = chain;
            for (int i = 0; i < numel; ++i) {
                uint64_t nxt;
                sl[i] = timed_load(p, nxt);
                p = reinterpret_cast<const uint64_t *>(nxt);
            }
        }
        __syncthreads();
        for (int i = (int)threadIdx.x; i < numel; i += (int)blockDim.x) lat[(size_t)pass * numel + i] = sl[i];
        __syncthreads();
    }
}

// MaskProbe: the workgroup that claims XCD `xcd` times, for every bit b in [b0, b1], the
// minimum over `reps` memory-side fetch-adds at buf + 2^b (and at buf itself as entry 0).
__global__ void __launch_bounds__(64) mask_probe_kernel(uint32_t *buf, int b0, int b1, int reps, int xcd,
                                                        uint32_t *lat, uint32_t *claim, uint32_t *who) {
    if (!claim_role(xcd, claim, who)) return;
    if (threadIdx.x != 0) return;
    for (int k = 0; k <= b1 - b0 + 1; ++k) {
        uint32_t *p = k == 0 ? buf : reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(buf) + (1ull << (b0 + k - 1)));
        uint32_t best = 0xffffffffu;
        for (int r = 0; r < reps; ++r) {
            const uint32_t c = timed_fetch_add0(p);
            best = c < best ? c : best;
        }
        lat[k] = best;
    }
}

}  // namespace xd

using namespace xd;

extern "C" {

int xd_xdom_pchase(int leader_xcd, int follower_xcd, void *chain, size_t chain_bytes, int numel, int stride_bytes,
                   const void *flush_buf, size_t flush_bytes, uint32_t *out, void *stream) {
    XD_REQUIRE(chain != nullptr && out != nullptr, "xd_xdom_pchase: NULL chain or out");
    XD_REQUIRE(leader_xcd >= 0 && leader_xcd < kNumXcd && follower_xcd >= 0 && follower_xcd < kNumXcd,
               "xd_xdom_pchase: XCD ids must be in [0, 8)");
    XD_REQUIRE(numel >= 2 && numel <= kMaxChase, "xd_xdom_pchase: numel must be in [2, 8192]");
    XD_REQUIRE(stride_bytes >= 8 && stride_bytes % 8 == 0, "xd_xdom_pchase: stride must be a multiple of 8 bytes");
    XD_REQUIRE((reinterpret_cast<uintptr_t>(chain) & 7u) == 0, "xd_xdom_pchase: chain must be 8-byte aligned");
    XD_REQUIRE((size_t)numel * (size_t)stride_bytes <= chain_bytes, "xd_xdom_pchase: chain buffer too small");
    hipStream_t s = (hipStream_t)stream;
    uint64_t *c = static_cast<uint64_t *>(chain);
    uint32_t *meta = out + 4 * (size_t)numel;  // [leader xcc, follower xcc, claim, claim]
    launch("chase_init_kernel", chase_init_kernel, dim3((numel + 255) / 256), dim3(256), 0, s, c, numel, stride_bytes / 8);
    launch("probe_clear_kernel", probe_clear_kernel, dim3(1), dim3(64), 0, s, meta, 4);
    if (flush_buf) {
        if (int rc = xd_cache_flush(flush_buf, flush_bytes, stream)) return rc;
    }
    // 8 workgroups per XCD so that every XCD surely receives some
    const int grid = 8 * kNumXcd;
    launch("pchase_role_kernel", pchase_role_kernel, dim3(grid), dim3(64), 0, s, c, numel, leader_xcd, out, meta + 2, meta);
    if (int rc = launch_status("pchase_role_kernel")) return rc;
    launch("pchase_role_kernel", pchase_role_kernel, dim3(grid), dim3(64), 0, s, c, numel, follower_xcd, out + 2 * (size_t)numel,
                       meta + 3, meta + 1);
    return launch_status("pchase_role_kernel");
}

int xd_mask_probe(void *buf, size_t bytes, int first_bit, int last_bit, int reps, uint32_t *out, void *stream) {
    XD_REQUIRE(buf != nullptr && out != nullptr, "xd_mask_probe: NULL buffer");
    XD_REQUIRE(first_bit >= 2 && first_bit <= last_bit && last_bit < 40, "xd_mask_probe: bad bit range");
    XD_REQUIRE((1ull << last_bit) + 4 <= bytes, "xd_mask_probe: buffer smaller than 2^last_bit + 4 bytes");
    XD_REQUIRE(reps >= 1 && reps <= 64, "xd_mask_probe: reps must be in [1, 64]");
    hipStream_t s = (hipStream_t)stream;
    const int nb = last_bit - first_bit + 2;  // base address + one entry per bit
    uint32_t *meta = out + 2 * (size_t)nb;    // [die-0 xcc, die-1 xcc, claim, claim]
    launch("probe_clear_kernel", probe_clear_kernel, dim3(1), dim3(64), 0, s, meta, 4);
    const int grid = 8 * kNumXcd;
    // XCD 0 sits on I/O die 0, XCD 4 on die 1
    launch("mask_probe_kernel", mask_probe_kernel, dim3(grid), dim3(64), 0, s, static_cast<uint32_t *>(buf), first_bit, last_bit,
                       reps, 0, out, meta + 2, meta);
    if (int rc = launch_status("mask_probe_kernel")) return rc;
    launch("mask_probe_kernel", mask_probe_kernel, dim3(grid), dim3(64), 0, s, static_cast<uint32_t *>(buf), first_bit, last_bit,
                       reps, kNumXcd / 2, out + nb, meta + 3, meta + 1);
    return launch_status("mask_probe_kernel");
}

}  // extern "C"
