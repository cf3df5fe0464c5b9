// Architecture probes: XDom-PChase (same-XCD vs cross-XCD hit latency of a pointer chase),
// MaskProbe (the address bits that move a line between the two I/O dies) and the channel
// probe (the address bits that select an XCD's L2 channel and, behind it, the memory-side
// channel of a line).
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

#include <algorithm>
#include <functional>
#include <vector>

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

// Placement key of the calling wave's compute unit: (xcc << 16) | (se << 8) | (sh << 4) | cu,
// the fields of an xd_domain_scan word shifted right by 8 (the SIMD dropped).
__device__ __forceinline__ uint32_t cu_key() {
    const uint32_t hw = hw_id_word();
    return (hw_xcc_id() << 16) | (((hw >> 13) & 0x7u) << 8) | (((hw >> 12) & 0x1u) << 4) | ((hw >> 8) & 0xfu);
}

// DomainScan latency curves, leader half: the first workgroup on XCD `xcd` loads base + 2^b
// for b in [b0, b1] (the lines land in that XCD's L2 and in the Infinity Cache).
__global__ void __launch_bounds__(64) scan_leader_kernel(const char *base, int b0, int b1, int xcd, uint32_t *claim,
                                                         uint32_t *who) {
    if (!claim_role(xcd, claim, who)) return;
    if (threadIdx.x != 0) return;
    uint64_t acc = 0;
    for (int b = b0; b <= b1; ++b) {
        uint64_t v;
        asm volatile("global_load_dwordx2 %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(base + (1ull << b)) : "memory");
        acc ^= v;
    }
    asm volatile("" ::"v"(acc));
}

// Follower half: the first workgroup running on compute unit `key` (cu_key) times one load of
// each of the leader's addresses, in the leader's order.
__global__ void __launch_bounds__(64) scan_follower_kernel(const char *base, int b0, int b1, uint32_t key,
                                                           uint32_t *lat, uint32_t *claim) {
    __shared__ int won;
    if (threadIdx.x == 0) won = cu_key() == key && atomicCAS(claim, 0u, 1u) == 0u;
    __syncthreads();
    if (!won || threadIdx.x != 0) return;
    for (int b = b0; b <= b1; ++b) {
        uint64_t next;
        lat[b - b0] = timed_load(reinterpret_cast<const uint64_t *>(base + (1ull << b)), next);
    }
}

// Channel probe (MaskProbe for the bits that select an L2 channel of an XCD, and behind the
// L2 the memory-side channel of a line). A query times one set of 64 lines: lane i of every
// wave reads base + (XOR of v[k] over the set bits k of i), so the set is the affine span of
// six address vectors. Every workgroup on XCD `xcd` (one wave each; the others leave at once)
// reads the set `iters` times. A channel serves its lines one after another, so the launch
// time is proportional to the largest number of the set's lines that share a channel: if the
// channel is a GF(2)-linear function H of the address bits (an XOR hash), the set covers
// 2^rank(H v) channels and the time is T_fast * 2^(rank_max - rank). The search below reads
// H off such times. The loads skip the vector L1 (sc1) and hit this XCD's L2 after the first
// pass. (Memory-side atomics and loads of uncached memory cross the same L2 channels, which
// stay the first bottleneck at this rate, so the channels behind the L2 are not separable
// from one XCD this way.)
constexpr int kChanLanes = 64;
constexpr int kChanWgsPerXcd = 128;
constexpr uint64_t kChanPage = 2ull << 20;  // 2 MiB: the bits below it are virtual = physical

struct ChanSet {
    uint64_t v[6];
};

__global__ void __launch_bounds__(kChanLanes) channel_load_kernel(const char *base, ChanSet set, int iters, int xcd) {
    if ((int)hw_xcc_id() != xcd) return;
    const uint32_t lane = threadIdx.x;
    uint64_t off = 0;
#pragma unroll
    for (int k = 0; k < 6; ++k) off ^= ((lane >> k) & 1u) ? set.v[k] : 0ull;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(base + off);
    uint32_t acc = 0;
    for (int it = 0; it < iters; it += 4) {
        uint32_t v0, v1, v2, v3;  // four requests per lane in flight
        asm volatile(
            "global_load_dword %0, %4, off sc1\n\t"
            "global_load_dword %1, %4, off sc1\n\t"
            "global_load_dword %2, %4, off sc1\n\t"
            "global_load_dword %3, %4, off sc1\n\t"
            "s_waitcnt vmcnt(0)"
            : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
            : "v"(p)
            : "memory");
        acc ^= v0 ^ v1 ^ v2 ^ v3;
    }
    asm volatile("" ::"v"(acc));
}

struct ChanProbe {
    const char *base;
    int xcd, iters;
    hipStream_t s;
    hipEvent_t e0 = nullptr, e1 = nullptr;

    // Microseconds of one set: the minimum of three launches after a warming one.
    int time(const ChanSet &set, float *us) {
        const dim3 grid(kChanWgsPerXcd * kNumXcd);
        float best = 1e30f;
        for (int r = 0; r < 4; ++r) {
            XD_HIP(hipEventRecord(e0, s));
            launch(nullptr, channel_load_kernel, grid, dim3(kChanLanes), 0, s, base, set, iters, xcd);
            if (int rc = launch_status("channel_load_kernel")) return rc;
            XD_HIP(hipEventRecord(e1, s));
            XD_HIP(hipEventSynchronize(e1));
            float ms = 0.0f;
            XD_HIP(hipEventElapsedTime(&ms, e0, e1));
            if (r > 0 && ms * 1000.0f < best) best = ms * 1000.0f;
        }
        *us = best;
        return XD_OK;
    }
};

// Validates the arguments common to both entry points and resolves the base of the probed
// region: the caller's buffer rounded up to 2 MiB. `span` = one past the largest offset + 4.
static int chan_setup(void *buf, size_t bytes, int xcd, int iters, uint64_t span, ChanProbe *p, void *stream) {
    XD_REQUIRE(buf != nullptr, "channel probe: NULL buffer");
    XD_REQUIRE(xcd >= 0 && xcd < kNumXcd, "channel probe: xcd must be in [0, 8)");
    XD_REQUIRE(iters >= 4 && iters <= (1 << 20) && iters % 4 == 0,
               "channel probe: iters must be a multiple of 4 in [4, 2^20]");
    const uintptr_t a = reinterpret_cast<uintptr_t>(buf);
    const uintptr_t base = (a + kChanPage - 1) & ~(uintptr_t)(kChanPage - 1);
    XD_REQUIRE(span <= bytes && base - a <= bytes - span,
               "channel probe: buffer must hold the probed span after rounding its start up to 2 MiB");
    p->base = reinterpret_cast<const char *>(base);
    p->xcd = xcd;
    p->iters = iters;
    p->s = (hipStream_t)stream;
    XD_HIP(hipEventCreate(&p->e0));
    XD_HIP(hipEventCreate(&p->e1));
    return XD_OK;
}

static void chan_release(ChanProbe *p) {
    if (p->e0) (void)hipEventDestroy(p->e0);
    if (p->e1) (void)hipEventDestroy(p->e1);
}

// Adds `m` to a GF(2) basis kept in reduced form by leading bit; false when m is already in
// its span.
static bool gf2_insert(uint64_t *basis, int *n, uint64_t m) {
    for (int i = 0; i < *n; ++i) {
        const uint64_t lead = 1ull << (63 - __builtin_clzll(basis[i]));
        if (m & lead) m ^= basis[i];
    }
    if (m == 0) return false;
    basis[(*n)++] = m;
    // keep the basis sorted by leading bit, descending, so the reduction above stays valid
    for (int i = *n - 1; i > 0 && __builtin_clzll(basis[i]) < __builtin_clzll(basis[i - 1]); --i) {
        const uint64_t t = basis[i];
        basis[i] = basis[i - 1];
        basis[i - 1] = t;
    }
    return true;
}

// Memory-side channel probe. Beyond the L2 a line is served by one of many memory-side units
// (Infinity-Cache slice / HBM channel); a returning atomic has to reach it. Every workgroup
// of a 2048-wave grid (all XCDs) adds 1 to the same 64 lines, spanned by six address vectors
// as above, wave w at dword (w mod 16) * 8 of each line (so that no single address serialises
// the launch); the launch time then tracks the largest number of the set's lines that share
// a unit: 790, 1402, 2800, 5596 us for image ranks 6, 5, 4, 3 at 64 iterations (a rank lost
// doubles it). The adds change the buffer. (An add of 0 with an unused result is idempotent
// and may become a plain load, which stops at the L2: the probe must add a non-zero value.)
constexpr int kMemWaves = 2048;

__global__ void __launch_bounds__(kChanLanes) memchannel_add_kernel(char *base, ChanSet set, int iters) {
    const uint32_t lane = threadIdx.x;
    uint64_t off = 0;
#pragma unroll
    for (int k = 0; k < 6; ++k) off ^= ((lane >> k) & 1u) ? set.v[k] : 0ull;
    off += (uint64_t)(blockIdx.x % 16u) * 8u;
    unsigned long long *p = reinterpret_cast<unsigned long long *>(base + off);
    for (int it = 0; it < iters; ++it) atomicAdd(p, 1ull);
}

struct MemProbe {
    char *base;
    int iters;
    hipStream_t s;
    hipEvent_t e0 = nullptr, e1 = nullptr;

    // Microseconds of one set: the minimum of two launches after a warming one.
    int time(const ChanSet &set, float *us) {
        float best = 1e30f;
        for (int r = 0; r < 3; ++r) {
            XD_HIP(hipEventRecord(e0, s));
            launch(nullptr, memchannel_add_kernel, dim3(kMemWaves), dim3(kChanLanes), 0, s, base, set, iters);
            if (int rc = launch_status("memchannel_add_kernel")) return rc;
            XD_HIP(hipEventRecord(e1, s));
            XD_HIP(hipEventSynchronize(e1));
            float ms = 0.0f;
            XD_HIP(hipEventElapsedTime(&ms, e0, e1));
            if (r > 0 && ms * 1000.0f < best) best = ms * 1000.0f;
        }
        *us = best;
        return XD_OK;
    }
};

// Base of the memory-side probe: buf rounded up to 2 MiB; span = largest line offset + 128
// (the dword offsets stay inside the line).
static int mem_setup(void *buf, size_t bytes, int iters, uint64_t span, MemProbe *p, void *stream) {
    XD_REQUIRE(buf != nullptr, "memory channel probe: NULL buffer");
    XD_REQUIRE(iters >= 1 && iters <= (1 << 16), "memory channel probe: iters must be in [1, 2^16]");
    const uintptr_t a = reinterpret_cast<uintptr_t>(buf);
    const uintptr_t base = (a + kChanPage - 1) & ~(uintptr_t)(kChanPage - 1);
    XD_REQUIRE(span <= bytes && base - a <= bytes - span,
               "memory channel probe: buffer must hold the probed span after rounding its start up to 2 MiB");
    p->base = reinterpret_cast<char *>(base);
    p->iters = iters;
    p->s = (hipStream_t)stream;
    XD_HIP(hipEventCreate(&p->e0));
    XD_HIP(hipEventCreate(&p->e1));
    return XD_OK;
}

static void mem_release(MemProbe *p) {
    if (p->e0) (void)hipEventDestroy(p->e0);
    if (p->e1) (void)hipEventDestroy(p->e1);
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

int xd_domain_scan_latency(void *buf, size_t bytes, int first_bit, int last_bit, int leader_xcd, uint32_t follower_cu,
                           const void *flush_buf, size_t flush_bytes, uint32_t *out, void *stream) {
    XD_REQUIRE(buf != nullptr && out != nullptr, "xd_domain_scan_latency: NULL buf or out");
    XD_REQUIRE(first_bit >= 3 && first_bit <= last_bit && last_bit < 40, "xd_domain_scan_latency: bad bit range");
    XD_REQUIRE((reinterpret_cast<uintptr_t>(buf) & 7u) == 0, "xd_domain_scan_latency: buf must be 8-byte aligned");
    XD_REQUIRE((1ull << last_bit) + 8 <= bytes, "xd_domain_scan_latency: buffer smaller than 2^last_bit + 8 bytes");
    XD_REQUIRE(leader_xcd >= 0 && leader_xcd < kNumXcd, "xd_domain_scan_latency: leader_xcd must be in [0, 8)");
    XD_REQUIRE((follower_cu >> 16) < (uint32_t)kNumXcd, "xd_domain_scan_latency: follower_cu names no XCD");
    hipStream_t s = (hipStream_t)stream;
    const int nb = last_bit - first_bit + 1;
    uint32_t *meta = out + nb;  // [leader found, follower found, leader xcc, unused]
    const char *base = static_cast<const char *>(buf);
    launch("probe_clear_kernel", probe_clear_kernel, dim3(1), dim3(64), 0, s, meta, 4);
    if (flush_buf) {
        if (int rc = xd_cache_flush(flush_buf, flush_bytes, stream)) return rc;
    }
    // 4 workgroups per compute unit: every CU of every XCD receives at least one
    const int grid = 4 * 32 * kNumXcd;
    launch("scan_leader_kernel", scan_leader_kernel, dim3(grid), dim3(64), 0, s, base, first_bit, last_bit, leader_xcd,
           meta, meta + 2);
    if (int rc = launch_status("scan_leader_kernel")) return rc;
    launch("scan_follower_kernel", scan_follower_kernel, dim3(grid), dim3(64), 0, s, base, first_bit, last_bit,
           follower_cu, out, meta + 1);
    return launch_status("scan_follower_kernel");
}

int xd_channel_time(void *buf, size_t bytes, int xcd, const uint64_t *vecs, int iters, float *out_us, void *stream) {
    XD_REQUIRE(vecs != nullptr && out_us != nullptr, "xd_channel_time: NULL vecs or out_us");
    ChanSet set;
    uint64_t reach = 0;
    for (int k = 0; k < 6; ++k) {
        XD_REQUIRE((vecs[k] & 127u) == 0 && vecs[k] < (1ull << 40),
                   "xd_channel_time: vectors must be multiples of 128 bytes below 2^40");
        set.v[k] = vecs[k];
        reach |= vecs[k];  // every XOR of the vectors is at most their OR
    }
    ChanProbe p;
    int rc = chan_setup(buf, bytes, xcd, iters, reach + 4, &p, stream);
    if (rc == XD_OK) rc = p.time(set, out_us);
    chan_release(&p);
    return rc;
}

int xd_channel_probe(void *buf, size_t bytes, int xcd, int bit0, int bit1, int iters, int max_sets,
                     float *out_window_us, float *out_fast_us, uint64_t *out_masks, float *out_curves, int *out_nmasks,
                     void *stream) {
    XD_REQUIRE(out_window_us && out_fast_us && out_masks && out_curves && out_nmasks, "xd_channel_probe: NULL output");
    XD_REQUIRE(bit0 >= 7 && bit1 - bit0 >= 6 && bit1 < 34, "xd_channel_probe: need 7 <= bit0, bit0 + 6 <= bit1 < 34");
    XD_REQUIRE(max_sets >= 1 && max_sets <= 4096, "xd_channel_probe: max_sets must be in [1, 4096]");
    const int nb = bit1 - bit0 + 1;
    ChanProbe p;
    // the largest offset: every line-granular bit from 7 to bit1 set
    int rc = chan_setup(buf, bytes, xcd, iters, (2ull << bit1) - 128 + 4, &p, stream);
    *out_nmasks = 0;
    // 1. windows: six consecutive bits b..b+5
    float fast = 1e30f;
    for (int b = bit0; b + 5 <= bit1 && rc == XD_OK; ++b) {
        ChanSet w;
        for (int k = 0; k < 6; ++k) w.v[k] = 1ull << (b + k);
        rc = p.time(w, &out_window_us[b - bit0]);
        if (rc == XD_OK) fast = std::min(fast, out_window_us[b - bit0]);
    }
    // 2. five-bit sets F in a fixed pseudo-random order. With H(F) of rank r, adding bit f
    // gives 64 lines on 2^(r+1) channels when H e_f lies outside the span of H(F) and on 2^r
    // when inside. For r = rank_max - 1 the times sit at T_fast and 2 T_fast, and the bits
    // at T_fast are exactly those with phi(e_f) = 1 for the one linear function phi (an XOR
    // of address bits, i.e. one channel-select bit up to relabelling) that vanishes on H(F):
    // its mask is read off directly. Sets of any other rank show other levels and are skipped.
    uint64_t basis[4];
    int nbasis = 0;
    uint32_t lcg = 0x2545F491u;
    std::vector<float> curve(nb);
    for (int t = 0; t < max_sets && rc == XD_OK && *out_nmasks < 4; ++t) {
        uint64_t fbits = 0;
        int picked = 0;
        while (picked < 5) {
            lcg = lcg * 1664525u + 1013904223u;
            const int bit = bit0 + (int)((lcg >> 8) % (uint32_t)nb);
            if (!(fbits >> bit & 1)) {
                fbits |= 1ull << bit;
                ++picked;
            }
        }
        ChanSet q;
        int k = 0;
        for (int bit = bit0; bit <= bit1; ++bit)
            if (fbits >> bit & 1) q.v[k++] = 1ull << bit;
        float lo = 1e30f, hi = 0.0f;
        for (int f = bit0; f <= bit1 && rc == XD_OK; ++f) {
            curve[f - bit0] = 0.0f;
            if (fbits >> f & 1) continue;
            q.v[5] = 1ull << f;
            rc = p.time(q, &curve[f - bit0]);
            lo = std::min(lo, curve[f - bit0]);
            hi = std::max(hi, curve[f - bit0]);
        }
        if (rc != XD_OK) break;
        fast = std::min(fast, lo);
        if (!(lo < 1.25f * fast && hi > 1.6f * fast && hi < 2.6f * fast)) continue;
        // two clean levels only: a time between them (lines of the set partly conflicting
        // elsewhere) makes the set ambiguous
        bool clean = true;
        uint64_t mask = 0;
        for (int f = bit0; f <= bit1; ++f) {
            const float c = curve[f - bit0];
            if (c <= 0.0f) continue;
            if (c > 1.25f * fast && c < 1.6f * fast) clean = false;
            if (c <= 1.25f * fast) mask |= 1ull << f;
        }
        if (!clean) continue;
        if (!gf2_insert(basis, &nbasis, mask)) continue;
        out_masks[*out_nmasks] = mask;
        std::copy(curve.begin(), curve.end(), out_curves + (size_t)(*out_nmasks) * nb);
        ++*out_nmasks;
    }
    *out_fast_us = fast;
    chan_release(&p);
    return rc;
}

int xd_memchannel_time(void *buf, size_t bytes, const uint64_t *vecs, int iters, float *out_us, void *stream) {
    XD_REQUIRE(vecs != nullptr && out_us != nullptr, "xd_memchannel_time: NULL vecs or out_us");
    ChanSet set;
    uint64_t reach = 0;
    for (int k = 0; k < 6; ++k) {
        XD_REQUIRE((vecs[k] & 127u) == 0 && vecs[k] < (1ull << 40),
                   "xd_memchannel_time: vectors must be multiples of 128 bytes below 2^40");
        set.v[k] = vecs[k];
        reach |= vecs[k];
    }
    MemProbe p;
    int rc = mem_setup(buf, bytes, iters, reach + 128, &p, stream);
    if (rc == XD_OK) rc = p.time(set, out_us);
    mem_release(&p);
    return rc;
}

int xd_memchannel_probe(void *buf, size_t bytes, int bit0, int bit1, int iters, int nsets, float *out_ratio,
                        uint64_t *out_inactive, uint64_t *out_masks, int *out_nmasks, void *stream) {
    XD_REQUIRE(out_ratio && out_inactive && out_masks && out_nmasks, "xd_memchannel_probe: NULL output");
    XD_REQUIRE(bit0 >= 7 && bit1 - bit0 >= 6 && bit1 < 34 && bit1 - bit0 < 32,
               "xd_memchannel_probe: need 7 <= bit0, bit0 + 6 <= bit1 < 34, at most 32 bits");
    XD_REQUIRE(nsets >= 1 && nsets <= 64, "xd_memchannel_probe: nsets must be in [1, 64]");
    const int nb = bit1 - bit0 + 1;
    MemProbe p;
    int rc = mem_setup(buf, bytes, iters, (2ull << bit1) - 128 + 128, &p, stream);
    // Test vectors: every bit and every pair of bits. A vector x "adds" against a five-vector
    // set F when F + x spans one more unit dimension than F: its time is then the lowest of
    // F's curve, one level (2x) faster than a vector that adds nothing. x never changes the
    // unit (x is in the kernel of the map) when it adds against none of the sets.
    // out_ratio[a * nb + b] (a <= b; a == b: the single bit) = min over the sets of
    // time(F + x) / lowest time of F's curve; above ~1.4 means "never adds".
    std::vector<uint64_t> tests;
    std::vector<int> ta, tb;
    for (int a = 0; a < nb; ++a)
        for (int b = a; b < nb; ++b) {
            tests.push_back((1ull << (bit0 + a)) | (1ull << (bit0 + b)));
            ta.push_back(a);
            tb.push_back(b);
        }
    std::vector<float> best(tests.size(), 1e30f), t(tests.size());
    uint32_t lcg = 0x9E3779B9u;
    for (int f = 0; f < nsets && rc == XD_OK; ++f) {
        ChanSet q;
        for (int k = 0; k < 5; ++k) {  // XOR of two distinct bits each
            lcg = lcg * 1664525u + 1013904223u;
            const int a = (int)((lcg >> 8) % (uint32_t)nb);
            lcg = lcg * 1664525u + 1013904223u;
            int b = (int)((lcg >> 8) % (uint32_t)(nb - 1));
            b += b >= a ? 1 : 0;
            q.v[k] = (1ull << (bit0 + a)) | (1ull << (bit0 + b));
        }
        float lo = 1e30f;
        for (size_t i = 0; i < tests.size() && rc == XD_OK; ++i) {
            q.v[5] = tests[i];
            rc = p.time(q, &t[i]);
            lo = std::min(lo, t[i]);
        }
        if (rc != XD_OK) break;
        for (size_t i = 0; i < tests.size(); ++i) best[i] = std::min(best[i], t[i] / lo);
    }
    mem_release(&p);
    if (rc != XD_OK) return rc;
    for (int i = 0; i < nb * nb; ++i) out_ratio[i] = 0.0f;
    for (size_t i = 0; i < tests.size(); ++i) out_ratio[ta[i] * nb + tb[i]] = best[i];
    // inactive bits: never change the unit; classes: active bits joined by pairs in the kernel
    // (two bits whose images are equal), each class's indicator one XOR mask of the map
    uint64_t inactive = 0;
    for (int a = 0; a < nb; ++a)
        if (out_ratio[a * nb + a] > 1.4f) inactive |= 1ull << (bit0 + a);
    std::vector<int> cls(nb);
    for (int a = 0; a < nb; ++a) cls[a] = a;
    std::function<int(int)> root = [&](int a) { return cls[a] == a ? a : (cls[a] = root(cls[a])); };
    for (int a = 0; a < nb; ++a)
        for (int b = a + 1; b < nb; ++b)
            if (!(inactive >> (bit0 + a) & 1) && !(inactive >> (bit0 + b) & 1) && out_ratio[a * nb + b] > 1.4f)
                cls[root(b)] = root(a);
    int nm = 0;
    for (int a = 0; a < nb && nm < 32; ++a) {
        if ((inactive >> (bit0 + a) & 1) || root(a) != a) continue;
        uint64_t m = 0;
        for (int b = 0; b < nb; ++b)
            if (!(inactive >> (bit0 + b) & 1) && root(b) == a) m |= 1ull << (bit0 + b);
        out_masks[nm++] = m;
    }
    *out_inactive = inactive;
    *out_nmasks = nm;
    return XD_OK;
}

}  // extern "C"
