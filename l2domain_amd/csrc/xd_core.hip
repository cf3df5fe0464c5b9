// Library core: error state, topology, DomainScan and the cache-flush kernel.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "xd_common.hpp"

namespace xd {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    g_last_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    return XD_ERR_HIP;
}

// One pass counter per device for XD_MODE_ROTATED. Returns the rotation for the first of
// `passes` consecutive passes and advances the counter past them.
static std::atomic<unsigned> g_rotation[64];

unsigned next_rotation(int passes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    return g_rotation[dev].fetch_add((unsigned)passes) + 1u;
}

// ---- placement hints: one pinned word per (device, stream), written by workgroup 0 of every
// dispatch that takes a hint, read by the next launch on the stream ----
namespace {
std::mutex g_hint_mu;
std::map<std::pair<int, uintptr_t>, uint32_t *> g_hint_slots;
uint32_t *g_hint_block = nullptr;
int g_hint_used = 0;
constexpr int kHintBlockWords = 1024;      // one 4 KiB pinned block per 1024 streams
constexpr size_t kMaxHintSlots = 16384;    // streams beyond this get no slot (offset 0)
}  // namespace

static uint32_t *hint_slot(hipStream_t s, bool create) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_hint_mu);
    const auto key = std::make_pair(dev, reinterpret_cast<uintptr_t>(s));
    const auto it = g_hint_slots.find(key);
    if (it != g_hint_slots.end()) return it->second;
    if (!create || g_hint_slots.size() >= kMaxHintSlots) return nullptr;
    if (g_hint_block == nullptr || g_hint_used == kHintBlockWords) {
        void *p = nullptr;
        if (hipHostMalloc(&p, kHintBlockWords * sizeof(uint32_t), hipHostMallocCoherent) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        std::memset(p, 0, kHintBlockWords * sizeof(uint32_t));
        g_hint_block = static_cast<uint32_t *>(p);
        g_hint_used = 0;
    }
    uint32_t *w = g_hint_block + g_hint_used++;
    g_hint_slots.emplace(key, w);
    return w;
}

static XcdHint hint_of(uint32_t *w) {
    const uint32_t v = w ? __atomic_load_n(w, __ATOMIC_RELAXED) : 0u;
    return XcdHint{(v & 0x100u) ? (v & (kNumXcd - 1u)) : 0u, w};
}

XcdHint xcd_hint(hipStream_t stream) { return hint_of(hint_slot(stream, true)); }
XcdHint xcd_hint_noalloc(hipStream_t stream) { return hint_of(hint_slot(stream, false)); }

static std::atomic<uint64_t> g_home_mask{kDefaultHomeMask};
uint64_t home_mask() { return g_home_mask.load(std::memory_order_relaxed); }

// ---- opt-in kernel timing ----
struct TimingRec {
    std::string name;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
    double total_ms = 0.0;
    long long launches = 0;
};
static std::mutex g_tmu;
static std::atomic<bool> g_timing{false};
static std::vector<TimingRec> g_recs;

bool timing_enabled() { return g_timing.load(std::memory_order_relaxed); }

void timing_record(const char *kernel, hipEvent_t start, hipEvent_t stop) {
    std::lock_guard<std::mutex> lk(g_tmu);
    for (auto &r : g_recs)
        if (r.name == kernel) {
            r.pending.emplace_back(start, stop);
            return;
        }
    g_recs.push_back(TimingRec{kernel, {{start, stop}}, 0.0, 0});
}

static void timing_drain_locked() {
    for (auto &r : g_recs) {
        for (auto &p : r.pending) {
            float ms = 0.0f;
            if (hipEventSynchronize(p.second) == hipSuccess && hipEventElapsedTime(&ms, p.first, p.second) == hipSuccess) {
                r.total_ms += ms;
                r.launches += 1;
            }
            (void)hipEventDestroy(p.first);
            (void)hipEventDestroy(p.second);
        }
        r.pending.clear();
    }
}

// DomainScan: every workgroup records where the hardware placed it.
__global__ void domain_scan_kernel(uint32_t *out, int num_wg) {
    if (threadIdx.x != 0) return;
    uint32_t xcc = hw_xcc_id();
    uint32_t hw = hw_id_word();
    uint32_t simd = (hw >> 4) & 0x3u;
    uint32_t cu = (hw >> 8) & 0xfu;
    uint32_t sh = (hw >> 12) & 0x1u;
    uint32_t se = (hw >> 13) & 0x7u;
    int wg = (int)blockIdx.x;
    if (wg < num_wg) out[wg] = (xcc << 24) | (se << 16) | (sh << 12) | (cu << 8) | simd;
}

// Streams `n16` 16-byte words with ordinary (allocating) loads, so that the flush data
// replaces what the L2s and the memory-side Infinity Cache held (non-temporal loads would
// not allocate in the Infinity Cache and leave it warm); the loaded values feed an asm sink
// so that the loads stay.
__global__ void __launch_bounds__(256) cache_flush_kernel(const u32x4 *buf, size_t n16) {
    uint32_t acc = 0;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        u32x4 v = buf[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    asm volatile("" ::"v"(acc));
}

// Read stream: every 16-byte word of a buffer loaded once, the roofline probe of
// cache-resident workloads (a warm GEMV's matrix). Oblivious: contiguous grid-stride.
// Aware: each 16 KiB pair of 8 KiB chunks holds one chunk homed on either I/O die, and the
// workgroups of a die load only the chunk their die homes (rotated: only the other one), four
// pairs in flight per workgroup. The loaded words feed an asm sink so that the loads stay.
constexpr int kStreamThreads = 256;

template <int kStreamPairsInFlight>
__global__ void __launch_bounds__(kStreamThreads)
read_stream_kernel(const u32x4 *buf, uint64_t nvec, uint64_t npairs, int mode, HomeMap home, XcdHint xh) {
    report_xcd(xh);
    __shared__ uint8_t lattr[2048];  // the buffer's home map (buffers up to 4 GiB)
    const StagedHome hs = stage_home_nosync(home, reinterpret_cast<uint64_t>(buf), nvec * 16, lattr, 2048,
                                            mode != XD_MODE_OBLIVIOUS && npairs != 0);
    __syncthreads();
    uint32_t acc = 0;
    if (mode == XD_MODE_OBLIVIOUS || npairs == 0) {
        const uint64_t stride = (uint64_t)gridDim.x * kStreamThreads;
        uint64_t i = (uint64_t)blockIdx.x * kStreamThreads + threadIdx.x;
        constexpr int D = 2 * kStreamPairsInFlight;  // loads in flight per thread
        for (; i + (D - 1) * stride < nvec; i += D * stride) {
            u32x4 v[D];
#pragma unroll
            for (int k = 0; k < D; ++k) v[k] = buf[i + (uint64_t)k * stride];
#pragma unroll
            for (int k = 0; k < D; ++k) acc ^= v[k].x ^ v[k].w;
        }
        for (; i < nvec; i += stride) acc ^= buf[i].x;
    } else {
        const int b = (int)blockIdx.x;
        const uint64_t per_die = gridDim.x / 2;
        const uint64_t rank = (uint64_t)die_rank(b, xh);
        const uint32_t want = mode == XD_MODE_AWARE ? wg_die(b, xh) : (wg_die(b, xh) ^ 1u);
        const uint64_t base = reinterpret_cast<uint64_t>(buf);
        constexpr uint64_t kChunkVec = kHomeChunk / 16;  // 512 vectors, two per thread
        for (uint64_t p0 = rank; p0 < npairs; p0 += per_die * kStreamPairsInFlight) {
            u32x4 v[2 * kStreamPairsInFlight];
#pragma unroll
            for (int k = 0; k < kStreamPairsInFlight; ++k) {
                uint64_t p = p0 + (uint64_t)k * per_die;
                p = p < npairs ? p : npairs - 1;  // past the end: re-read the last pair
                const uint64_t c = 2 * p + (hs(base + 2 * p * kHomeChunk) ^ want);
                v[2 * k] = buf[c * kChunkVec + threadIdx.x];
                v[2 * k + 1] = buf[c * kChunkVec + kStreamThreads + threadIdx.x];
            }
#pragma unroll
            for (int k = 0; k < 2 * kStreamPairsInFlight; ++k) acc ^= v[k].x ^ v[k].w;
        }
    }
    asm volatile("" ::"v"(acc));
}

// ---- home map (MaskProbe) ----
// Round trip of one memory-side atomic (fetch-add of 0: the word is unchanged), in shader
// cycles. On gfx950 every global atomic is executed beyond the XCD's L2, so the time
// reflects the path from the issuing XCD to the die that homes the line, never an L2 hit.
__device__ __forceinline__ uint64_t timed_atomic_cycles(uint32_t *p) {
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
    return (t1 - t0) + (v & 0u);
}

constexpr int kHomeProbeLines = 4;     // probe words per page: offsets 0, 16, 32, 48 KiB (bit 13 = 0)
constexpr int kHomeProbeWgsPerXcd = 16;

// Probe word `k` of 2 MiB page `p` (counted from the 2 MiB boundary at or below buf).
__device__ __forceinline__ uint32_t *home_probe_word(uint64_t page0, uint64_t p, int k, uint64_t lo, uint64_t hi) {
    uint64_t a = (page0 + p) * kHomePage + (uint64_t)k * 16384;
    if (a < lo) a = (lo + 16383) & ~(uint64_t)16383;  // first page may start inside the buffer
    if (a + 4 > hi) return nullptr;
    return reinterpret_cast<uint32_t *>(a);
}

// Workgroups on XCD 2 load the probe words first, so that both timed passes find the lines
// in the Infinity Cache rather than one of them paying the HBM miss. (Roles by the XCD read
// from the hardware; workgroup b of each XCD takes pages b / 8, b / 8 + W, ...: with the
// round-robin dispatch every XCD holds one workgroup of each b / 8.)
__global__ void home_touch_kernel(uint64_t page0, uint64_t npages, uint64_t lo, uint64_t hi, uint32_t *sink) {
    const int b = (int)blockIdx.x;
    if (hw_xcc_id() != 2u || threadIdx.x != 0) return;
    uint32_t acc = 0;
    for (uint64_t p = (uint64_t)(b / kNumXcd); p < npages; p += kHomeProbeWgsPerXcd)
        for (int k = 0; k < kHomeProbeLines; ++k) {
            const uint32_t *q = home_probe_word(page0, p, k, lo, hi);
            if (q) acc += __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    if (acc == 0x5bd1e995u) sink[0] = acc;
}

// Workgroups on XCD 0 (die 0), then in a second launch on XCD 4 (die 1), time atomics on the
// same words; the page is homed on the die that completes them faster.
__global__ void home_measure_kernel(uint64_t page0, uint64_t npages, uint64_t lo, uint64_t hi, uint32_t *lat,
                                    int die) {
    const int b = (int)blockIdx.x;
    if (hw_xcc_id() != (uint32_t)(4 * die) || threadIdx.x != 0) return;
    for (uint64_t p = (uint64_t)(b / kNumXcd); p < npages; p += kHomeProbeWgsPerXcd) {
        uint32_t best = 0xffffffffu;
        for (int k = 0; k < kHomeProbeLines; ++k) {
            uint32_t *q = home_probe_word(page0, p, k, lo, hi);
            if (q) {
                const uint64_t c = timed_atomic_cycles(q);
                if (c < best) best = (uint32_t)c;
            }
        }
        lat[2 * p + die] = best;
    }
}

__global__ void home_classify_kernel(const uint32_t *lat, uint64_t npages, uint8_t *attr) {
    for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < npages; p += (uint64_t)gridDim.x * blockDim.x)
        attr[p] = lat[2 * p + 1] < lat[2 * p] ? 1 : 0;
}

}  // namespace xd

using namespace xd;

extern "C" {

const char *xd_version(void) { return "xdom 0.1.0 (gfx950)"; }

const char *xd_last_error(void) { return g_last_error.c_str(); }

int xd_timing_enable(int on) {
    std::lock_guard<std::mutex> lk(g_tmu);
    timing_drain_locked();
    g_recs.clear();
    g_timing.store(on != 0);
    return XD_OK;
}

int xd_timing_query(int index, char *name, int name_len, double *total_ms, long long *launches) {
    std::lock_guard<std::mutex> lk(g_tmu);
    timing_drain_locked();
    if (index < 0 || index >= (int)g_recs.size()) return XD_ERR_INVALID_ARG;
    const TimingRec &r = g_recs[(size_t)index];
    if (name && name_len > 0) std::snprintf(name, (size_t)name_len, "%s", r.name.c_str());
    if (total_ms) *total_ms = r.total_ms;
    if (launches) *launches = r.launches;
    return XD_OK;
}

int xd_topology_query(int device, xd_topology_t *out) {
    XD_REQUIRE(out != nullptr, "xd_topology_query: out is NULL");
    hipDeviceProp_t prop;
    XD_HIP(hipGetDeviceProperties(&prop, device));
    std::memset(out, 0, sizeof(*out));
    out->device = device;
    out->num_cu = prop.multiProcessorCount;
    int xcc = 0;
    if (hipDeviceGetAttribute(&xcc, hipDeviceAttributeNumberOfXccs, device) != hipSuccess || xcc <= 0) {
        (void)hipGetLastError();
        xcc = 1;
    }
    out->num_xcd = xcc;
    out->cu_per_xcd = xcc > 0 ? prop.multiProcessorCount / xcc : prop.multiProcessorCount;
    out->wave_size = prop.warpSize;
    out->clock_khz = prop.clockRate;
    out->l2_bytes = prop.l2CacheSize;
    out->lds_bytes_per_wg = (long long)prop.sharedMemPerBlock;
    out->hbm_bytes = (long long)prop.totalGlobalMem;
    std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
    // the marketing name comes from a table the driver may not ship; fall back to the ISA
    if (prop.name[0]) std::snprintf(out->name, sizeof(out->name), "%s", prop.name);
    else std::snprintf(out->name, sizeof(out->name), "AMD Instinct %s", prop.gcnArchName);
    return XD_OK;
}

int xd_domain_scan(int num_wg, uint32_t *out_placement, void *stream) {
    XD_REQUIRE(num_wg > 0 && num_wg <= (1 << 24), "xd_domain_scan: num_wg out of range");
    XD_REQUIRE(out_placement != nullptr, "xd_domain_scan: out_placement is NULL");
    launch("domain_scan_kernel", domain_scan_kernel, dim3(num_wg), dim3(64), 0, (hipStream_t)stream,
                       out_placement, num_wg);
    return launch_status("domain_scan_kernel");
}

int xd_xcd_offset(void *stream) {
    uint32_t *w = hint_slot(static_cast<hipStream_t>(stream), false);
    const uint32_t v = w ? __atomic_load_n(w, __ATOMIC_RELAXED) : 0u;
    return (v & 0x100u) ? (int)(v & (kNumXcd - 1u)) : -1;
}

uint64_t xd_home_mask(void) { return home_mask(); }

int xd_set_home_mask(uint64_t mask) {
    XD_REQUIRE(mask != 0 && (mask & (kHomeChunk - 1)) == 0,
               "xd_set_home_mask: mask must be non-zero and select bits at or above bit 13");
    g_home_mask.store(mask);
    return XD_OK;
}

size_t xd_home_map_pages(const void *buf, size_t bytes) {
    if (buf == nullptr || bytes == 0) return 0;
    const uint64_t lo = reinterpret_cast<uint64_t>(buf);
    return (size_t)(((lo + bytes - 1) / kHomePage) - (lo / kHomePage) + 1);
}

size_t xd_home_map_workspace_size(const void *buf, size_t bytes) {
    return xd_home_map_pages(buf, bytes) * 2 * sizeof(uint32_t);
}

int xd_home_map(const void *buf, size_t bytes, uint8_t *attr, void *workspace, size_t workspace_bytes, void *stream) {
    XD_REQUIRE(buf != nullptr && bytes > 0 && attr != nullptr, "xd_home_map: NULL buffer or attr");
    XD_REQUIRE((reinterpret_cast<uintptr_t>(buf) & 3u) == 0, "xd_home_map: buf must be 4-byte aligned");
    const size_t npages = xd_home_map_pages(buf, bytes);
    if (workspace == nullptr || workspace_bytes < npages * 2 * sizeof(uint32_t) || (reinterpret_cast<uintptr_t>(workspace) & 3u))
        return fail(XD_ERR_WORKSPACE, "xd_home_map: workspace smaller than xd_home_map_workspace_size()");
    const uint64_t lo = reinterpret_cast<uint64_t>(buf), hi = lo + bytes;
    const uint64_t page0 = lo / kHomePage;
    hipStream_t s = (hipStream_t)stream;
    const unsigned grid = kNumXcd * kHomeProbeWgsPerXcd;
    uint32_t *lat = static_cast<uint32_t *>(workspace);
    launch("home_touch_kernel", home_touch_kernel, dim3(grid), dim3(64), 0, s, page0, (uint64_t)npages, lo, hi, lat);
    if (int rc = launch_status("home_touch_kernel")) return rc;
    for (int die = 0; die < 2; ++die) {
        launch("home_measure_kernel", home_measure_kernel, dim3(grid), dim3(64), 0, s, page0, (uint64_t)npages, lo, hi, lat, die);
        if (int rc = launch_status("home_measure_kernel")) return rc;
    }
    launch("home_classify_kernel", home_classify_kernel, dim3(64), dim3(256), 0, s, lat, (uint64_t)npages, attr);
    return launch_status("home_classify_kernel");
}

size_t xd_cache_flush_bytes(void) { return (size_t)1 << 30; }

int xd_cache_flush(const void *buf, size_t bytes, void *stream) {
    XD_REQUIRE(buf != nullptr, "xd_cache_flush: buf is NULL");
    XD_REQUIRE(aligned16(buf), "xd_cache_flush: buf must be 16-byte aligned");
    size_t n16 = bytes / 16;
    if (n16 == 0) return XD_OK;
    launch("cache_flush_kernel", cache_flush_kernel, dim3(2048), dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<const u32x4 *>(buf), n16);
    return launch_status("cache_flush_kernel");
}

int xd_read_stream(const void *buf, size_t bytes, int mode, const uint8_t *home_attr, int workgroups, int depth,
                   void *stream) {
    XD_REQUIRE(buf != nullptr, "xd_read_stream: buf is NULL");
    XD_REQUIRE(aligned16(buf) && bytes % 16 == 0, "xd_read_stream: buf and bytes must be 16-byte aligned");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "xd_read_stream: bad mode");
    const uint64_t nvec = bytes / 16;
    if (nvec == 0) return XD_OK;
    // the home modes walk whole 16 KiB pairs: buf 16 KiB aligned, bytes a multiple of 16 KiB
    const bool pairs = mode != XD_MODE_OBLIVIOUS && reinterpret_cast<uintptr_t>(buf) % (2 * kHomeChunk) == 0 &&
                       bytes % (2 * kHomeChunk) == 0;
    XD_REQUIRE(mode == XD_MODE_OBLIVIOUS || pairs,
               "xd_read_stream: the aware and rotated modes need buf and bytes in whole 16 KiB pairs");
    XD_REQUIRE(workgroups >= 0 && workgroups <= (1 << 20) && workgroups % kNumXcd == 0,
               "xd_read_stream: workgroups must be a multiple of 8 and at most 2^20 (0: 2048)");
    XD_REQUIRE(depth == 0 || depth == 1 || depth == 2 || depth == 4 || depth == 8,
               "xd_read_stream: depth must be 1, 2, 4 or 8 (0: 4)");
    const unsigned grid = workgroups ? (unsigned)workgroups : 2048u;
    const HomeMap home{home_attr, reinterpret_cast<uint64_t>(buf) / kHomePage, home_mask()};
    const u32x4 *b16 = reinterpret_cast<const u32x4 *>(buf);
    const uint64_t np = pairs ? (uint64_t)(bytes / (2 * kHomeChunk)) : 0ull;
    hipStream_t s = (hipStream_t)stream;
    const XcdHint xh = xcd_hint(s);
    switch (depth) {
        case 1: launch("read_stream_kernel", read_stream_kernel<1>, dim3(grid), dim3(kStreamThreads), 0, s, b16, nvec, np, mode, home, xh); break;
        case 2: launch("read_stream_kernel", read_stream_kernel<2>, dim3(grid), dim3(kStreamThreads), 0, s, b16, nvec, np, mode, home, xh); break;
        case 8: launch("read_stream_kernel", read_stream_kernel<8>, dim3(grid), dim3(kStreamThreads), 0, s, b16, nvec, np, mode, home, xh); break;
        default: launch("read_stream_kernel", read_stream_kernel<4>, dim3(grid), dim3(kStreamThreads), 0, s, b16, nvec, np, mode, home, xh); break;
    }
    return launch_status("read_stream_kernel");
}

}  // extern "C"
