// Library core: error state, topology, DomainScan and the cache-flush kernel.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
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

// Streams `n16` 16-byte words; the loaded values feed an asm sink so that the loads stay.
__global__ void __launch_bounds__(256) cache_flush_kernel(const u32x4 *buf, size_t n16) {
    uint32_t acc = 0;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        u32x4 v = __builtin_nontemporal_load(buf + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    asm volatile("" ::"v"(acc));
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
    std::snprintf(out->name, sizeof(out->name), "%s", prop.name);
    return XD_OK;
}

int xd_domain_scan(int num_wg, uint32_t *out_placement, void *stream) {
    XD_REQUIRE(num_wg > 0 && num_wg <= (1 << 24), "xd_domain_scan: num_wg out of range");
    XD_REQUIRE(out_placement != nullptr, "xd_domain_scan: out_placement is NULL");
    hipLaunchKernelGGL(domain_scan_kernel, dim3(num_wg), dim3(64), 0, (hipStream_t)stream,
                       out_placement, num_wg);
    return launch_status("domain_scan_kernel");
}

size_t xd_cache_flush_bytes(void) { return (size_t)1 << 30; }

int xd_cache_flush(const void *buf, size_t bytes, void *stream) {
    XD_REQUIRE(buf != nullptr, "xd_cache_flush: buf is NULL");
    XD_REQUIRE(aligned16(buf), "xd_cache_flush: buf must be 16-byte aligned");
    size_t n16 = bytes / 16;
    if (n16 == 0) return XD_OK;
    hipLaunchKernelGGL(cache_flush_kernel, dim3(2048), dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<const u32x4 *>(buf), n16);
    return launch_status("cache_flush_kernel");
}

}  // extern "C"
