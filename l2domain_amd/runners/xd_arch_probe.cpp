// Architecture probe runner: DomainScan, XDom-PChase and MaskProbe with the CSV schemas of
// the reference's architecture figures (architecture/src/architecture_probe.cu: figure 2
// columns :587, figure 4 columns of run_figure_4; data in architecture/data/figure_0*.csv).
//
//   xd_arch_probe domainscan [num_wg=4096]                          [--csv=FILE]
//   xd_arch_probe pchase [leader_xcd=0] [follower_xcd=4] [numel=2048] [stride=128] [--csv=FILE]
//   xd_arch_probe maskprobe [first_bit=5] [last_bit=29] [reps=8]    [--csv=FILE]
//
// The SM columns of the reference's schemas (leader_sm, follower_sm, sm_a, sm_b) carry XCD
// ids here: the XCD is the L2 domain on MI355X. pchase flushes every L2 and the Infinity
// Cache before the leader's first chase. maskprobe compares I/O die 0 (XCD 0) with die 1
// (XCD 4); active = the latency relation flips against the base address and the bit is
// below the 2 MiB page (derive_active_bits, run_mask_probe :495-523, :644-670).
#include "runner_common.hpp"

using namespace runner;

static std::string quoted(const char *s) { return std::string("\"") + s + "\""; }

static double med(const uint32_t *p, int n) {
    std::vector<float> v(p, p + n);
    return median(v);
}

int main(int argc, char **argv) {
    Options o(argc, argv);
    const std::string what = o.gets(0, "");
    if (o.help || (what != "domainscan" && what != "pchase" && what != "maskprobe")) {
        printf("usage: %s domainscan [num_wg] | pchase [leader_xcd] [follower_xcd] [numel] [stride] | "
               "maskprobe [first_bit] [last_bit] [reps]  [--csv=FILE]\n",
               argv[0]);
        return o.help ? 0 : 2;
    }
    const xd_topology_t topo = topology();
    hipStream_t s;
    RUN_HIP(hipStreamCreate(&s));
    const std::string dev = "0," + quoted(topo.name);

    if (what == "domainscan") {
        const int nwg = (int)o.geti(1, 4096);
        if (nwg < 1 || nwg > (1 << 20)) return 2;
        uint32_t *d;
        RUN_HIP(hipMalloc(&d, (size_t)nwg * 4));
        RUN_XD(xd_domain_scan(nwg, d, s));
        std::vector<uint32_t> w(nwg);
        RUN_HIP(hipMemcpy(w.data(), d, (size_t)nwg * 4, hipMemcpyDeviceToHost));
        int rr = 0;
        std::vector<int> per(8, 0);
        for (int i = 0; i < nwg; ++i) {
            const int x = (int)(w[i] >> 24);
            rr += x == i % 8;
            if (x < 8) per[x]++;
            csv_append(o.csv, "device_index,device_name,workgroup,xcc_id,se_id,sh_id,cu_id,simd_id",
                       dev + "," + std::to_string(i) + "," + std::to_string(x) + "," +
                           std::to_string((w[i] >> 16) & 0xff) + "," + std::to_string((w[i] >> 12) & 0xf) + "," +
                           std::to_string((w[i] >> 8) & 0xf) + "," + std::to_string(w[i] & 0xff));
        }
        printf("domainscan workgroups=%d round_robin_matches=%d per_xcc=%d,%d,%d,%d,%d,%d,%d,%d\n", nwg, rr, per[0],
               per[1], per[2], per[3], per[4], per[5], per[6], per[7]);
        (void)hipFree(d);
        return rr == nwg ? 0 : 3;
    }
    if (what == "pchase") {
        const int a = (int)o.geti(1, 0), b = (int)o.geti(2, 4), n = (int)o.geti(3, 2048), stride = (int)o.geti(4, 128);
        void *chain;
        uint32_t *d;
        RUN_HIP(hipMalloc(&chain, (size_t)n * stride));
        RUN_HIP(hipMalloc(&d, (4 * (size_t)n + 4) * 4));
        Flusher fl;
        RUN_XD(xd_xdom_pchase(a, b, chain, (size_t)n * stride, n, stride, fl.buf, fl.bytes, d, s));
        std::vector<uint32_t> h(4 * (size_t)n + 4);
        RUN_HIP(hipMemcpy(h.data(), d, h.size() * 4, hipMemcpyDeviceToHost));
        if (h[4 * n + 2] != 1 || h[4 * n + 3] != 1) {
            fprintf(stderr, "a role found no workgroup on its XCD\n");
            return 3;
        }
        for (int i = 0; i < n; ++i)
            csv_append(o.csv,
                       "device_index,device_name,leader_sm,follower_sm,index,offset_bytes,leader_first_cycles,"
                       "leader_second_cycles,follower_first_cycles,follower_second_cycles",
                       dev + "," + std::to_string(h[4 * n]) + "," + std::to_string(h[4 * n + 1]) + "," +
                           std::to_string(i) + "," + std::to_string((size_t)i * stride) + "," + std::to_string(h[i]) +
                           "," + std::to_string(h[n + i]) + "," + std::to_string(h[2 * n + i]) + "," +
                           std::to_string(h[3 * n + i]));
        printf("pchase leader_xcd=%u follower_xcd=%u numel=%d stride=%d median_cycles leader_first=%.0f "
               "leader_second=%.0f follower_first=%.0f follower_second=%.0f\n",
               h[4 * n], h[4 * n + 1], n, stride, med(&h[0], n), med(&h[n], n), med(&h[2 * n], n), med(&h[3 * n], n));
        (void)hipFree(chain);
        (void)hipFree(d);
        return 0;
    }
    // maskprobe
    const int b0 = (int)o.geti(1, 5), b1 = (int)o.geti(2, 29), reps = (int)o.geti(3, 8);
    if (b0 < 2 || b1 < b0 || b1 > 34) return 2;
    const size_t bytes = (1ull << b1) + 4096;
    void *buf;
    uint32_t *d;
    const int nb = b1 - b0 + 2;
    RUN_HIP(hipMalloc(&buf, bytes));
    RUN_HIP(hipMemset(buf, 0, bytes));
    RUN_HIP(hipMalloc(&d, (2 * (size_t)nb + 4) * 4));
    RUN_XD(xd_mask_probe(buf, bytes, b0, b1, reps, d, s));
    std::vector<uint32_t> h(2 * (size_t)nb + 4);
    RUN_HIP(hipMemcpy(h.data(), d, h.size() * 4, hipMemcpyDeviceToHost));
    if (h[2 * nb + 2] != 1 || h[2 * nb + 3] != 1) {
        fprintf(stderr, "a die found no workgroup on its XCD\n");
        return 3;
    }
    auto rel = [](uint32_t x, uint32_t y) { return x == y ? 0 : (x > y ? 1 : -1); };
    int base = 0;
    for (int k = 0; k < nb && base == 0; ++k) base = rel(h[k], h[nb + k]);
    uint64_t mask = 0;
    std::string flips;
    for (int k = 1; k < nb; ++k) {
        const int bit = b0 + k - 1;
        const int r = rel(h[k], h[nb + k]);
        const bool flip = r != 0 && r != base;
        const bool stable = bit < 21;
        if (flip && stable) mask |= 1ull << bit;
        if (flip) flips += (flips.empty() ? "" : ",") + std::to_string(bit);
        csv_append(o.csv,
                   "device_index,device_name,sm_a,sm_b,address_bit,sm_a_follower_cycles,sm_b_follower_cycles,"
                   "observed_flip,page_stable,active",
                   dev + "," + std::to_string(h[2 * nb]) + "," + std::to_string(h[2 * nb + 1]) + "," +
                       std::to_string(bit) + "," + std::to_string(h[k]) + "," + std::to_string(h[nb + k]) + "," +
                       std::to_string((int)flip) + "," + std::to_string((int)stable) + "," +
                       std::to_string((int)(flip && stable)));
    }
    printf("maskprobe bits=%d..%d base_cycles=%u/%u observed_flip_bits=%s active_mask=0x%llx\n", b0, b1, h[0], h[nb],
           flips.c_str(), (unsigned long long)mask);
    (void)hipFree(buf);
    (void)hipFree(d);
    return 0;
}
