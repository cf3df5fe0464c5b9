// Architecture probe runner: DomainScan, XDom-PChase, MaskProbe and the L2 channel probe with
// the CSV schemas of the reference's architecture figures (architecture/src/
// architecture_probe.cu: figure 2 columns :587, figure 3 columns :613, figure 4 columns of
// run_figure_4; data in architecture/data/figure_0*.csv).
//
//   xd_arch_probe domainscan [num_wg=4096]                          [--csv=FILE]
//   xd_arch_probe scanlat [first_bit=7] [last_bit=31] [leader_xcd=0] [--csv=FILE]
//   xd_arch_probe pchase [leader_xcd=0] [follower_xcd=4] [numel=2048] [stride=128] [--csv=FILE]
//   xd_arch_probe maskprobe [first_bit=5] [last_bit=29] [reps=8]    [--csv=FILE]
//   xd_arch_probe chanprobe [xcd=0] [first_bit=7] [last_bit=20]     [--csv=FILE]
//   xd_arch_probe memprobe [first_bit=7] [last_bit=20] [nsets=6]    [--csv=FILE]
//
// scanlat (figure 3): for every compute unit in turn, a flushed-cache leader/follower round
// (xd_domain_scan_latency) run twice, the second kept; tpc_id = follower index, resource_id =
// its placement key, tpc_sm0 = its XCD, tpc_sm1 = its rank inside the XCD, follower_sm = its
// global index XCD * 32 + rank. chanprobe: the L2 channel functions of one XCD as XOR masks;
// rows per (function, bit) with the time of the bit added to the function's five-bit set
// (function -1: the windows of six consecutive bits starting at address_bit). memprobe: the
// memory-side units beyond the L2 (returning atomics from every XCD); one row per bit pair
// (bit_a == bit_b: the bit alone) with the smallest slowdown it caused, whether it never
// changes the unit, and the class of equal-effect bits each active bit belongs to.
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
    if (o.help || (what != "domainscan" && what != "scanlat" && what != "pchase" && what != "maskprobe" &&
                   what != "chanprobe" && what != "memprobe")) {
        printf("usage: %s domainscan [num_wg] | scanlat [first_bit] [last_bit] [leader_xcd] | pchase [leader_xcd] "
               "[follower_xcd] [numel] [stride] | maskprobe [first_bit] [last_bit] [reps] | chanprobe [xcd] "
               "[first_bit] [last_bit] | memprobe [first_bit] [last_bit] [nsets]  [--csv=FILE]\n",
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
    if (what == "scanlat") {
        const int b0 = (int)o.geti(1, 7), b1 = (int)o.geti(2, 31), leader = (int)o.geti(3, 0);
        if (b0 < 3 || b1 < b0 || b1 > 34 || leader < 0 || leader > 7) return 2;
        // the compute units a DomainScan reaches, XCD-major
        const int nwg = 4096;
        uint32_t *d;
        RUN_HIP(hipMalloc(&d, (size_t)nwg * 4));
        RUN_XD(xd_domain_scan(nwg, d, s));
        std::vector<uint32_t> w(nwg);
        RUN_HIP(hipMemcpy(w.data(), d, (size_t)nwg * 4, hipMemcpyDeviceToHost));
        (void)hipFree(d);
        std::vector<uint32_t> keys;
        for (uint32_t x : w) keys.push_back(x >> 8);
        std::sort(keys.begin(), keys.end());
        keys.erase(std::unique(keys.begin(), keys.end()), keys.end());
        const int nb = b1 - b0 + 1;
        const size_t bytes = (1ull << b1) + 4096;
        void *buf;
        uint32_t *out;
        RUN_HIP(hipMalloc(&buf, bytes));
        RUN_HIP(hipMemset(buf, 0, bytes));
        RUN_HIP(hipMalloc(&out, (size_t)(nb + 4) * 4));
        Flusher fl;
        std::vector<uint32_t> h(nb + 4);
        std::vector<double> same, other;
        int rank = 0;
        uint32_t prev_xcd = 0xffffffffu;
        for (size_t t = 0; t < keys.size(); ++t) {
            const uint32_t xcd = keys[t] >> 16;
            rank = xcd == prev_xcd ? rank + 1 : 0;
            prev_xcd = xcd;
            for (int rep = 0; rep < 2; ++rep)
                RUN_XD(xd_domain_scan_latency(buf, bytes, b0, b1, leader, keys[t], fl.buf, fl.bytes, out, s));
            RUN_HIP(hipMemcpy(h.data(), out, h.size() * 4, hipMemcpyDeviceToHost));
            if (h[nb] != 1 || h[nb + 1] != 1) {
                fprintf(stderr, "scanlat: no workgroup on the leader XCD or on CU key 0x%x\n", keys[t]);
                return 3;
            }
            std::vector<float> c(h.begin(), h.begin() + nb);
            ((int)xcd == leader ? same : other).push_back(median(c));
            for (int k = 0; k < nb; ++k)
                csv_append(o.csv,
                           "device_index,device_name,leader_sm,tpc_id,resource_id,tpc_sm0,tpc_sm1,follower_sm,"
                           "address_bit,latency_cycles",
                           dev + "," + std::to_string(h[nb + 2]) + "," + std::to_string(t) + "," +
                               std::to_string(keys[t]) + "," + std::to_string(xcd) + "," + std::to_string(rank) +
                               "," + std::to_string(xcd * 32 + rank) + "," + std::to_string(b0 + k) + "," +
                               std::to_string(h[k]));
        }
        auto avg = [](const std::vector<double> &v) {
            double a = 0;
            for (double x : v) a += x;
            return v.empty() ? 0.0 : a / v.size();
        };
        printf("scanlat followers=%zu bits=%d..%d leader_xcd=%d mean_median_cycles same_xcd=%.0f other_xcd=%.0f\n",
               keys.size(), b0, b1, leader, avg(same), avg(other));
        (void)hipFree(buf);
        (void)hipFree(out);
        return 0;
    }
    if (what == "chanprobe") {
        const int xcd = (int)o.geti(1, 0), b0 = (int)o.geti(2, 7), b1 = (int)o.geti(3, 20);
        if (xcd < 0 || xcd > 7 || b0 < 7 || b1 - b0 < 6 || b1 > 33) return 2;
        const size_t bytes = (2ull << b1) + (2ull << 20);
        void *buf;
        RUN_HIP(hipMalloc(&buf, bytes));
        RUN_HIP(hipMemset(buf, 0, bytes));
        const int nb = b1 - b0 + 1, nw = b1 - b0 - 4;
        std::vector<float> win(nw), curves(4 * (size_t)nb);
        float fast = 0.0f;
        uint64_t masks[4] = {0, 0, 0, 0};
        int nm = 0;
        RUN_XD(xd_channel_probe(buf, bytes, xcd, b0, b1, 256, 256, win.data(), &fast, masks, curves.data(), &nm, s));
        const char *hdr = "device_index,device_name,xcd,function,mask,address_bit,us,in_function,page_stable";
        for (int k = 0; k < nw; ++k)
            csv_append(o.csv, hdr,
                       dev + "," + std::to_string(xcd) + ",-1,0," + std::to_string(b0 + k) + "," +
                           std::to_string(win[k]) + ",0," + std::to_string((int)(b0 + k + 5 <= 20)));
        uint64_t active = 0;
        std::string ms;
        for (int f = 0; f < nm; ++f) {
            active |= masks[f];
            char hx[32];
            snprintf(hx, sizeof hx, "0x%llx", (unsigned long long)masks[f]);
            ms += (ms.empty() ? "" : ",") + std::string(hx);
            for (int k = 0; k < nb; ++k)
                csv_append(o.csv, hdr,
                           dev + "," + std::to_string(xcd) + "," + std::to_string(f) + "," + hx + "," +
                               std::to_string(b0 + k) + "," + std::to_string(curves[(size_t)f * nb + k]) + "," +
                               std::to_string((int)(masks[f] >> (b0 + k) & 1)) + "," +
                               std::to_string((int)(b0 + k <= 20)));
        }
        printf("chanprobe xcd=%d bits=%d..%d fast_us=%.1f functions=%d masks=%s active_mask=0x%llx\n", xcd, b0, b1,
               fast, nm, ms.c_str(), (unsigned long long)active);
        (void)hipFree(buf);
        return nm > 0 ? 0 : 3;
    }
    if (what == "memprobe") {
        const int b0 = (int)o.geti(1, 7), b1 = (int)o.geti(2, 20), nsets = (int)o.geti(3, 6);
        if (b0 < 7 || b1 - b0 < 6 || b1 > 33 || b1 - b0 > 31 || nsets < 1 || nsets > 64) return 2;
        const size_t bytes = (2ull << b1) + (2ull << 20);
        void *buf;
        RUN_HIP(hipMalloc(&buf, bytes));
        RUN_HIP(hipMemset(buf, 0, bytes));
        const int nb = b1 - b0 + 1;
        std::vector<float> ratio((size_t)nb * nb);
        uint64_t inactive = 0, masks[32] = {};
        int nm = 0;
        RUN_XD(xd_memchannel_probe(buf, bytes, b0, b1, 64, nsets, ratio.data(), &inactive, masks, &nm, s));
        auto cls = [&](int bit) {
            for (int k = 0; k < nm; ++k)
                if (masks[k] >> bit & 1) return k;
            return -1;
        };
        for (int a = 0; a < nb; ++a)
            for (int b = a; b < nb; ++b) {
                const float r = ratio[(size_t)a * nb + b];
                csv_append(o.csv,
                           "device_index,device_name,bit_a,bit_b,min_slowdown,never_changes_unit,class_a,class_b,"
                           "page_stable",
                           dev + "," + std::to_string(b0 + a) + "," + std::to_string(b0 + b) + "," + std::to_string(r) +
                               "," + std::to_string((int)(r > 1.4f)) + "," + std::to_string(cls(b0 + a)) + "," +
                               std::to_string(cls(b0 + b)) + "," + std::to_string((int)(b0 + b <= 20)));
            }
        std::string ms;
        for (int k = 0; k < nm; ++k) {
            char hx[32];
            snprintf(hx, sizeof hx, "0x%llx", (unsigned long long)masks[k]);
            ms += (ms.empty() ? "" : ",") + std::string(hx);
        }
        printf("memprobe bits=%d..%d inactive=0x%llx classes=%d masks=%s\n", b0, b1, (unsigned long long)inactive, nm,
               ms.c_str());
        (void)hipFree(buf);
        return nm > 0 ? 0 : 3;
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
