// Shared plumbing of the per-application runner executables: argv parsing in the
// reference's positional style (argi: argument i or a default), HIP error checks that exit
// with status 1, event timing on one stream, and the optional CSV row writer.
//
// The reference's runners abort through CHECK_CUDA / LATOPT_CHECK (utility/latopt.cuh:12-29)
// and return 3 when results mismatch (applications/histogram/src/histogram256_sideaware.cu:558,
// applications/bfs/src/bfs.cu:558); these runners keep both conventions.
#pragma once

#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <string>
#include <vector>

#include "xdom.h"

namespace runner {

#define RUN_HIP(expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess) {                                                                \
            fprintf(stderr, "HIP error %s at %s:%d: %s\n", hipGetErrorString(e_), __FILE__,   \
                    __LINE__, #expr);                                                          \
            exit(1);                                                                           \
        }                                                                                      \
    } while (0)

#define RUN_XD(expr)                                                                           \
    do {                                                                                       \
        int rc_ = (expr);                                                                      \
        if (rc_ != XD_OK) {                                                                    \
            fprintf(stderr, "libxdom error %d at %s:%d: %s\n", rc_, __FILE__, __LINE__,        \
                    xd_last_error());                                                          \
            exit(1);                                                                           \
        }                                                                                      \
    } while (0)

// Positional arguments; "--key=value" options are collected separately by Options.
struct Options {
    std::vector<std::string> pos;
    std::vector<std::pair<std::string, std::string>> kv;  // other --key=value options
    std::string csv;        // --csv=FILE: append one CSV row (header written if the file is new)
    bool help = false;
    Options(int argc, char **argv) {
        for (int i = 1; i < argc; ++i) {
            const char *eq = strchr(argv[i], '=');
            if (!strncmp(argv[i], "--csv=", 6)) csv = argv[i] + 6;
            else if (!strcmp(argv[i], "--help") || !strcmp(argv[i], "-h")) help = true;
            else if (!strncmp(argv[i], "--", 2) && eq) kv.emplace_back(std::string(argv[i] + 2, (size_t)(eq - argv[i] - 2)), std::string(eq + 1));
            else pos.emplace_back(argv[i]);
        }
    }
    std::string opt(const char *key, const char *dflt) const {
        for (auto &p : kv)
            if (p.first == key) return p.second;
        return dflt;
    }
    long long geti(size_t i, long long dflt) const { return i < pos.size() ? atoll(pos[i].c_str()) : dflt; }
    double getd(size_t i, double dflt) const { return i < pos.size() ? atof(pos[i].c_str()) : dflt; }
    std::string gets(size_t i, const char *dflt) const { return i < pos.size() ? pos[i] : std::string(dflt); }
};

inline xd_topology_t topology() {
    xd_topology_t t{};
    RUN_XD(xd_topology_query(0, &t));
    return t;
}

// Milliseconds of `fn` launched on `s`, bracketed by events on the same stream.
template <typename F>
float time_ms(hipStream_t s, F &&fn) {
    hipEvent_t e0, e1;
    RUN_HIP(hipEventCreate(&e0));
    RUN_HIP(hipEventCreate(&e1));
    RUN_HIP(hipEventRecord(e0, s));
    fn();
    RUN_HIP(hipEventRecord(e1, s));
    RUN_HIP(hipEventSynchronize(e1));
    float ms = 0.0f;
    RUN_HIP(hipEventElapsedTime(&ms, e0, e1));
    RUN_HIP(hipEventDestroy(e0));
    RUN_HIP(hipEventDestroy(e1));
    return ms;
}

// Evicts every XCD's L2 and the Infinity Cache (the reference's GlobalL2Cache::reset).
struct Flusher {
    void *buf = nullptr;
    size_t bytes = 0;
    Flusher() {
        bytes = xd_cache_flush_bytes();
        RUN_HIP(hipMalloc(&buf, bytes));
        RUN_HIP(hipMemset(buf, 0, bytes));
    }
    ~Flusher() { (void)hipFree(buf); }
    void operator()(hipStream_t s) const { RUN_XD(xd_cache_flush(buf, bytes, s)); }
};

inline double wall_ms(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

inline double median(std::vector<float> v) {
    std::sort(v.begin(), v.end());
    if (v.empty()) return 0.0;
    const size_t n = v.size();
    return n % 2 ? v[n / 2] : 0.5 * (v[n / 2 - 1] + v[n / 2]);
}

// Appends `row` under `header` to `path`, writing the header first when the file is new.
inline void csv_append(const std::string &path, const char *header, const std::string &row) {
    if (path.empty()) return;
    FILE *f = fopen(path.c_str(), "r");
    const bool fresh = f == nullptr;
    if (f) fclose(f);
    f = fopen(path.c_str(), "a");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path.c_str());
        exit(1);
    }
    if (fresh) fprintf(f, "%s\n", header);
    fprintf(f, "%s\n", row.c_str());
    fclose(f);
}

// Device buffer holding the home map (xd_home_map) of [p, p + bytes).
struct HomeMap {
    uint8_t *attr = nullptr;
    HomeMap(const void *p, size_t bytes, hipStream_t s) {
        const size_t pages = xd_home_map_pages(p, bytes);
        const size_t wsb = xd_home_map_workspace_size(p, bytes);
        void *ws = nullptr;
        RUN_HIP(hipMalloc(&attr, pages));
        RUN_HIP(hipMalloc(&ws, wsb));
        RUN_XD(xd_home_map(p, bytes, attr, ws, wsb, s));
        RUN_HIP(hipStreamSynchronize(s));
        RUN_HIP(hipFree(ws));
    }
    ~HomeMap() { (void)hipFree(attr); }
};

}  // namespace runner
