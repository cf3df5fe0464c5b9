// Seeded host generators for the GEMV inputs (fp32 uniform, fp16 normal).
//
// The reference draws its GEMV inputs on the device from mix32 (GEMV.cu:118-139) and its
// other inputs from std::mt19937 + std::uniform_int_distribution (HASH.cu:229-252,
// BFS.cu:393-397), whose output is implementation defined. Here every generator is a fully
// specified function of (seed, index) built on the splitmix64 output function, so the
// same inputs can be rebuilt by any implementation.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "xdom.h"

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline uint64_t splitmix64_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t rand64(uint64_t seed, uint64_t index) { return splitmix64_mix(seed + (index + 1) * kGolden); }

// lowbias32, the reference's integer finalizer (GEMV.cu:56-63)
inline uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// binary16 bit pattern nearest to d (round to nearest, ties to even).
uint16_t f64_to_f16_rne(double d) {
    uint64_t bits;
    memcpy(&bits, &d, sizeof bits);
    uint16_t sign = (uint16_t)((bits >> 48) & 0x8000u);
    if (isnan(d)) return (uint16_t)(sign | 0x7E00u);
    double a = fabs(d);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u);  // 65520 is the tie to 2^16 -> inf
    if (a < 6.103515625e-05) {                           // below 2^-14: subnormal grid 2^-24
        double scaled = a * 16777216.0;                  // exact
        double m = floor(scaled);
        double frac = scaled - m;
        uint32_t mi = (uint32_t)m;
        if (frac > 0.5 || (frac == 0.5 && (mi & 1u))) ++mi;  // mi == 1024 encodes 2^-14
        return (uint16_t)(sign | mi);
    }
    int e;
    double f = frexp(a, &e);  // a = f * 2^e, f in [0.5, 1)
    double scaled = f * 2048.0;
    double m = floor(scaled);
    double frac = scaled - m;
    uint32_t mi = (uint32_t)m;
    if (frac > 0.5 || (frac == 0.5 && (mi & 1u))) ++mi;
    if (mi == 2048u) {
        mi = 1024u;
        ++e;
    }
    int hexp = e + 14;
    if (hexp >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)hexp << 10) | (mi - 1024u));
}

template <typename F>
void parallel_for(size_t n, F &&body) {
    unsigned hw = std::thread::hardware_concurrency();
    size_t nt = std::max<size_t>(1, std::min<size_t>(hw ? hw : 1, 16));
    if (n < (1u << 16)) nt = 1;
    if (nt == 1) {
        body(size_t(0), n);
        return;
    }
    std::vector<std::thread> ts;
    size_t per = (n + nt - 1) / nt;
    for (size_t t = 0; t < nt; ++t) {
        size_t b = t * per, e = std::min(n, b + per);
        if (b >= e) break;
        ts.emplace_back([&, b, e] { body(b, e); });
    }
    for (auto &t : ts) t.join();
}

}  // namespace

extern "C" {

uint64_t xd_rand64(uint64_t seed, uint64_t index) { return rand64(seed, index); }

int xd_gen_uniform_f32(float *out, size_t n, uint64_t seed) {
    if (out == nullptr && n != 0) return XD_ERR_INVALID_ARG;
    parallel_for(n, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) {
            // (k - 2^23) * 2^-23 with k a 24-bit integer: exact in binary32, in [-1, 1).
            uint32_t k = (uint32_t)(rand64(seed, i) >> 40);
            out[i] = (float)k * 1.1920928955078125e-07f - 1.0f;
        }
    });
    return XD_OK;
}

int xd_gen_normal_f16(uint16_t *out, size_t n, double mean, double stddev, uint64_t seed) {
    if (out == nullptr && n != 0) return XD_ERR_INVALID_ARG;
    const double two_pi = 6.283185307179586476925286766559;
    size_t pairs = (n + 1) / 2;
    parallel_for(pairs, [&](size_t b, size_t e) {
        for (size_t j = b; j < e; ++j) {
            double u1 = (double)((rand64(seed, 2 * j) >> 11) + 1) * 0x1.0p-53;  // (0, 1]
            double u2 = (double)(rand64(seed, 2 * j + 1) >> 11) * 0x1.0p-53;    // [0, 1)
            double r = sqrt(-2.0 * log(u1));
            double z0 = r * cos(two_pi * u2);
            double z1 = r * sin(two_pi * u2);
            out[2 * j] = f64_to_f16_rne(mean + stddev * z0);
            if (2 * j + 1 < n) out[2 * j + 1] = f64_to_f16_rne(mean + stddev * z1);
        }
    });
    return XD_OK;
}

int xd_gen_mix32_words(uint32_t *out, size_t n, uint32_t seed) {
    if (out == nullptr && n != 0) return XD_ERR_INVALID_ARG;
    parallel_for(n, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) out[i] = mix32((uint32_t)i ^ seed);
    });
    return XD_OK;
}

int xd_gen_mix32_f32(float *out, size_t n, uint32_t seed, uint32_t modulus, int32_t offset) {
    if (out == nullptr && n != 0) return XD_ERR_INVALID_ARG;
    parallel_for(n, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) {
            const uint32_t h = mix32((uint32_t)i ^ seed);
            // binary32 division and subtraction, each rounded to nearest (no excess precision)
            out[i] = modulus ? (float)((int32_t)(h % modulus) - offset) : (float)(h & 0xffu) / 255.0f - 0.5f;
        }
    });
    return XD_OK;
}

int xd_zipf_thresholds(uint64_t *out, uint32_t num_bins, double s) {
    if (out == nullptr || num_bins == 0 || !(s > 0.0)) return XD_ERR_INVALID_ARG;
    // P(rank = k) = (k+1)^-s / H, H = sum_{r=1..N} r^-s accumulated in rank order.
    double H = 0.0;
    for (uint32_t r = 1; r <= num_bins; ++r) H += pow((double)r, -s);
    double cum = 0.0;
    for (uint32_t k = 0; k < num_bins; ++k) {
        cum += pow((double)(k + 1), -s);
        const double f = cum / H;
        out[k] = (k + 1 == num_bins || f >= 1.0) ? UINT64_MAX : (uint64_t)ldexp(f, 64);
    }
    return XD_OK;
}

}  // extern "C"
