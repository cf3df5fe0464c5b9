// GEMV y = A.x for fp32 and fp16-with-fp32-accumulate, XCD-oblivious / aware / rotated.
//
// Reference: applications/gemv/src/gemv_k1024_persistent_subwarp.cu
//   dot_subwarp (149-161): float4 loads, per-lane partial dot over a strided K range
//   subgroup_reduce (141-147): shuffle tree over the 32 lanes of a row
//   gemv_partitioned_kernel (163-197) / gemv_baseline_kernel (199-231): row placement
//
// MI355X design: one wave64 per row at a time, 16-byte (dwordx4) loads of A, x staged once
// per workgroup in LDS, DPP wave reduction, and a workgroup -> row-chunk map that gives
// every XCD one contiguous 1/8 of the rows (aware) or interleaves chunks across XCDs
// (oblivious). No MFMA: GEMV is 0.5 (fp32) or 1 (fp16) flop per byte of A.
#include <hip/hip_runtime.h>

#include "xd_common.hpp"

namespace xd {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kGemvMaxLdsBytes = 64 * 1024;

__device__ __forceinline__ float dot16_f32(uint4 a, uint4 b, float acc) {
    acc = __builtin_fmaf(__uint_as_float(a.x), __uint_as_float(b.x), acc);
    acc = __builtin_fmaf(__uint_as_float(a.y), __uint_as_float(b.y), acc);
    acc = __builtin_fmaf(__uint_as_float(a.z), __uint_as_float(b.z), acc);
    acc = __builtin_fmaf(__uint_as_float(a.w), __uint_as_float(b.w), acc);
    return acc;
}

__device__ __forceinline__ float dot16_f16(uint4 a, uint4 b, float acc) {
    // v_dot2_f32_f16: fp16 products are exact in fp32; accumulation is fp32.
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a.x), __builtin_bit_cast(half2_t, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a.y), __builtin_bit_cast(half2_t, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a.z), __builtin_bit_cast(half2_t, b.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a.w), __builtin_bit_cast(half2_t, b.w), acc, false);
    return acc;
}

// nv = 16-byte vectors per row. U = vectors each lane keeps in flight per batch.
template <bool F16, int U>
__global__ void __launch_bounds__(kGemvThreads)
gemv_kernel(const uint4 *__restrict__ A, const uint4 *__restrict__ x, float *__restrict__ y, int M, int nv,
            int rows_per_wg, int nchunks, int mode, unsigned rot) {
    extern __shared__ uint4 xs[];
    const int b = (int)blockIdx.x;
    int chunk;
    if (mode == XD_MODE_OBLIVIOUS) {
        chunk = b;
    } else {
        XcdSlot s = xcd_slot(b, (int)gridDim.x, mode, rot);
        chunk = s.slice * s.per_xcd + s.rank;
    }
    if (chunk >= nchunks) return;  // whole workgroup leaves before any barrier
    const int r0 = chunk * rows_per_wg;
    const int r1 = min(M, r0 + rows_per_wg);

    for (int i = (int)threadIdx.x; i < nv; i += kGemvThreads) xs[i] = x[i];
    __syncthreads();

    const int wave = (int)threadIdx.x / kWave;
    const int lane = (int)threadIdx.x % kWave;
    for (int row = r0 + wave; row < r1; row += kGemvWaves) {
        const uint4 *arow = A + (size_t)row * (size_t)nv;
        float acc = 0.0f;
        for (int v0 = 0; v0 < nv; v0 += kWave * U) {
            uint4 a[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int v = v0 + u * kWave + lane;
                a[u] = (v < nv) ? arow[v] : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int v = v0 + u * kWave + lane;
                if (v < nv) acc = F16 ? dot16_f16(a[u], xs[v], acc) : dot16_f32(a[u], xs[v], acc);
            }
        }
        acc = wave_sum_f32(acc);
        if (lane == 0) y[row] = acc;
    }
}

static int rows_per_workgroup(int M, int nv) {
    // Aim for >= 4 workgroups per CU on 256 CUs and one row per wave for long rows.
    int rpw = kGemvWaves;
    while ((long long)M / (rpw * 2) >= 1024 && nv * 16 * rpw * 2 <= 256 * 1024) rpw *= 2;
    return rpw;
}

template <bool F16>
static int launch_gemv(const void *A, const void *x, float *y, int M, int K, int mode, void *stream) {
    const int per_vec = F16 ? 8 : 4;
    XD_REQUIRE(A != nullptr && x != nullptr && y != nullptr, "gemv: NULL pointer");
    XD_REQUIRE(M > 0 && K > 0, "gemv: M and K must be positive");
    XD_REQUIRE(K % per_vec == 0, F16 ? "gemv_f16f32: K must be a multiple of 8" : "gemv_f32: K must be a multiple of 4");
    XD_REQUIRE(aligned16(A) && aligned16(x), "gemv: A and x must be 16-byte aligned");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "gemv: bad mode");
    const int nv = K / per_vec;
    const size_t lds = (size_t)nv * 16;
    if (lds > (size_t)kGemvMaxLdsBytes) return fail(XD_ERR_UNSUPPORTED, "gemv: K too large for the LDS-staged x");
    const int rpw = rows_per_workgroup(M, nv);
    const int nchunks = (M + rpw - 1) / rpw;
    const int grid = ((nchunks + kNumXcd - 1) / kNumXcd) * kNumXcd;
    const unsigned rot = mode == XD_MODE_ROTATED ? next_rotation(1) : 0u;
    hipStream_t s = (hipStream_t)stream;
    const uint4 *A4 = reinterpret_cast<const uint4 *>(A);
    const uint4 *x4 = reinterpret_cast<const uint4 *>(x);
    if (nv >= kWave * 16) {
        hipLaunchKernelGGL((gemv_kernel<F16, 16>), dim3(grid), dim3(kGemvThreads), lds, s, A4, x4, y, M, nv, rpw,
                           nchunks, mode, rot);
    } else {
        hipLaunchKernelGGL((gemv_kernel<F16, 8>), dim3(grid), dim3(kGemvThreads), lds, s, A4, x4, y, M, nv, rpw,
                           nchunks, mode, rot);
    }
    return launch_status("gemv_kernel");
}

}  // namespace xd

using namespace xd;

extern "C" {

int xd_gemv_f32(const float *A, const float *x, float *y, int M, int K, int mode, void *stream) {
    return launch_gemv<false>(A, x, y, M, K, mode, stream);
}

int xd_gemv_f16f32(const uint16_t *W, const uint16_t *x, float *y, int M, int K, int mode, void *stream) {
    return launch_gemv<true>(W, x, y, M, K, mode, stream);
}

}  // extern "C"
