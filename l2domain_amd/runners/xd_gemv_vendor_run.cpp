// Vendor-library GEMV runner: the command line and stdout line of the reference's cuBLAS
// comparison (applications/gemv/src/gemv_cublas_benchmark.cu:42-101, parsed by
// applications/gemv/run.sh:86), on rocBLAS.
//
//   xd_gemv_vendor_run [M=65536] [K=1024] [runs=20] [warmups=5] [flush_l2=0] [inputs=mix32]
//
// inputs: mix32 (default), the reference's init_matrix_vector (seed 4242: A[i] =
// (mix32(i ^ 4242) & 0xff) / 255 - 0.5, x with seed + 0x9e37; xd_gen_mix32_f32), fp32 sgemv;
// f32, the fp32 configuration of this build (A and x U[-1,1) on a 2^-23 grid, seeds 4242 and
// 4242 + 0x9e37), fp32 sgemv; f16, the fp16 decode configuration (W ~ N(0, 0.02) seed 4243,
// x ~ N(0, 1) seed 4244, both binary16), rocBLAS's mixed-precision gemv (fp16 A and x, fp32
// compute and y: rocblas_hssgemv_strided_batched with one batch). Row-major A times x is
// computed as the transposed product of the K x M column-major matrix with the same memory
// (the reference's own trick, :73-75). The time is printed under the reference's key,
// `cublas_ms`, so that run.sh parsers read it unchanged; the `vendor=` line names the library
// routine. The result is checked (the reference does not check it): fp32, against the fp32
// CPU row loop, exit 3 when the largest error exceeds 1e-3; f16, against an fp64 row loop,
// exit 3 when the largest error exceeds 2e-2 of the largest |y|.
#include <math.h>
#include <rocblas/rocblas.h>

#include "runner_common.hpp"

using namespace runner;

#define RUN_BLAS(expr)                                                                           \
    do {                                                                                         \
        rocblas_status st_ = (expr);                                                             \
        if (st_ != rocblas_status_success) {                                                     \
            fprintf(stderr, "rocBLAS error %d at %s:%d: %s\n", (int)st_, __FILE__, __LINE__, #expr); \
            exit(1);                                                                             \
        }                                                                                        \
    } while (0)

// binary16 -> double (the check's own decoding: sign, 5-bit exponent, 10-bit fraction)
static double half_to_double(uint16_t h) {
    const int e = (h >> 10) & 31, f = h & 1023;
    double v;
    if (e == 0) v = ldexp((double)f, -24);                   // subnormal
    else if (e == 31) v = f ? NAN : INFINITY;
    else v = ldexp((double)(1024 + f), e - 25);
    return (h & 0x8000) ? -v : v;
}

int main(int argc, char **argv) {
    Options o(argc, argv);
    if (o.help) {
        printf("usage: %s [M=65536] [K=1024] [runs=20] [warmups=5] [flush_l2=0] [inputs=mix32|f32|f16]\n", argv[0]);
        return 0;
    }
    const int M = (int)std::max<long long>(o.geti(0, 65536), 1);
    const int K = (int)std::max<long long>(o.geti(1, 1024), 1);
    const int runs = (int)std::max<long long>(o.geti(2, 20), 1);
    const int warmups = (int)std::max<long long>(o.geti(3, 5), 0);
    const int flush_l2 = (int)std::min<long long>(std::max<long long>(o.geti(4, 0), 0), 1);
    const std::string inputs = o.gets(5, "mix32");
    if (inputs != "mix32" && inputs != "f32" && inputs != "f16") {
        fprintf(stderr, "inputs must be mix32, f32 or f16\n");
        return 2;
    }
    const bool f16 = inputs == "f16";
    const xd_topology_t topo = topology();
    hipStream_t s;
    RUN_HIP(hipStreamCreate(&s));

    const size_t elems = (size_t)M * K;
    const size_t esz = f16 ? 2 : 4;
    std::vector<float> hA, hx;
    std::vector<uint16_t> hA16, hx16;
    if (f16) {
        hA16.resize(elems);
        hx16.resize(K);
        RUN_XD(xd_gen_normal_f16(hA16.data(), elems, 0.0, 0.02, 4243u));
        RUN_XD(xd_gen_normal_f16(hx16.data(), K, 0.0, 1.0, 4244u));
    } else {
        hA.resize(elems);
        hx.resize(K);
        if (inputs == "f32") {
            RUN_XD(xd_gen_uniform_f32(hA.data(), elems, 4242u));
            RUN_XD(xd_gen_uniform_f32(hx.data(), K, 4242u + 0x9e37u));
        } else {
            RUN_XD(xd_gen_mix32_f32(hA.data(), elems, 4242u, 0u, 0));
            RUN_XD(xd_gen_mix32_f32(hx.data(), K, 4242u + 0x9e37u, 0u, 0));
        }
    }
    void *A = nullptr, *x = nullptr;
    float *y = nullptr;
    RUN_HIP(hipMalloc(&A, elems * esz));
    RUN_HIP(hipMalloc(&x, (size_t)K * esz));
    RUN_HIP(hipMalloc(&y, (size_t)M * 4));
    RUN_HIP(hipMemcpy(A, f16 ? (const void *)hA16.data() : (const void *)hA.data(), elems * esz, hipMemcpyHostToDevice));
    RUN_HIP(hipMemcpy(x, f16 ? (const void *)hx16.data() : (const void *)hx.data(), (size_t)K * esz,
                      hipMemcpyHostToDevice));

    rocblas_handle h;
    RUN_BLAS(rocblas_create_handle(&h));
    RUN_BLAS(rocblas_set_stream(h, s));
    const float alpha = 1.0f, beta = 0.0f;
    auto launch = [&] {
        if (f16)
            RUN_BLAS(rocblas_hssgemv_strided_batched(h, rocblas_operation_transpose, K, M, &alpha,
                                                     static_cast<const rocblas_half *>(A), K, (rocblas_stride)elems,
                                                     static_cast<const rocblas_half *>(x), 1, (rocblas_stride)K, &beta,
                                                     y, 1, (rocblas_stride)M, 1));
        else
            RUN_BLAS(rocblas_sgemv(h, rocblas_operation_transpose, K, M, &alpha, static_cast<const float *>(A), K,
                                   static_cast<const float *>(x), 1, &beta, y, 1));
    };
    for (int i = 0; i < warmups; ++i) launch();
    RUN_HIP(hipStreamSynchronize(s));
    Flusher flush;
    double total = 0.0;
    for (int r = 0; r < runs; ++r) {
        if (flush_l2) flush(s);
        total += time_ms(s, launch);
    }
    const double ms = total / runs;
    std::vector<float> hy(M);
    RUN_HIP(hipMemcpy(hy.data(), y, (size_t)M * 4, hipMemcpyDeviceToHost));
    double err = 0.0, ymax = 0.0;
    if (f16) {
        std::vector<double> wx(K);
        for (int k = 0; k < K; ++k) wx[k] = half_to_double(hx16[k]);
        for (int i = 0; i < M; ++i) {
            double sum = 0.0;
            for (int k = 0; k < K; ++k) sum += half_to_double(hA16[(size_t)i * K + k]) * wx[k];
            err = std::max(err, fabs((double)hy[i] - sum));
            ymax = std::max(ymax, fabs(sum));
        }
    } else {
        for (int i = 0; i < M; ++i) {
            float sum = 0.0f;
            for (int k = 0; k < K; ++k) sum += hA[(size_t)i * K + k] * hx[k];
            err = std::max(err, (double)fabsf(hy[i] - sum));
        }
    }
    const double flops = 2.0 * M * K, bytes = (double)esz * elems + (double)esz * K + 4.0 * M;
    printf("=== rocBLAS %s ===\n", f16 ? "HSSGEMV" : "SGEMV");
    printf("gpu=%s M=%d K=%d runs=%d flush_l2=%d inputs=%s matrix=%.1f MiB\n", topo.name, M, K, runs, flush_l2,
           inputs.c_str(), (double)elems * esz / (1024.0 * 1024.0));
    printf("cublas_ms %.6f ms %.2f GFLOP/s\n", ms, flops / (ms * 1e6));
    printf("vendor=rocblas_%s gbps=%.1f max_abs_error=%.6g\n", f16 ? "hssgemv_strided_batched" : "sgemv",
           bytes / (ms * 1e6), err);
    rocblas_destroy_handle(h);
    (void)hipFree(A);
    (void)hipFree(x);
    (void)hipFree(y);
    const bool ok = f16 ? err <= 2e-2 * std::max(ymax, 1e-30) : err <= 1e-3;
    return ok ? 0 : 3;
}
