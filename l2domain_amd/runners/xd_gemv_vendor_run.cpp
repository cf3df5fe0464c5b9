// Vendor-library GEMV runner: the command line and stdout line of the reference's cuBLAS
// comparison (applications/gemv/src/gemv_cublas_benchmark.cu:42-101, parsed by
// applications/gemv/run.sh:86), on rocBLAS sgemv.
//
//   xd_gemv_vendor_run [M=65536] [K=1024] [runs=20] [warmups=5] [flush_l2=0]
//
// Inputs are the reference's init_matrix_vector (seed 4242: A[i] = (mix32(i ^ 4242) & 0xff)
// / 255 - 0.5, x with seed + 0x9e37; xd_gen_mix32_f32). Row-major A times x is computed as the
// transposed product of the K x M column-major matrix with the same memory (the reference's
// own trick, :73-75). The time is printed under the reference's key, `cublas_ms`, so that
// run.sh parsers read it unchanged; the `vendor=` line names the library. The result is
// checked against the fp32 CPU row loop and the maximum error printed (the reference does
// not check it); exit 3 when it exceeds 1e-3.
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

int main(int argc, char **argv) {
    Options o(argc, argv);
    if (o.help) {
        printf("usage: %s [M=65536] [K=1024] [runs=20] [warmups=5] [flush_l2=0]\n", argv[0]);
        return 0;
    }
    const int M = (int)std::max<long long>(o.geti(0, 65536), 1);
    const int K = (int)std::max<long long>(o.geti(1, 1024), 1);
    const int runs = (int)std::max<long long>(o.geti(2, 20), 1);
    const int warmups = (int)std::max<long long>(o.geti(3, 5), 0);
    const int flush_l2 = (int)std::min<long long>(std::max<long long>(o.geti(4, 0), 0), 1);
    const xd_topology_t topo = topology();
    hipStream_t s;
    RUN_HIP(hipStreamCreate(&s));

    const size_t elems = (size_t)M * K;
    std::vector<float> hA(elems), hx(K), hy(M);
    RUN_XD(xd_gen_mix32_f32(hA.data(), elems, 4242u, 0u, 0));
    RUN_XD(xd_gen_mix32_f32(hx.data(), K, 4242u + 0x9e37u, 0u, 0));
    float *A = nullptr, *x = nullptr, *y = nullptr;
    RUN_HIP(hipMalloc(&A, elems * 4));
    RUN_HIP(hipMalloc(&x, (size_t)K * 4));
    RUN_HIP(hipMalloc(&y, (size_t)M * 4));
    RUN_HIP(hipMemcpy(A, hA.data(), elems * 4, hipMemcpyHostToDevice));
    RUN_HIP(hipMemcpy(x, hx.data(), (size_t)K * 4, hipMemcpyHostToDevice));

    rocblas_handle h;
    RUN_BLAS(rocblas_create_handle(&h));
    RUN_BLAS(rocblas_set_stream(h, s));
    const float alpha = 1.0f, beta = 0.0f;
    auto launch = [&] {
        RUN_BLAS(rocblas_sgemv(h, rocblas_operation_transpose, K, M, &alpha, A, K, x, 1, &beta, y, 1));
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
    RUN_HIP(hipMemcpy(hy.data(), y, (size_t)M * 4, hipMemcpyDeviceToHost));
    double err = 0.0;
    for (int i = 0; i < M; ++i) {
        float sum = 0.0f;
        for (int k = 0; k < K; ++k) sum += hA[(size_t)i * K + k] * hx[k];
        err = std::max(err, (double)fabsf(hy[i] - sum));
    }
    const double flops = 2.0 * M * K, bytes = 4.0 * elems + 4.0 * K + 4.0 * M;
    printf("=== rocBLAS SGEMV ===\n");
    printf("gpu=%s M=%d K=%d runs=%d flush_l2=%d matrix=%.1f MiB\n", topo.name, M, K, runs, flush_l2,
           (double)elems * 4 / (1024.0 * 1024.0));
    printf("cublas_ms %.6f ms %.2f GFLOP/s\n", ms, flops / (ms * 1e6));
    printf("vendor=rocblas gbps=%.1f max_abs_error=%.6g\n", bytes / (ms * 1e6), err);
    rocblas_destroy_handle(h);
    (void)hipFree(A);
    (void)hipFree(x);
    (void)hipFree(y);
    return err <= 1e-3 ? 0 : 3;
}
