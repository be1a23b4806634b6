/*
 * gemm_ladder_gpu.c -- the gemm_bench.c harness (gemm_bench.c:327-416) driving
 * libpcl_hip instead of the CPU rungs.
 *
 * It keeps the reference's flow: srand(1234), glibc rand() fills A then B
 * (gemm_bench.c:50-52, 344, 403), a trusted i-k-j reference on the host
 * (gemm_bench.c:345), best-of-N timing of a gemm_fn (gemm_bench.c:328-337),
 * then the INT8 rung through quantize_A / quantize_B_pack / gemm_int8_kernel
 * with corr = 128*colsum and dq = a_scale*bscale (gemm_bench.c:368-384).
 * Two GPU rungs are timed:
 *   "matmul (host ptrs)"  the drop-in, including PCIe copies, as a caller
 *                         relinking gemm_bench.c would see it;
 *   "pcl_sgemm (device)"  inputs resident in HBM, HIP-event timed.
 *
 * Build: gcc -O2 -I include pure-c-llm_amd/drivers/gemm_ladder_gpu.c \
 *            -L pure-c-llm_amd -lpcl_hip -lm -fopenmp -o gemm_ladder_gpu
 * Run:   LD_LIBRARY_PATH=pure-c-llm_amd ./gemm_ladder_gpu [M K N]
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pcl_hip.h"

typedef void (*gemm_fn)(const float *, const float *, float *, int, int, int);

static double now(void) { return omp_get_wtime(); }

static void fill_rand(float *p, long n) {
    for (long i = 0; i < n; i++) p[i] = (float)rand() / (float)RAND_MAX * 2.0f - 1.0f;
}

static void host_ikj(const float *A, const float *B, float *C, int M, int K, int N) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++) {
        float *o = C + (size_t)i * N;
        for (int n = 0; n < N; n++) o[n] = 0.0f;
        for (int k = 0; k < K; k++) {
            float a = A[(size_t)i * K + k];
            const float *wr = B + (size_t)k * N;
            for (int n = 0; n < N; n++) o[n] += a * wr[n];
        }
    }
}

static double max_rel(const float *X, const float *R, long n) {
    double d = 0.0, r = 0.0;
    for (long i = 0; i < n; i++) {
        double e = fabs((double)X[i] - R[i]);
        if (e > d) d = e;
        if (fabs((double)R[i]) > r) r = fabs((double)R[i]);
    }
    return r > 0 ? d / r : d;
}

static double rms_rel(const float *X, const float *R, long n) {
    double se = 0.0, sr = 0.0;
    for (long i = 0; i < n; i++) {
        double d = (double)X[i] - R[i];
        se += d * d;
        sr += (double)R[i] * R[i];
    }
    return sqrt(se / (sr + 1e-30));
}

static double bench(gemm_fn fn, const float *A, const float *B, float *C, int M, int K, int N,
                    int reps) {
    double best = 1e30;
    for (int r = 0; r < reps; r++) {
        double t0 = now();
        fn(A, B, C, M, K, N);
        double dt = now() - t0;
        if (dt < best) best = dt;
    }
    return 2.0 * M * N * K / best / 1e9;
}

#define CHECK(x)                                                                       \
    do {                                                                               \
        int s_ = (x);                                                                  \
        if (s_ != PCL_OK) {                                                            \
            fprintf(stderr, "%s failed (%d): %s\n", #x, s_, pcl_last_error());         \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

static void run_shape(int M, int K, int N) {
    float *A = malloc((size_t)M * K * 4), *B = malloc((size_t)K * N * 4);
    float *C = malloc((size_t)M * N * 4), *Cref = malloc((size_t)M * N * 4);
    fill_rand(A, (long)M * K);
    fill_rand(B, (long)K * N);
    host_ikj(A, B, Cref, M, K, N);
    printf("--- shape M=%d K=%d N=%d ---\n", M, K, N);

    double g1 = bench(matmul, A, B, C, M, K, N, 6);
    pcl_set_abort_on_error(1);
    printf("  %-26s %9.1f GF/s   max rel %.1e\n", "matmul (host ptrs)", g1,
           max_rel(C, Cref, (long)M * N));

    float *dA = pcl_malloc((size_t)M * K * 4), *dB = pcl_malloc((size_t)K * N * 4);
    float *dC = pcl_malloc((size_t)M * N * 4);
    CHECK(pcl_memcpy_h2d(dA, A, (size_t)M * K * 4));
    CHECK(pcl_memcpy_h2d(dB, B, (size_t)K * N * 4));
    void *e0 = pcl_event_create(), *e1 = pcl_event_create();
    const int reps = 50;
    CHECK(pcl_sgemm(PCL_OP_N, PCL_OP_N, M, N, K, dA, K, dB, N, NULL, 0, dC, N, NULL));
    CHECK(pcl_event_record(e0));
    for (int r = 0; r < reps; r++)
        CHECK(pcl_sgemm(PCL_OP_N, PCL_OP_N, M, N, K, dA, K, dB, N, NULL, 0, dC, N, NULL));
    CHECK(pcl_event_record(e1));
    float ms = 0;
    CHECK(pcl_event_elapsed_ms(e0, e1, &ms));
    CHECK(pcl_memcpy_d2h(C, dC, (size_t)M * N * 4));
    double tf = 2.0 * M * N * K / (ms / reps * 1e-3) / 1e12;
    printf("  %-26s %9.2f TF/s   max rel %.1e\n", "pcl_sgemm (device)", tf,
           max_rel(C, Cref, (long)M * N));

    /* ---- INT8 rung (gemm_bench.c:368-384) ---- */
    int Kpad = (K + 3) & ~3;
    uint8_t *Au = malloc((size_t)M * Kpad);
    int8_t *Bp = malloc((size_t)(N / 16) * (Kpad / 4) * 64);
    float *bscale = malloc((size_t)N * 4), *dq = malloc((size_t)N * 4);
    int32_t *colsum = malloc((size_t)N * 4), *corr = malloc((size_t)N * 4);
    quantize_B_pack(B, Bp, bscale, colsum, K, N, Kpad);
    float a_scale = quantize_A(A, Au, M, K, Kpad);
    for (int n = 0; n < N; n++) {
        corr[n] = 128 * colsum[n];
        dq[n] = a_scale * bscale[n];
    }
    double bi = 1e30;
    for (int r = 0; r < 6; r++) {
        double t0 = now();
        gemm_int8_kernel(Au, Kpad, Bp, corr, dq, C, M, N);
        double dt = now() - t0;
        if (dt < bi) bi = dt;
    }
    printf("  %-26s %9.1f GOP/s  rel.err %.1e vs FP32\n", "gemm_int8_kernel (host)",
           2.0 * M * N * K / bi / 1e9, rms_rel(C, Cref, (long)M * N));

    pcl_event_destroy(e0);
    pcl_event_destroy(e1);
    pcl_free(dA);
    pcl_free(dB);
    pcl_free(dC);
    free(Au), free(Bp), free(bscale), free(dq), free(colsum), free(corr);
    free(A), free(B), free(C), free(Cref);
}

int main(int argc, char **argv) {
    srand(1234);
    char name[128];
    int cus = 0, clk = 0;
    CHECK(pcl_device_info(name, sizeof name, &cus, &clk));
    printf("=== libpcl_hip on %s: %d CUs, %d MHz ===\n", name, cus, clk / 1000);
    if (argc == 4) {
        run_shape(atoi(argv[1]), atoi(argv[2]), atoi(argv[3]));
    } else {
        run_shape(1024, 1024, 1024);  /* gemm_bench.c:413 */
        run_shape(1024, 1024, 4096);  /* gemm_bench.c:414 */
    }
    return 0;
}
