/*
 * ref_shim_gemm_bench.c -- build-time harness around the reference's own
 * gemm_bench.c (pure-c-llm). TEST INFRASTRUCTURE ONLY.
 *
 * The reference file is compiled where it lies (the path comes from the
 * Makefile as REF_GEMM_BENCH_C); nothing of it is copied here. Its kernels are
 * `static`, so this translation unit includes it and exports thin wrappers
 * under pcl_ref_* names. Its main() is renamed by -Dmain=... on the command
 * line. The result, oracle/_ref/libref_gemm_bench.so, is used to pin the
 * oracle restatement and as the CPU baseline ("kind": "reference").
 */
#include REF_GEMM_BENCH_C

int pcl_ref_cpu_ok(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vnni");
}
void pcl_ref_set_threads(int n) { omp_set_num_threads(n); }
int pcl_ref_max_threads(void) { return omp_get_max_threads(); }

/* gemm_bench.c:60-192 FP32 rungs */
void pcl_ref_gemm_naive(const float *A, const float *B, float *C, int M, int K, int N) { gemm_naive(A, B, C, M, K, N); }
void pcl_ref_gemm_ikj(const float *A, const float *B, float *C, int M, int K, int N) { gemm_ikj(A, B, C, M, K, N); }
void pcl_ref_gemm_micro(const float *A, const float *B, float *C, int M, int K, int N) { gemm_micro(A, B, C, M, K, N); }
void pcl_ref_gemm_packed(const float *A, const float *B, float *C, int M, int K, int N) { gemm_packed(A, B, C, M, K, N); }
void pcl_ref_gemm_packed_mt(const float *A, const float *B, float *C, int M, int K, int N) { gemm_packed_mt(A, B, C, M, K, N); }

/* gemm_bench.c:225-285 INT8 rung */
float pcl_ref_quantize_A(const float *A, uint8_t *Au, int M, int K, int Kpad) { return quantize_A(A, Au, M, K, Kpad); }
void pcl_ref_quantize_B_pack(const float *B, int8_t *Bp, float *bscale, int32_t *colsum, int K, int N, int Kpad) {
    quantize_B_pack(B, Bp, bscale, colsum, K, N, Kpad);
}
void pcl_ref_gemm_int8_kernel(const uint8_t *Au, int Kpad, const int8_t *Bp, const int32_t *corr,
                              const float *dq, float *C, int M, int N) {
    gemm_int8_kernel(Au, Kpad, Bp, corr, dq, C, M, N);
}
double pcl_ref_rms_rel(const float *X, const float *R, long n) { return rms_rel(X, R, n); }
double pcl_ref_max_abs_diff(const float *X, const float *Y, long n) { return max_abs_diff(X, Y, n); }
/* gemm_bench.c:50-52: glibc rand() after the caller's srand() */
void pcl_ref_srand(unsigned s) { srand(s); }
void pcl_ref_fill_rand(float *p, long n) { fill_rand(p, n); }

/* The reference INT8 rung (gemm_int8_kernel, single-threaded in gemm_bench)
 * driven over row bands of Au and C, one band per OpenMP thread: the
 * multi-threaded CPU baseline over M tiles. Bands are multiples of the
 * kernel's 8-row microkernel (M % 8 == 0, as the reference requires). */
void pcl_ref_gemm_int8_mt(int threads, const uint8_t *Au, int Kpad, const int8_t *Bp,
                          const int32_t *corr, const float *dq, float *C, int M, int N) {
#pragma omp parallel num_threads(threads)
    {
        const int t = omp_get_thread_num(), nt = omp_get_num_threads();
        const long blocks = M / 8;
        const int b0 = (int)(blocks * t / nt) * 8, b1 = (int)(blocks * (t + 1) / nt) * 8;
        if (b1 > b0)
            gemm_int8_kernel(Au + (size_t)b0 * Kpad, Kpad, Bp, corr, dq, C + (size_t)b0 * N, b1 - b0, N);
    }
}
/* gemm_bench.c:195-210, 287-325: the reference's own 1-core roofs and triad */
double pcl_ref_peak_gflops(void) { return measure_peak_gflops(); }
double pcl_ref_peak_int8_gops(void) { return measure_peak_int8_gops(); }
double pcl_ref_bandwidth_gbs(void) { return measure_bandwidth_gbs(); }
