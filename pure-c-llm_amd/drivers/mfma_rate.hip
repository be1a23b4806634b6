// mfma_rate.hip -- sustained matrix-core rate versus operand data.
//
// The MI355X holds the cycle count of an MFMA fixed (32 cycles for
// v_mfma_i32_32x32x32_i8, 16 for v_mfma_f32_32x32x2f32 per wave) but lowers
// the shader clock with the switching activity of the operands, so the
// attainable TOP/s of a GEMM depends on its data. This program measures it:
// one 256-thread workgroup per CU, four independent 32x32 accumulators per
// wave, operands held in registers (no memory traffic), for operands that are
// all zero, small integers, random nibbles and uniformly random bytes (the
// gemm_bench INT8 workload), and random fp32 for the f32 MFMA. It prints the
// rate, the cycles per MFMA from the shader-clock counter and the implied
// clock.
#include <hip/hip_runtime.h>
#include <cstdio>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int ITERS = 1024;  // 4 MFMAs each

template <int MODE>
__global__ void __launch_bounds__(256) i8_rate(int *out, unsigned long long *cyc, unsigned seed) {
    const int tid = threadIdx.x;
    unsigned s = seed ^ (tid * 2654435761u) ^ (blockIdx.x * 40503u);
    auto rnd = [&]() {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        return (int)s;
    };
    v4i a[2], b[2];
    for (int i = 0; i < 2; i++) {
        for (int e = 0; e < 4; e++) {
            if (MODE == 0) a[i][e] = b[i][e] = 0;
            else if (MODE == 1) { a[i][e] = (tid + e) & 7; b[i][e] = (i + e) & 3; }
            else if (MODE == 2) { a[i][e] = rnd() & 0x0f0f0f0f; b[i][e] = rnd() & 0x0f0f0f0f; }
            else { a[i][e] = rnd(); b[i][e] = rnd(); }
        }
    }
    v16i acc[2][2];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0;
    const unsigned long long c0 = __builtin_readcyclecounter();
    for (int it = 0; it < ITERS; it++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    const unsigned long long c1 = __builtin_readcyclecounter();
    int t = 0;
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int v = 0; v < 16; v++) t += acc[i][j][v];
    out[blockIdx.x * 256 + tid] = t;
    if ((tid & 63) == 0) cyc[blockIdx.x * 4 + (tid >> 6)] = c1 - c0;
}

__global__ void __launch_bounds__(256) f32_rate(float *out, unsigned long long *cyc, unsigned seed) {
    const int tid = threadIdx.x;
    unsigned s = seed ^ (tid * 2654435761u) ^ (blockIdx.x * 40503u);
    auto rndf = [&]() {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        return (float)(s >> 8) * (1.0f / 16777216.0f) - 0.5f;
    };
    float a[2], b[2];
    for (int i = 0; i < 2; i++) { a[i] = rndf(); b[i] = rndf(); }
    v16f acc[2][2];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;
    const unsigned long long c0 = __builtin_readcyclecounter();
    for (int it = 0; it < ITERS; it++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    const unsigned long long c1 = __builtin_readcyclecounter();
    float t = 0.f;
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int v = 0; v < 16; v++) t += acc[i][j][v];
    out[blockIdx.x * 256 + tid] = t;
    if ((tid & 63) == 0) cyc[blockIdx.x * 4 + (tid >> 6)] = c1 - c0;
}

template <typename K, typename T>
static void run(const char *name, K kern, T *out, unsigned long long *cyc, double ops_per_mfma,
                int cus) {
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    hipLaunchKernelGGL(kern, dim3(cus), dim3(256), 0, 0, out, cyc, 12345u);
    (void)hipEventRecord(e0, 0);
    for (int r = 0; r < 10; r++) hipLaunchKernelGGL(kern, dim3(cus), dim3(256), 0, 0, out, cyc, 777u + r);
    (void)hipEventRecord(e1, 0);
    (void)hipEventSynchronize(e1);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    static unsigned long long h[4096];
    (void)hipMemcpy(h, cyc, (size_t)cus * 4 * 8, hipMemcpyDeviceToHost);
    double avg = 0;
    for (int i = 0; i < cus * 4; i++) avg += (double)h[i];
    avg /= cus * 4;
    const double us = ms / 10 * 1e3;
    const double rate = (double)cus * 4 * ITERS * 4 * ops_per_mfma / (us * 1e-6) / 1e12;
    printf("%-26s %8.2f us  %5.1f cycles/MFMA  clock %.2f GHz  %8.1f T(FL)OP/s\n", name, us,
           avg / (ITERS * 4), avg / (us * 1e3), rate);
}

int main() {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return 1;
    const int cus = prop.multiProcessorCount;
    int *iout;
    float *fout;
    unsigned long long *cyc;
    if (hipMalloc(&iout, (size_t)cus * 256 * 4) || hipMalloc(&fout, (size_t)cus * 256 * 4) ||
        hipMalloc(&cyc, (size_t)cus * 4 * 8))
        return 1;
    printf("%s, %d CUs; one workgroup of 4 waves per CU, 4 accumulators per wave\n", prop.gcnArchName, cus);
    const double i8 = 32.0 * 32 * 32 * 2, f32 = 32.0 * 32 * 2 * 2;
    run("i8 32x32x32, zeros", i8_rate<0>, iout, cyc, i8, cus);
    run("i8 32x32x32, small ints", i8_rate<1>, iout, cyc, i8, cus);
    run("i8 32x32x32, random nibbles", i8_rate<2>, iout, cyc, i8, cus);
    run("i8 32x32x32, random bytes", i8_rate<3>, iout, cyc, i8, cus);
    run("f32 32x32x2, random", f32_rate, fout, cyc, f32, cus);
    return 0;
}
