// roofs.hip -- the MI355X's own roofs, measured: the GPU counterparts of
// gemm_bench.c's measure_peak_int8_gops (:287-301), measure_peak_gflops
// (:309-325) and measure_bandwidth_gbs (STREAM triad, :195-210). The
// reference times its rungs against roofs it measures on the machine it runs
// on; these do the same for the matrix cores and HBM, so a kernel's fraction
// can be read against what the part sustains as well as its datasheet peak.
//
// Matrix cores: every CU runs eight waves (two per SIMD), each holding
// independent accumulators (four 32x32 for i8, eight 16x16 for f32: the
// instructions the GEMMs use) and its operands in registers, so nothing but
// the MFMA pipe is exercised. The MI355X lowers its shader clock with the
// switching activity of the operands, so the rate is measured for the data a
// GEMM sees: uniformly random bytes (the gemm_bench INT8 workload) or zeros
// for i8, uniform random floats for f32. Thirty warm-up launches (10-20 ms of
// load) bring the clock up first: a short run from idle reads 5-15% low.
//
// HBM: the triad a[i] = b[i] + s*c[i] over arrays far larger than the 256 MB
// Infinity Cache, a copy, a read-only and a write-only pass, with 16-byte
// non-temporal accesses, grid-stride; best of several passes (as gemm_bench's
// best of 5). The read-only rate is the roof of the weight-streaming GEMVs.
#include "internal.h"

namespace pcl {

typedef int rf_v4i __attribute__((ext_vector_type(4)));
typedef int rf_v16i __attribute__((ext_vector_type(16)));
typedef float rf_v4f __attribute__((ext_vector_type(4)));

constexpr int RF_WAVES = 8;     // per CU: two per SIMD
constexpr int RF_ITERS = 4096;  // four i8 or eight f32 MFMAs each
constexpr int RF_F32_CHAINS = 8;

__device__ __forceinline__ unsigned rf_next(unsigned &s) {
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    return s;
}

template <bool RANDOM>
__global__ __launch_bounds__(64 * RF_WAVES) void roof_i8_kernel(int *out, unsigned seed) {
    unsigned s = seed ^ (threadIdx.x * 2654435761u) ^ (blockIdx.x * 40503u) ^ 1u;
    rf_v4i a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            a[i][e] = RANDOM ? (int)rf_next(s) : 0;
            b[i][e] = RANDOM ? (int)rf_next(s) : 0;
        }
    rf_v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0;
    for (int it = 0; it < RF_ITERS; it++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    int t = 0;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) t += acc[i][j][v];
    out[blockIdx.x * blockDim.x + threadIdx.x] = t;
}

__global__ __launch_bounds__(64 * RF_WAVES) void roof_f32_kernel(float *out, unsigned seed) {
    unsigned s = seed ^ (threadIdx.x * 2654435761u) ^ (blockIdx.x * 40503u) ^ 1u;
    float a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a[i] = (float)(rf_next(s) >> 8) * (1.0f / 16777216.0f) - 0.5f;
        b[i] = (float)(rf_next(s) >> 8) * (1.0f / 16777216.0f) - 0.5f;
    }
    rf_v4f acc[RF_F32_CHAINS];
#pragma unroll
    for (int i = 0; i < RF_F32_CHAINS; i++)
#pragma unroll
        for (int v = 0; v < 4; v++) acc[i][v] = 0.f;
    for (int it = 0; it < RF_ITERS; it++)
#pragma unroll
        for (int i = 0; i < RF_F32_CHAINS; i++)
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i & 3], b[(i >> 2) & 3], acc[i], 0, 0, 0);
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < RF_F32_CHAINS; i++)
#pragma unroll
        for (int v = 0; v < 4; v++) t += acc[i][v];
    out[blockIdx.x * blockDim.x + threadIdx.x] = t;
}

// Streaming kernels over n4 16-byte elements with RF_U independent elements
// per thread per iteration (all loads issued before any use) and
// non-temporal accesses. A workgroup's iteration covers 256 * RF_U
// consecutive elements (16 KB: the thread's RF_U elements 4 KB apart), the
// grid strides over the array: each iteration stays within few DRAM pages
// (elements a grid stride apart in one iteration read ~25% slower here).
// mode 0: a = b + s*c (triad); 1: a = b (copy); 2: read b (one value per
// thread written); 3: write a.
constexpr int RF_U = 4;
template <int MODE>
__global__ __launch_bounds__(256) void roof_stream_kernel(rf_v4f *__restrict__ a, const rf_v4f *__restrict__ b,
                                                          const rf_v4f *__restrict__ c, float sc, long n4,
                                                          float *__restrict__ sink) {
    const long stride = (long)gridDim.x * 256 * RF_U;
    rf_v4f acc = {0.f, 0.f, 0.f, 0.f};
    long i = blockIdx.x * 256L * RF_U + threadIdx.x;
    for (; i + (RF_U - 1) * 256 < n4; i += stride) {
        rf_v4f x[RF_U], y[RF_U];
#pragma unroll
        for (int u = 0; u < RF_U; u++) {
            if (MODE != 3) x[u] = __builtin_nontemporal_load(b + i + u * 256);
            if (MODE == 0) y[u] = __builtin_nontemporal_load(c + i + u * 256);
        }
#pragma unroll
        for (int u = 0; u < RF_U; u++) {
            if (MODE == 0) __builtin_nontemporal_store(x[u] + sc * y[u], a + i + u * 256);
            else if (MODE == 1) __builtin_nontemporal_store(x[u], a + i + u * 256);
            else if (MODE == 2) acc += x[u];
            else __builtin_nontemporal_store(rf_v4f{sc, sc, sc, sc}, a + i + u * 256);
        }
    }
    // the last partial iteration: elements i, i + 256, ... below n4
    for (; i < n4; i += 256) {
        if (MODE == 0) a[i] = b[i] + sc * c[i];
        else if (MODE == 1) a[i] = b[i];
        else if (MODE == 2) acc += b[i];
        else a[i] = rf_v4f{sc, sc, sc, sc};
    }
    if (MODE == 2) sink[blockIdx.x * 256 + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

__global__ void roof_fill_kernel(rf_v4f *p, long n4, float v) {
    for (long i = blockIdx.x * 256L + threadIdx.x; i < n4; i += (long)gridDim.x * 256)
        p[i] = rf_v4f{v, v, v, v};
}

// Best time of `reps` launches of f (each bracketed by events), in ms.
template <typename F>
static hipError_t best_ms(F f, int reps, hipStream_t s, float *best) {
    hipEvent_t e0, e1;
    hipError_t err = hipEventCreate(&e0);
    if (err != hipSuccess) return err;
    err = hipEventCreate(&e1);
    if (err != hipSuccess) {
        (void)hipEventDestroy(e0);
        return err;
    }
    *best = 1e30f;
    for (int r = 0; r < reps && err == hipSuccess; r++) {
        err = hipEventRecord(e0, s);
        if (err == hipSuccess) f();
        if (err == hipSuccess) err = hipGetLastError();
        if (err == hipSuccess) err = hipEventRecord(e1, s);
        if (err == hipSuccess) err = hipEventSynchronize(e1);
        float ms = 0.f;
        if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
        if (err == hipSuccess && ms < *best) *best = ms;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return err;
}

hipError_t measure_peak_mfma(int kind, int cus, double *rate, hipStream_t s) {
    void *out = nullptr;
    hipError_t err = hipMalloc(&out, (size_t)cus * 64 * RF_WAVES * 4);
    if (err != hipSuccess) return err;
    const dim3 grid(cus), block(64 * RF_WAVES);
    unsigned seed = 12345u;
    auto launch = [&]() {
        seed += 7919u;
        if (kind == 0) hipLaunchKernelGGL(roof_i8_kernel<true>, grid, block, 0, s, (int *)out, seed);
        else if (kind == 1) hipLaunchKernelGGL(roof_i8_kernel<false>, grid, block, 0, s, (int *)out, seed);
        else hipLaunchKernelGGL(roof_f32_kernel, grid, block, 0, s, (float *)out, seed);
    };
    for (int w = 0; w < 30; w++) launch();  // warm-up: 10-20 ms of load brings the clock up
    float ms = 0.f;
    err = best_ms(launch, 5, s, &ms);
    if (err == hipSuccess) {
        // ops per wave per iteration: four 32x32x32 i8 or eight 16x16x4 f32 MFMAs
        const double per_iter = kind == 2 ? RF_F32_CHAINS * 16.0 * 16 * 4 * 2 : 4 * 32.0 * 32 * 32 * 2;
        const double ops = (double)cus * RF_WAVES * RF_ITERS * per_iter;
        *rate = ops / (ms * 1e-3) / 1e12;
    }
    (void)hipFree(out);
    return err;
}

hipError_t measure_bandwidth(long bytes_per_array, double gbs[4], hipStream_t s) {
    const long n4 = bytes_per_array / 16;
    const int GRID = 4096;
    void *a = nullptr, *b = nullptr, *c = nullptr, *sink = nullptr;
    hipError_t err = hipMalloc(&a, n4 * 16);
    if (err == hipSuccess) err = hipMalloc(&b, n4 * 16);
    if (err == hipSuccess) err = hipMalloc(&c, n4 * 16);
    if (err == hipSuccess) err = hipMalloc(&sink, (size_t)GRID * 256 * 4);
    const dim3 grid(GRID), block(256);
    if (err == hipSuccess) {
        hipLaunchKernelGGL(roof_fill_kernel, grid, block, 0, s, (rf_v4f *)a, n4, 0.f);
        hipLaunchKernelGGL(roof_fill_kernel, grid, block, 0, s, (rf_v4f *)b, n4, 1.f);
        hipLaunchKernelGGL(roof_fill_kernel, grid, block, 0, s, (rf_v4f *)c, n4, 2.f);
        err = hipGetLastError();
    }
    // bytes moved per pass: triad 3 arrays, copy 2, read 1, write 1
    const double arrays[4] = {3.0, 2.0, 1.0, 1.0};
    for (int mode = 0; mode < 4 && err == hipSuccess; mode++) {
        auto pass = [&]() {
            rf_v4f *A = (rf_v4f *)a;
            const rf_v4f *B = (const rf_v4f *)b, *Cc = (const rf_v4f *)c;
            float *Sk = (float *)sink;
            if (mode == 0) hipLaunchKernelGGL(roof_stream_kernel<0>, grid, block, 0, s, A, B, Cc, 3.0f, n4, Sk);
            else if (mode == 1) hipLaunchKernelGGL(roof_stream_kernel<1>, grid, block, 0, s, A, B, Cc, 0.f, n4, Sk);
            else if (mode == 2) hipLaunchKernelGGL(roof_stream_kernel<2>, grid, block, 0, s, A, B, Cc, 0.f, n4, Sk);
            else hipLaunchKernelGGL(roof_stream_kernel<3>, grid, block, 0, s, A, B, Cc, 5.0f, n4, Sk);
        };
        pass();
        float ms = 0.f;
        err = best_ms(pass, 5, s, &ms);
        if (err == hipSuccess) gbs[mode] = arrays[mode] * 16.0 * n4 / (ms * 1e-3) / 1e9;
    }
    if (a) (void)hipFree(a);
    if (b) (void)hipFree(b);
    if (c) (void)hipFree(c);
    if (sink) (void)hipFree(sink);
    return err;
}

// ---- the operand feed of a 128x128-tile INT8 GEMM: L2 -> LDS ----
// One workgroup per 128x128 output tile of an M x N x K product (A M x K
// bytes, B N x K bytes, rows K bytes apart), in the INT8 kernels' tile order
// (xcd_remap + grouped tiles): four waves stream the tile's A and B panels
// over K into a 3-deep LDS ring with global_load_lds_dwordx4, exactly as the
// kernels' producer waves issue them (eight rows of 128 bytes per instruction,
// chunks swizzled), two K tiles in flight, with no products. Its rate is the
// ceiling of those kernels' K loop when the operands must come through L2.
constexpr int RF_FEED_NWP = 4;
__global__ __launch_bounds__(64 * RF_FEED_NWP) void roof_feed_kernel(const int8_t *__restrict__ A,
                                                                     const int8_t *__restrict__ B, int M,
                                                                     int N, int K, int *__restrict__ sink) {
    constexpr int BM = 128, BN = 128, BK = 128, CH = 8, RPI = 8, SIZE_A = BM * BK, STAGE = (BM + BN) * BK;
    constexpr int PIA = BM / (RPI * RF_FEED_NWP), PIB = BN / (RPI * RF_FEED_NWP), PL = PIA + PIB;
    constexpr int STAGES = 3;
    __shared__ __attribute__((aligned(1024))) int8_t lds[STAGES * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, pw = tid >> 6;
    const int nbm = M / BM, nbn = N / BN;
    int bm, bn;
    tile_coords(xcd_remap(blockIdx.x, nbm * nbn), nbm, nbn, 8, bm, bn);
    unsigned voff[PL];
    int ldso[PL];
#pragma unroll
    for (int d = 0; d < PL; d++) {
        const bool isA = d < PIA;
        const int rb = ((isA ? d : d - PIA) * RF_FEED_NWP + pw) * RPI;
        const int r = rb + lane / CH;
        const int c = (lane % CH) ^ ((r >> 1) & (CH - 1));
        voff[d] = (unsigned)((isA ? bm * BM : bn * BN) + r) * (unsigned)K + (unsigned)(c * 16);
        ldso[d] = (isA ? 0 : SIZE_A) + rb * BK;
    }
    const int nk = K / BK;
    for (int t = 0; t < nk; t++) {
        int8_t *stage = lds + (t % STAGES) * STAGE;
#pragma unroll
        for (int d = 0; d < PL; d++)
            __builtin_amdgcn_global_load_lds((const void *)((d < PIA ? A : B) + (long)t * BK + voff[d]),
                                             (__attribute__((address_space(3))) void *)(stage + ldso[d]), 16, 0,
                                             0);
        // two K tiles in flight: "vmcnt <= PL", expcnt and lgkmcnt unchecked
        __builtin_amdgcn_s_waitcnt((PL & 15) | (((PL >> 4) & 3) << 14) | (7 << 4) | (15 << 8));
    }
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
    if (tid == 0) sink[blockIdx.x] = lds[lane];
}

// The same operand stream (addresses and tile order as roof_feed_kernel)
// read into registers instead of LDS: eight waves, each with the loads of two
// K tiles in flight, folded by xor. Equal rates say the ceiling is the path
// from L2 to the CU, not the LDS DMA.
constexpr int RF_VG_NWP = 8;
__global__ __launch_bounds__(64 * RF_VG_NWP) void roof_feed_vgpr_kernel(const int8_t *__restrict__ A,
                                                                        const int8_t *__restrict__ B, int M,
                                                                        int N, int K, int *__restrict__ sink) {
    typedef int rf_v4i __attribute__((ext_vector_type(4)));
    constexpr int BM = 128, BN = 128, BK = 128, CH = 8, RPI = 8;
    constexpr int PIA = BM / (RPI * RF_VG_NWP), PIB = BN / (RPI * RF_VG_NWP), PL = PIA + PIB;
    const int tid = threadIdx.x, lane = tid & 63, pw = tid >> 6;
    const int nbm = M / BM, nbn = N / BN;
    int bm, bn;
    tile_coords(xcd_remap(blockIdx.x, nbm * nbn), nbm, nbn, 8, bm, bn);
    unsigned voff[PL];
#pragma unroll
    for (int d = 0; d < PL; d++) {
        const bool isA = d < PIA;
        const int rb = ((isA ? d : d - PIA) * RF_VG_NWP + pw) * RPI;
        const int r = rb + lane / CH;
        const int c = (lane % CH) ^ ((r >> 1) & (CH - 1));
        voff[d] = (unsigned)((isA ? bm * BM : bn * BN) + r) * (unsigned)K + (unsigned)(c * 16);
    }
    auto load = [&](rf_v4i (&v)[PL], int t) {
#pragma unroll
        for (int d = 0; d < PL; d++)
            v[d] = *reinterpret_cast<const rf_v4i *>((d < PIA ? A : B) + (long)t * BK + voff[d]);
    };
    const int nk = K / BK;
    rf_v4i cur[PL], nxt[PL], acc = {0, 0, 0, 0};
    load(cur, 0);
    for (int t = 0; t < nk; t++) {
        if (t + 1 < nk) load(nxt, t + 1);
#pragma unroll
        for (int d = 0; d < PL; d++) acc ^= cur[d];
#pragma unroll
        for (int d = 0; d < PL; d++) cur[d] = nxt[d];
    }
    if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x5a5a5a5a) sink[blockIdx.x] = 1;
}

hipError_t measure_lds_feed(int M, int N, int K, double *gbs, hipStream_t s, bool vgpr) {
    if (M % 128 || N % 128 || K % 128 || M <= 0 || N <= 0 || K <= 0 || (long)M * K >= (1L << 31) ||
        (long)N * K >= (1L << 31))
        return hipErrorInvalidValue;
    void *a = nullptr, *b = nullptr, *sink = nullptr;
    const int tiles = (M / 128) * (N / 128);
    hipError_t err = hipMalloc(&a, (size_t)M * K);
    if (err == hipSuccess) err = hipMalloc(&b, (size_t)N * K);
    if (err == hipSuccess) err = hipMalloc(&sink, (size_t)tiles * 4);
    if (err == hipSuccess) err = hipMemsetAsync(a, 1, (size_t)M * K, s);
    if (err == hipSuccess) err = hipMemsetAsync(b, 2, (size_t)N * K, s);
    if (err == hipSuccess) {
        // batches of back-to-back launches: a launch alone between two events
        // would add the event overhead (a few us) to a kernel of a few us
        constexpr int BATCH = 50;
        auto pass = [&]() {
            for (int i = 0; i < BATCH; i++) {
                if (vgpr)
                    hipLaunchKernelGGL(roof_feed_vgpr_kernel, dim3(tiles), dim3(64 * RF_VG_NWP), 0, s,
                                       (const int8_t *)a, (const int8_t *)b, M, N, K, (int *)sink);
                else
                    hipLaunchKernelGGL(roof_feed_kernel, dim3(tiles), dim3(64 * RF_FEED_NWP), 0, s,
                                       (const int8_t *)a, (const int8_t *)b, M, N, K, (int *)sink);
            }
        };
        pass();
        float ms = 0.f;
        err = best_ms(pass, 5, s, &ms);
        if (err == hipSuccess) *gbs = (double)tiles * 256.0 * K * BATCH / (ms * 1e-3) / 1e9;
    }
    if (a) (void)hipFree(a);
    if (b) (void)hipFree(b);
    if (sink) (void)hipFree(sink);
    return err;
}

}  // namespace pcl
