// quant.hip -- the INT8 rung's quantisers and weight packers on the GPU.
//
// Rules of gemm_bench.c:225-259, kept operation for operation so the bytes
// match the CPU restatement exactly:
//   amax starts at 1e-8f; scale = amax * fl(1/127); inv = 1.0f / scale;
//   q = clamp(round_half_away(x * inv), -127, 127)
//   activations: Au = q + 128, K padded to Kpad with 128 (quantize_A :225-236)
//   weights: per output column (quantize_B_pack :238-259), colsum[n] = sum q
// The source writes amax/127.0f; the reference is built with -ffast-math
// (README.md:104), which turns that into amax * fl(1/127), so its bytes come
// from the multiplication and so do ours. 1.0f/scale is a correctly rounded
// division (hipcc's default for fp32 `/`), and roundf rounds half away from
// zero like lroundf.
//
// Output layouts for weights: the native packed layout (N rows of ldb bytes,
// K-contiguous, zero beyond K) read by igemm/igemv, or the reference VNNI
// panel layout Bp[p*(Kpad/4)*64 + kg*64 + i*4 + j] = Bq[kg*4+j][p*16+i].
#include "internal.h"

namespace pcl {

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// ---------------------------------------------------------- per tensor ----
__global__ void amax_init_kernel(unsigned *amax_bits) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *amax_bits = __float_as_uint(AMAX_INIT);
}

// |x| >= 0, so the IEEE bit patterns order like the values: atomicMax on the
// bits is the float max (order-independent, hence exact).
__global__ void amax_tensor_kernel(const float *__restrict__ A, long n, unsigned *amax_bits) {
    float m = 0.f;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n;
         i += (long)gridDim.x * blockDim.x)
        m = fmaxf(m, fabsf(A[i]));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) atomicMax(amax_bits, __float_as_uint(m));
}

__global__ void quantize_a_tensor_kernel(const float *__restrict__ A, int M, int K,
                                         uint8_t *__restrict__ Au, int Kpad,
                                         const unsigned *__restrict__ amax_bits,
                                         float *__restrict__ scale_dev) {
    const float amax = __uint_as_float(*amax_bits);
    const float scale = amax * RCP127, inv = 1.0f / scale;
    if (blockIdx.x == 0 && threadIdx.x == 0 && scale_dev) *scale_dev = scale;
    const long total = (long)M * Kpad;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total;
         i += (long)gridDim.x * blockDim.x) {
        const int m = (int)(i / Kpad), k = (int)(i % Kpad);
        const int q = k < K ? quant_q(A[(long)m * K + k], inv) : 0;
        Au[i] = (uint8_t)(q + 128);
    }
}

static int grid_for(long n) {
    long b = (n + 255) / 256;
    if (b > 2048) b = 2048;
    if (b < 1) b = 1;
    return (int)b;
}

hipError_t launch_quantize_a_tensor(const float *A, int M, int K, uint8_t *Au, int Kpad,
                                    float *scale_dev, unsigned *amax_bits, hipStream_t s) {
    hipLaunchKernelGGL(amax_init_kernel, dim3(1), dim3(64), 0, s, amax_bits);
    long n = (long)M * K;
    if (n > 0) hipLaunchKernelGGL(amax_tensor_kernel, dim3(grid_for(n)), dim3(256), 0, s, A, n, amax_bits);
    long t = (long)M * Kpad;
    hipLaunchKernelGGL(quantize_a_tensor_kernel, dim3(grid_for(t)), dim3(256), 0, s, A, M, K, Au,
                       Kpad, amax_bits, scale_dev);
    return hipGetLastError();
}

// ------------------------------------------------------------- per row ----
__global__ __launch_bounds__(256) void quantize_a_rows_kernel(const float *__restrict__ A, int K,
                                                              uint8_t *__restrict__ Au, int Kpad,
                                                              float *__restrict__ sa) {
    __shared__ float wmax[4];
    const int m = blockIdx.x;
    const float *a = A + (long)m * K;
    float mx = 0.f;
    for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(a[k]));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float amax = fmaxf(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])), AMAX_INIT);
    const float scale = amax * RCP127, inv = 1.0f / scale;
    if (threadIdx.x == 0) sa[m] = scale;
    uint8_t *o = Au + (long)m * Kpad;
    for (int k = threadIdx.x; k < Kpad; k += 256) {
        const int q = k < K ? quant_q(a[k], inv) : 0;
        o[k] = (uint8_t)(q + 128);
    }
}

hipError_t launch_quantize_a_rows(const float *A, int M, int K, uint8_t *Au, int Kpad, float *sa,
                                  hipStream_t s) {
    if (M <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_a_rows_kernel, dim3(M), dim3(256), 0, s, A, K, Au, Kpad, sa);
    return hipGetLastError();
}

// ---------------------------------------------------- weights per column ----
// One block per 64-column strip. Phase 1: column amax -> bscale. Phase 2:
// 64x64 tiles read along N (coalesced), quantised, transposed through LDS and
// written K-contiguous (native) or in VNNI panels. colsum sums exact ints.
__device__ __forceinline__ long vnni_index(int n, int k, int Kpad) {
    return (long)(n / 16) * (Kpad / 4) * 64 + (long)(k / 4) * 64 + (n % 16) * 4 + (k % 4);
}

template <bool QUANT>
__global__ __launch_bounds__(256) void pack_cols_kernel(const float *__restrict__ Bf,
                                                        const int8_t *__restrict__ Bs, long ldb_in,
                                                        int K, int N, int layout,
                                                        int8_t *__restrict__ dst, long ldb,
                                                        int Kpad, float *__restrict__ bscale,
                                                        int32_t *__restrict__ colsum) {
    __shared__ float cmax[4][64];
    __shared__ float cinv[64];
    __shared__ int csum[64];
    __shared__ int8_t tile[64][64 + 4];  // [column][k]
    const int tid = threadIdx.x;
    const int c = tid & 63, rp = tid >> 6;
    const int n0 = blockIdx.x * 64, n = n0 + c;

    if (QUANT) {
        float mx = 0.f;
        if (n < N)
            for (int k = rp; k < K; k += 4) mx = fmaxf(mx, fabsf(Bf[(long)k * ldb_in + n]));
        cmax[rp][c] = mx;
    }
    if (tid < 64) csum[tid] = 0;
    __syncthreads();
    if (QUANT && tid < 64) {
        float bmax = fmaxf(fmaxf(fmaxf(cmax[0][tid], cmax[1][tid]), fmaxf(cmax[2][tid], cmax[3][tid])),
                           AMAX_INIT);
        const float sc = bmax * RCP127;
        cinv[tid] = 1.0f / sc;
        if (n0 + tid < N) bscale[n0 + tid] = sc;
    }
    __syncthreads();

    const int kext = layout == 0 ? (int)ldb : Kpad;  // bytes written per column
    int my_sum = 0;
    for (int k0 = 0; k0 < kext; k0 += 64) {
        // load: thread (c, rp) handles k = k0 + rp + 4i, i < 16
#pragma unroll 4
        for (int i = 0; i < 16; i++) {
            const int kk = rp + 4 * i, k = k0 + kk;
            int q = 0;
            if (n < N && k < K) {
                if (QUANT) q = quant_q(Bf[(long)k * ldb_in + n], cinv[c]);
                else q = Bs[(long)k * ldb_in + n];
            }
            my_sum += q;
            tile[c][kk] = (int8_t)q;
        }
        __syncthreads();
        if (layout == 0) {
            // 64 columns x 4 chunks of 16 bytes
            const int cc = tid >> 2, ch = (tid & 3) * 16;
            const int nn = n0 + cc;
            if (nn < N && k0 + ch < kext) {
                int8_t *o = dst + (long)nn * ldb + k0 + ch;
#pragma unroll
                for (int e = 0; e < 16; e++)
                    if (k0 + ch + e < kext) o[e] = tile[cc][ch + e];
            }
        } else {
            for (int e = tid; e < 64 * 64; e += 256) {
                const int cc = e & 63, kk = e >> 6;
                const int nn = n0 + cc, k = k0 + kk;
                if (nn < N && k < kext) dst[vnni_index(nn, k, Kpad)] = tile[cc][kk];
            }
        }
        __syncthreads();
    }
    atomicAdd(&csum[c], my_sum);
    __syncthreads();
    if (colsum && tid < 64 && n0 + tid < N) colsum[n0 + tid] = csum[tid];
}

hipError_t launch_quantize_b_cols(const float *B, int K, int N, int layout, int8_t *dst, long ldb,
                                  int Kpad, float *bscale, int32_t *colsum, hipStream_t s) {
    if (N <= 0) return hipSuccess;
    int strips = (N + 63) / 64;
    hipLaunchKernelGGL((pack_cols_kernel<true>), dim3(strips), dim3(256), 0, s, B,
                       (const int8_t *)nullptr, (long)N, K, N, layout, dst, ldb, Kpad, bscale,
                       colsum);
    return hipGetLastError();
}

hipError_t launch_pack_b_s8(const int8_t *B, long ldb_in, int K, int N, int8_t *Bpk, long ldb,
                            int32_t *colsum, hipStream_t s) {
    if (N <= 0) return hipSuccess;
    int strips = (N + 63) / 64;
    hipLaunchKernelGGL((pack_cols_kernel<false>), dim3(strips), dim3(256), 0, s,
                       (const float *)nullptr, B, ldb_in, K, N, 0, Bpk, ldb, 0, (float *)nullptr,
                       colsum);
    return hipGetLastError();
}

// VNNI panels -> native rows. Thread (c = tid%64, rp = tid/64) moves the
// 4-byte words kg = rp + 4i of column n0+c: in VNNI the 4 k-bytes of one
// column are adjacent, so each move is one 32-bit load and store.
__global__ __launch_bounds__(256) void vnni_to_native_kernel(const int8_t *__restrict__ Bp, int K,
                                                             int Kpad, int N,
                                                             int8_t *__restrict__ Bpk, long ldb,
                                                             int32_t *__restrict__ colsum) {
    __shared__ int csum[64];
    const int tid = threadIdx.x;
    const int c = tid & 63, rp = tid >> 6;
    const int n = blockIdx.x * 64 + c;
    if (tid < 64) csum[tid] = 0;
    __syncthreads();
    int my_sum = 0;
    if (n < N) {
        const int nwords = (int)(ldb / 4);
        for (int kg = rp; kg < nwords; kg += 4) {
            union { int w; int8_t b[4]; } u;
            u.w = 0;
            const int k = kg * 4;
            if (k < K) {  // k < K <= Kpad: the word lies inside the panel
                u.w = *reinterpret_cast<const int *>(Bp + vnni_index(n, k, Kpad));
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (k + j >= K) u.b[j] = 0;
            }
            my_sum += u.b[0] + u.b[1] + u.b[2] + u.b[3];
            *reinterpret_cast<int *>(Bpk + (long)n * ldb + k) = u.w;
        }
    }
    atomicAdd(&csum[c], my_sum);
    __syncthreads();
    if (colsum && tid < 64 && blockIdx.x * 64 + tid < N) colsum[blockIdx.x * 64 + tid] = csum[tid];
}

hipError_t launch_pack_b_vnni(const int8_t *Bp, int K, int Kpad, int N, int8_t *Bpk, long ldb,
                              int32_t *colsum, hipStream_t s) {
    if (N <= 0) return hipSuccess;
    hipLaunchKernelGGL(vnni_to_native_kernel, dim3((N + 63) / 64), dim3(256), 0, s, Bp, K, Kpad, N,
                       Bpk, ldb, colsum);
    return hipGetLastError();
}

__global__ void corr_to_offset_kernel(const int32_t *__restrict__ colsum,
                                      const int32_t *__restrict__ corr, int32_t *__restrict__ off,
                                      int N) {
    int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n < N) off[n] = (int32_t)(128u * (unsigned)colsum[n] - (unsigned)corr[n]);
}

hipError_t launch_corr_to_offset(const int32_t *colsum, const int32_t *corr, int32_t *off, int N,
                                 hipStream_t s) {
    if (N <= 0) return hipSuccess;
    hipLaunchKernelGGL(corr_to_offset_kernel, dim3((N + 255) / 256), dim3(256), 0, s, colsum, corr,
                       off, N);
    return hipGetLastError();
}

}  // namespace pcl
