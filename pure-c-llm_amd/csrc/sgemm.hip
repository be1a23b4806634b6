// sgemm.hip -- FP32 GEMM on the CDNA4 f32 matrix cores (v_mfma_f32_32x32x2f32).
//
// One kernel template covers every row-major layout the reference uses:
//   NN  C = A.B + bias          tensor.c:34-53, train.c:181-211, gpu_kernels.cu:112-120
//   NT  C ?= A.B^T              train.c:219-232 (dX), 412-423 (head), gpu_kernels.cu:122-129
//   TN  C += A^T.B              train.c:234-242 (dW), 434-446 (dwte), gpu_kernels.cu:131-138
// An operand is either "K-contiguous" (consecutive k adjacent in memory) or
// "MN-contiguous"; each is staged through LDS in the layout it has in HBM, so
// global loads are 16-byte vectors along the contiguous dimension for every
// layout and no transpose pass exists.
//
// Tiling: 256 threads = 4 waves in a 2x2 grid; a wave owns a (BM/2)x(BN/2)
// sub-tile made of 32x32 MFMA blocks whose accumulators live in AGPR/VGPRs.
// K advances in BK-deep LDS tiles, double-buffered: the next tile's global
// loads are issued before the current tile's MFMAs and written to the other
// LDS buffer afterwards, one barrier per tile.
//
// K order inside an 8-deep chunk: the MFMA consumes k pairs (k = lane/32).
// Lane group g (= lane/32) at MFMA step s (0..3) feeds k = 4g + s, the same
// for A and B, so a K-contiguous operand is read as one 16-byte LDS vector
// per chunk. The sum over k is unchanged; only fp32 rounding order differs
// from the reference's sequential loop (checked to 1e-4 in the tests).
#include "internal.h"

namespace pcl {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int SG_THREADS = 256;
constexpr int SG_PAD_K = 4;   // floats of padding per K-contiguous LDS row
constexpr int SG_PAD_MN = 4;  // floats of padding per MN-contiguous LDS row

template <int ROWS, int BK, bool KC>
struct OperandTile {
    // LDS footprint of one buffer, in floats
    static constexpr int LD = KC ? (BK + SG_PAD_K) : (ROWS + SG_PAD_MN);
    static constexpr int SIZE = KC ? ROWS * LD : BK * LD;
    // 4-float vectors per tile and per thread
    static constexpr int VECS = ROWS * BK / 4;
    static constexpr int PER_THREAD = VECS / SG_THREADS;
    static_assert(VECS % SG_THREADS == 0, "tile must split evenly over 256 threads");

    // global -> registers. rows0: first row (m or n) of the tile; k0: first k.
    template <bool VEC>
    __device__ __forceinline__ static void load(v4f (&r)[PER_THREAD], const float *__restrict__ P,
                                                long ld, int rows0, int nrows, int k0, int K,
                                                int tid) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            int e = tid + i * SG_THREADS;
            int row, k;
            if (KC) {
                row = e / (BK / 4);
                k = (e % (BK / 4)) * 4;
            } else {
                k = e / (ROWS / 4);
                row = (e % (ROWS / 4)) * 4;
            }
            int grow = rows0 + row, gk = k0 + k;
            v4f v = {0.f, 0.f, 0.f, 0.f};
            if (VEC) {
                // VEC guarantees the 4-vector lies entirely inside or outside
                bool ok = KC ? (grow < nrows && gk < K) : (gk < K && grow < nrows);
                if (ok) {
                    const float *src = KC ? P + (long)grow * ld + gk : P + (long)gk * ld + grow;
                    v = *reinterpret_cast<const v4f *>(src);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    int rr = KC ? grow : grow + j;
                    int kk = KC ? gk + j : gk;
                    if (rr < nrows && kk < K) v[j] = P[KC ? (long)rr * ld + kk : (long)kk * ld + rr];
                }
            }
            r[i] = v;
        }
    }

    __device__ __forceinline__ static void store(const v4f (&r)[PER_THREAD], float *lds, int tid) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            int e = tid + i * SG_THREADS;
            int off;
            if (KC) off = (e / (BK / 4)) * LD + (e % (BK / 4)) * 4;
            else off = (e / (ROWS / 4)) * LD + (e % (ROWS / 4)) * 4;
            *reinterpret_cast<v4f *>(lds + off) = r[i];
        }
    }

    // MFMA operand fetch for chunk kc: f[s] is the value for MFMA step s.
    // row: tile row (m or n) this lane feeds; g: lane group (0/1).
    __device__ __forceinline__ static v4f frag(const float *lds, int row, int kc, int g) {
        if (KC) {
            return *reinterpret_cast<const v4f *>(lds + row * LD + kc * 8 + 4 * g);
        } else {
            v4f f;
#pragma unroll
            for (int s = 0; s < 4; s++) f[s] = lds[(kc * 8 + 4 * g + s) * LD + row];
            return f;
        }
    }
};

template <int BM, int BN, int BK, bool A_KC, bool B_KC, bool VEC>
__global__ __launch_bounds__(SG_THREADS) void sgemm_mfma_kernel(
    const float *__restrict__ A, long lda, const float *__restrict__ B, long ldb,
    const float *__restrict__ bias, float *__restrict__ C, long ldc, int M, int N, int K,
    int accumulate) {
    using TA = OperandTile<BM, BK, A_KC>;
    using TB = OperandTile<BN, BK, B_KC>;
    constexpr int WTM = BM / 2, WTN = BN / 2;   // wave tile
    constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 MFMA blocks per wave
    static_assert(BK % 8 == 0, "BK must be a multiple of 8");

    // two buffers, each [A tile | B tile]
    constexpr int BUF = TA::SIZE + TB::SIZE;
    __shared__ __attribute__((aligned(16))) float lds[2 * BUF];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int r32 = lane & 31, g = lane >> 5;

    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int bm, bn;
    tile_coords(xcd_remap(blockIdx.x, nbm * nbn), nbm, nbn, 8, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;

    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    v4f ra[TA::PER_THREAD], rb[TB::PER_THREAD];
    const int nk = (K + BK - 1) / BK;

    if (nk > 0) {
        TA::template load<VEC>(ra, A, lda, m0, M, 0, K, tid);
        TB::template load<VEC>(rb, B, ldb, n0, N, 0, K, tid);
        TA::store(ra, lds, tid);
        TB::store(rb, lds + TA::SIZE, tid);
    }
    __syncthreads();

    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            TA::template load<VEC>(ra, A, lda, m0, M, (kt + 1) * BK, K, tid);
            TB::template load<VEC>(rb, B, ldb, n0, N, (kt + 1) * BK, K, tid);
        }
        const float *la = lds + cur * BUF;
        const float *lb = la + TA::SIZE;
#pragma unroll
        for (int kc = 0; kc < BK / 8; kc++) {
            v4f fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) fa[i] = TA::frag(la, wm * WTM + i * 32 + r32, kc, g);
#pragma unroll
            for (int j = 0; j < TN; j++) fb[j] = TB::frag(lb, wn * WTN + j * 32 + r32, kc, g);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[j][s],
                                                                         acc[i][j], 0, 0, 0);
        }
        if (more) {
            TA::store(ra, lds + (cur ^ 1) * BUF, tid);
            TB::store(rb, lds + (cur ^ 1) * BUF + TA::SIZE, tid);
        }
        __syncthreads();
    }

    // Epilogue. 32x32 accumulator layout: register v of lane l holds
    // row (v/4)*8 + (l/32)*4 + v%4, column l%32 of the block.
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int col = n0 + wn * WTN + j * 32 + r32;
        if (col >= N) continue;
        const float bv = bias ? bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = m0 + wm * WTM + i * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
                if (row < M) {
                    float *c = C + (long)row * ldc + col;
                    float out = acc[i][j][v] + bv;
                    if (accumulate) out = *c + out;
                    *c = out;
                }
            }
        }
    }
}

template <int BM, int BN, int BK, bool A_KC, bool B_KC>
static hipError_t launch_cfg(bool vec, int M, int N, int K, const float *A, long lda,
                             const float *B, long ldb, const float *bias, int accumulate, float *C,
                             long ldc, hipStream_t stream) {
    const int nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (nblk == 0) return hipSuccess;
    dim3 grid(nblk), block(SG_THREADS);
    if (vec)
        hipLaunchKernelGGL((sgemm_mfma_kernel<BM, BN, BK, A_KC, B_KC, true>), grid, block, 0,
                           stream, A, lda, B, ldb, bias, C, ldc, M, N, K, accumulate);
    else
        hipLaunchKernelGGL((sgemm_mfma_kernel<BM, BN, BK, A_KC, B_KC, false>), grid, block, 0,
                           stream, A, lda, B, ldb, bias, C, ldc, M, N, K, accumulate);
    return hipGetLastError();
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <bool A_KC, bool B_KC>
static hipError_t dispatch_layout(int M, int N, int K, const float *A, long lda, const float *B,
                                  long ldb, const float *bias, int accumulate, float *C, long ldc,
                                  hipStream_t stream) {
    // 16-byte vector loads need the contiguous extent and leading dimension to
    // be multiples of 4 floats and 16-byte aligned bases.
    bool vec = aligned16(A) && aligned16(B) && lda % 4 == 0 && ldb % 4 == 0 &&
               (A_KC ? K % 4 == 0 : M % 4 == 0) && (B_KC ? K % 4 == 0 : N % 4 == 0);
    // 128x128 tiles when they still give >= 2 workgroups per CU (512 on the
    // 256-CU MI355X); 64x64 otherwise so small GEMMs fill the chip.
    long big = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (big >= 512)
        return launch_cfg<128, 128, 16, A_KC, B_KC>(vec, M, N, K, A, lda, B, ldb, bias, accumulate,
                                                    C, ldc, stream);
    return launch_cfg<64, 64, 16, A_KC, B_KC>(vec, M, N, K, A, lda, B, ldb, bias, accumulate, C,
                                              ldc, stream);
}

hipError_t launch_sgemm(bool a_kcontig, bool b_kcontig, int M, int N, int K, const float *A,
                        long lda, const float *B, long ldb, const float *bias, int accumulate,
                        float *C, long ldc, hipStream_t stream) {
    if (a_kcontig && !b_kcontig)
        return dispatch_layout<true, false>(M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, stream);
    if (a_kcontig && b_kcontig)
        return dispatch_layout<true, true>(M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, stream);
    if (!a_kcontig && !b_kcontig)
        return dispatch_layout<false, false>(M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, stream);
    return dispatch_layout<false, true>(M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, stream);
}

}  // namespace pcl
