// igemm.hip -- u8 x s8 -> int32 GEMM on the CDNA4 int8 matrix cores
// (v_mfma_i32_32x32x32_i8), with the dequantising epilogue.
//
// Reference semantics (gemm_bench.c:212-285): activations are u8 with a +128
// offset, weights s8; vpdpbusd forms acc = sum Au*Bq and the kernel subtracts
// corr = 128*colsum, i.e. v = sum (Au-128)*Bq (gemm_bench.c:216-217, 274).
// The i8 MFMA is signed x signed, so A is re-centred on load with Au ^ 0x80,
// which is exactly Au-128 as an s8 byte: the MFMA then produces v directly,
// bit-exact, with no column-sum pass. An optional per-column int32 offset
// reproduces a caller-supplied `corr` (off = 128*colsum - corr).
// Dequant (gemm_bench.c:272-275, dq precomputed at :378) is fp32 RNE in the
// same order: C = float(v) * dq with dq = sb[n] or sa[m]*sb[n].
//
// Layouts: A is M x K u8 row-major (K-contiguous). B is pre-packed N x Kp s8
// (K-contiguous per output column; the reference packs its weights offline
// too, gemm_bench.c:218-220). Both tiles are therefore staged identically:
// 16-byte global loads along K into [row][BK+16] LDS rows, read back as one
// 16-byte MFMA operand per lane. The +16-byte row pad puts 8 consecutive rows
// in 8 distinct 16-byte bank groups (conflict-free ds_read_b128).
//
// K order: the 32x32x32 MFMA takes 16 bytes per lane; lane group g = lane/32
// supplies k = 16g..16g+15 of each 32-deep chunk for A and for B alike, so
// the integer sum is the same whatever order the hardware reduces it in.
#include "internal.h"

namespace pcl {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int IG_THREADS = 256;
constexpr int IG_PAD = 16;  // bytes of padding per LDS row

template <int ROWS, int BK>
struct ITile {
    static constexpr int LD = BK + IG_PAD;  // bytes per LDS row
    static constexpr int SIZE = ROWS * LD;  // bytes per buffer
    static constexpr int VECS = ROWS * BK / 16;
    static constexpr int PER_THREAD = VECS / IG_THREADS;
    static_assert(VECS % IG_THREADS == 0, "tile must split evenly over 256 threads");

    // XOR: 0x80808080 for the u8 activations (re-centre to s8), 0 for weights.
    __device__ __forceinline__ static void load(v4i (&r)[PER_THREAD], const int8_t *__restrict__ P,
                                                long ld, int rows0, int nrows, int k0, int K,
                                                int tid, unsigned xor_mask) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            int e = tid + i * IG_THREADS;
            int row = e / (BK / 16), k = (e % (BK / 16)) * 16;
            int grow = rows0 + row, gk = k0 + k;
            v4i v = {0, 0, 0, 0};
            if (grow < nrows && gk < K)
                v = *reinterpret_cast<const v4i *>(P + (long)grow * ld + gk);
            // rows >= nrows and k >= K load zero before the XOR: out-of-range
            // A rows only feed discarded outputs, and k >= K meets B == 0.
            v ^= (int)xor_mask;
            r[i] = v;
        }
    }

    __device__ __forceinline__ static void store(const v4i (&r)[PER_THREAD], int8_t *lds, int tid) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            int e = tid + i * IG_THREADS;
            int off = (e / (BK / 16)) * LD + (e % (BK / 16)) * 16;
            *reinterpret_cast<v4i *>(lds + off) = r[i];
        }
    }

    __device__ __forceinline__ static v4i frag(const int8_t *lds, int row, int kc, int g) {
        return *reinterpret_cast<const v4i *>(lds + row * LD + kc * 32 + 16 * g);
    }
};

template <int BM, int BN, int BK, int OUT>
__global__ __launch_bounds__(IG_THREADS) void igemm_mfma_kernel(
    const uint8_t *__restrict__ A, long lda, const int8_t *__restrict__ B, long ldb,
    const int32_t *__restrict__ col_off, const float *__restrict__ sa,
    const float *__restrict__ sb, void *__restrict__ Cv, long ldc, int M, int N, int K) {
    using TA = ITile<BM, BK>;
    using TB = ITile<BN, BK>;
    constexpr int WTM = BM / 2, WTN = BN / 2;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(BK % 32 == 0, "BK must be a multiple of 32");

    // two buffers, each [A tile | B tile]
    constexpr int BUF = TA::SIZE + TB::SIZE;
    __shared__ __attribute__((aligned(16))) int8_t lds[2 * BUF];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int r32 = lane & 31, g = lane >> 5;

    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int bm, bn;
    tile_coords(xcd_remap(blockIdx.x, nbm * nbn), nbm, nbn, 8, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;

    const int8_t *A8 = reinterpret_cast<const int8_t *>(A);

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0;

    v4i ra[TA::PER_THREAD], rb[TB::PER_THREAD];
    const int nk = (K + BK - 1) / BK;
    if (nk > 0) {
        TA::load(ra, A8, lda, m0, M, 0, K, tid, 0x80808080u);
        TB::load(rb, B, ldb, n0, N, 0, K, tid, 0u);
        TA::store(ra, lds, tid);
        TB::store(rb, lds + TA::SIZE, tid);
    }
    __syncthreads();

    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            TA::load(ra, A8, lda, m0, M, (kt + 1) * BK, K, tid, 0x80808080u);
            TB::load(rb, B, ldb, n0, N, (kt + 1) * BK, K, tid, 0u);
        }
        const int8_t *la = lds + cur * BUF;
        const int8_t *lb = la + TA::SIZE;
#pragma unroll
        for (int kc = 0; kc < BK / 32; kc++) {
            v4i fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) fa[i] = TA::frag(la, wm * WTM + i * 32 + r32, kc, g);
#pragma unroll
            for (int j = 0; j < TN; j++) fb[j] = TB::frag(lb, wn * WTN + j * 32 + r32, kc, g);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            TA::store(ra, lds + (cur ^ 1) * BUF, tid);
            TB::store(rb, lds + (cur ^ 1) * BUF + TA::SIZE, tid);
        }
        __syncthreads();
    }

    // Epilogue: register v of lane l holds row (v/4)*8 + (l/32)*4 + v%4,
    // column l%32 of each 32x32 block.
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int col = n0 + wn * WTN + j * 32 + r32;
        if (col >= N) continue;
        const unsigned off = col_off ? (unsigned)col_off[col] : 0u;
        const float sbv = (OUT != 0) ? sb[col] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = m0 + wm * WTM + i * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
                if (row >= M) continue;
                if (OUT == 0) {
                    reinterpret_cast<int32_t *>(Cv)[(long)row * ldc + col] = acc[i][j][v];
                } else {
                    const int32_t vv = (int32_t)((unsigned)acc[i][j][v] + off);
                    const float dq = (OUT == 2) ? sa[row] * sbv : sbv;
                    reinterpret_cast<float *>(Cv)[(long)row * ldc + col] = (float)vv * dq;
                }
            }
        }
    }
}

template <int BM, int BN, int BK>
static hipError_t launch_icfg(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                              const int8_t *B, long ldb, const int32_t *col_off, const float *sa,
                              const float *sb, void *C, long ldc, hipStream_t stream) {
    const int nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (nblk == 0) return hipSuccess;
    dim3 grid(nblk), block(IG_THREADS);
    switch (out_mode) {
        case 0:
            hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, BK, 0>), grid, block, 0, stream, A, lda,
                               B, ldb, col_off, sa, sb, C, ldc, M, N, K);
            break;
        case 1:
            hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, BK, 1>), grid, block, 0, stream, A, lda,
                               B, ldb, col_off, sa, sb, C, ldc, M, N, K);
            break;
        default:
            hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, BK, 2>), grid, block, 0, stream, A, lda,
                               B, ldb, col_off, sa, sb, C, ldc, M, N, K);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_igemm(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                        const int8_t *Bpk, long ldb, const int32_t *col_off, const float *sa,
                        const float *sb, void *C, long ldc, hipStream_t stream) {
    long big = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (big >= 256)
        return launch_icfg<128, 128, 64>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C,
                                         ldc, stream);
    return launch_icfg<64, 64, 64>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C, ldc,
                                   stream);
}

// Copy A into a K16-wide buffer padded with 0x80 (zero after re-centring; the
// packed weights are zero there as well).
__global__ void pad_a_u8_kernel(const uint8_t *__restrict__ A, long lda, int M, int K,
                                uint8_t *__restrict__ dst, int K16) {
    long total = (long)M * K16;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total;
         i += (long)gridDim.x * blockDim.x) {
        int m = (int)(i / K16), k = (int)(i % K16);
        dst[i] = k < K ? A[(long)m * lda + k] : (uint8_t)0x80;
    }
}

hipError_t launch_pad_a_u8(const uint8_t *A, long lda, int M, int K, uint8_t *dst, int K16,
                           hipStream_t stream) {
    long total = (long)M * K16;
    if (total == 0) return hipSuccess;
    int blocks = (int)((total + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(pad_a_u8_kernel, dim3(blocks), dim3(256), 0, stream, A, lda, M, K, dst, K16);
    return hipGetLastError();
}

}  // namespace pcl
