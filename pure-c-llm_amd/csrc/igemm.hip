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
// (K-contiguous per output column, zero beyond K; the reference packs its
// weights offline too, gemm_bench.c:218-220). Both tiles are staged alike:
// 16-byte global loads along K (8 or 16 consecutive lanes cover one 128/256-
// byte row segment) into LDS rows of BK bytes with no padding. The 16-byte
// chunk c of row r is stored at chunk c ^ (r & 7): the 8 lanes of one
// ds_read_b128 phase (8 consecutive rows, same chunk) then hit 8 different
// 16-byte bank groups, and the stores of 8 lanes writing one row stay a
// contiguous 128 bytes -- conflict-free both ways without padding bytes.
//
// Pipeline: the next K tile's global loads are issued into registers before
// the current tile's MFMAs and written to the other LDS buffer after them;
// one barrier per BK-deep tile. BK is 128 or 256 bytes so that every barrier
// is amortised over 16-64 MFMAs per wave. The loads are branch-free: row
// indices past M (or N) are clamped to the last row -- they only feed output
// rows (columns) that are never stored -- and an A chunk past K is clamped to
// the last in-bounds chunk, whose bytes meet the zero padding of the packed
// weights (rows of Kp = roundup(K, 256) bytes and BK divides 256, so a B
// chunk never leaves its row). Nothing reads a loaded value before the MFMAs, so the loads of the
// next tile stay in flight during the current tile's math; the A re-centring
// XOR happens when the registers are written to LDS.
//
// K order: the 32x32x32 MFMA takes 16 bytes per lane; lane group g = lane/32
// supplies k = 16g..16g+15 of each 32-deep chunk for A and for B alike, so
// the integer sum is the same whatever order the hardware reduces it in.
#include "internal.h"

namespace pcl {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// One operand tile: ROWS rows x BK bytes, loaded by NT threads.
template <int ROWS, int BK, int NT>
struct ITile {
    static constexpr int CPR = BK / 16;           // 16-byte chunks per row
    static constexpr int SIZE = ROWS * BK;        // bytes per LDS buffer
    static constexpr int PER_THREAD = ROWS * CPR / NT;
    static_assert(CPR >= 8, "the XOR swizzle needs >= 8 chunks per row");
    static_assert(ROWS * CPR % NT == 0, "tile must split evenly over the threads");

    __device__ __forceinline__ static int lds_off(int r, int c) {
        return r * BK + ((c ^ (r & 7)) << 4);
    }

    // Unconditional 16-byte loads: row clamped to nrows-1, k chunk clamped to
    // kmax (the last chunk that may be read in this operand's rows).
    __device__ __forceinline__ static void load(v4i (&v)[PER_THREAD], const int8_t *__restrict__ P,
                                                long ld, int rows0, int nrows, int k0, int kmax,
                                                int tid) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            const int e = tid + i * NT;
            const int r = e / CPR, c = e % CPR;
            const int grow = min(rows0 + r, nrows - 1), gk = min(k0 + c * 16, kmax);
            v[i] = *reinterpret_cast<const v4i *>(P + (long)grow * ld + gk);
        }
    }

    __device__ __forceinline__ static void store(const v4i (&v)[PER_THREAD], int8_t *lds, int tid,
                                                 int xor_mask) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            const int e = tid + i * NT;
            *reinterpret_cast<v4i *>(lds + lds_off(e / CPR, e % CPR)) = v[i] ^ xor_mask;
        }
    }

    // MFMA operand for lane (row, g) of 32-deep chunk kc.
    __device__ __forceinline__ static v4i frag(const int8_t *lds, int row, int kc, int g) {
        return *reinterpret_cast<const v4i *>(lds + lds_off(row, kc * 2 + g));
    }
};

template <int BM, int BN, int BK, int WM, int WN, int OUT>
__global__ __launch_bounds__(64 * WM * WN) void igemm_mfma_kernel(
    const uint8_t *__restrict__ A, long lda, const int8_t *__restrict__ B, long ldb,
    const int32_t *__restrict__ col_off, const float *__restrict__ sa,
    const float *__restrict__ sb, void *__restrict__ Cv, long ldc, int M, int N, int K) {
    constexpr int NT = 64 * WM * WN;
    using TA = ITile<BM, BK, NT>;
    using TB = ITile<BN, BK, NT>;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1 && BK % 32 == 0 && 256 % BK == 0, "bad tile configuration");
    constexpr int BUF = TA::SIZE + TB::SIZE;

    // two buffers, each [A tile | B tile]
    __shared__ __attribute__((aligned(16))) int8_t lds[2 * BUF];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int r32 = lane & 31, g = lane >> 5;

    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int bm, bn;
    tile_coords(xcd_remap(blockIdx.x, nbm * nbn), nbm, nbn, 8, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;

    const int8_t *A8 = reinterpret_cast<const int8_t *>(A);
    const int XA = (int)0x80808080u;

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0;

    v4i ra[TA::PER_THREAD], rb[TB::PER_THREAD];
    const int nk = (K + BK - 1) / BK;
    const int ka_max = K - 16;         // K % 16 == 0, K > 0 whenever nk > 0
    const int kb_max = nk * BK - 16;   // < Kp: B rows are zero-padded past K
    if (nk > 0) {
        TA::load(ra, A8, lda, m0, M, 0, ka_max, tid);
        TB::load(rb, B, ldb, n0, N, 0, kb_max, tid);
        TA::store(ra, lds, tid, XA);
        TB::store(rb, lds + TA::SIZE, tid, 0);
    }
    __syncthreads();

    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            TA::load(ra, A8, lda, m0, M, (kt + 1) * BK, ka_max, tid);
            TB::load(rb, B, ldb, n0, N, (kt + 1) * BK, kb_max, tid);
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
            TA::store(ra, lds + (cur ^ 1) * BUF, tid, XA);
            TB::store(rb, lds + (cur ^ 1) * BUF + TA::SIZE, tid, 0);
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

template <int BM, int BN, int BK, int WM, int WN>
static hipError_t launch_icfg(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                              const int8_t *B, long ldb, const int32_t *col_off, const float *sa,
                              const float *sb, void *C, long ldc, hipStream_t stream) {
    const int nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (nblk == 0) return hipSuccess;
    dim3 grid(nblk), block(64 * WM * WN);
    switch (out_mode) {
        case 0:
            hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, BK, WM, WN, 0>), grid, block, 0, stream,
                               A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K);
            break;
        case 1:
            hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, BK, WM, WN, 1>), grid, block, 0, stream,
                               A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K);
            break;
        default:
            hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, BK, WM, WN, 2>), grid, block, 0, stream,
                               A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_igemm(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                        const int8_t *Bpk, long ldb, const int32_t *col_off, const float *sa,
                        const float *sb, void *C, long ldc, hipStream_t stream) {
    long big = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (big >= 256)
        return launch_icfg<128, 128, 128, 2, 2>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa,
                                                sb, C, ldc, stream);
    return launch_icfg<64, 64, 128, 2, 2>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C,
                                          ldc, stream);
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
