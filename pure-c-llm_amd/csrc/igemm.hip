// igemm.hip -- u8 x s8 -> int32 GEMM on the CDNA4 int8 matrix cores
// (v_mfma_i32_32x32x32_i8), with the dequantising epilogue.
//
// Reference semantics (gemm_bench.c:212-285): activations are u8 with a +128
// offset, weights s8; vpdpbusd forms acc = sum Au*Bq and the kernel subtracts
// corr = 128*colsum, i.e. v = sum (Au-128)*Bq (gemm_bench.c:216-217, 274).
// The i8 MFMA is signed x signed, so A is re-centred with Au ^ 0x80, which is
// exactly Au-128 as an s8 byte: the MFMA then produces v directly, bit-exact,
// with no column-sum pass. An optional per-column int32 offset reproduces a
// caller-supplied `corr` (off = 128*colsum - corr). Dequant
// (gemm_bench.c:272-275, dq precomputed at :378) is fp32 RNE in the same
// order: C = float(v) * dq with dq = sb[n] or sa[m]*sb[n].
//
// Layouts: A is M x K u8 row-major (K-contiguous). B is pre-packed N x Kp s8
// (K-contiguous per output column, zero from K to Kp = roundup(K, 256); the
// reference packs its weights offline too, gemm_bench.c:218-220).
//
// Data movement. Tiles of BM (BN) rows x 128 bytes of K go from HBM straight
// into LDS with global_load_lds_dwordx4: each wave instruction moves 64 x 16
// bytes into 1 KB of consecutive LDS, no VGPRs involved, so STAGES tiles can
// be in flight at once. A K tile is consumed from LDS by 16-byte fragment
// reads (ds_read_b128) feeding the MFMA; the A fragment is re-centred by XOR
// in registers.
//
// LDS layout: row r of a tile is 128 bytes = 8 chunks of 16 bytes; logical
// chunk c lives at physical chunk c ^ ((r >> 1) & 7). The LDS serves a
// ds_read_b128 16 lanes at a time out of 64 four-byte banks (16 chunk slots
// per 256 bytes), and 16 consecutive lanes read 16 consecutive rows at the
// same logical chunk: rows 2q and 2q+1 differ in the 256-byte half, pairs
// differ in the swizzled chunk, so the 16 reads hit 16 distinct slots. A DMA
// instruction fills 8 whole rows, lanes choosing their global chunk so the
// physical layout comes out swizzled.
//
// Tails are handled without branches or masks: rows past M (N) are clamped to
// the last row and only feed outputs that are never stored; an A chunk past K
// is clamped to the last in-bounds chunk, whose bytes meet the zero padding of
// the packed weights (every B chunk read lies below nk*128 <= Kp).
//
// Synchronisation: one s_barrier per K tile. Before it, each wave waits with
// s_waitcnt vmcnt for its own DMA loads of the tile about to be read (leaving
// the STAGES-2 younger tiles in flight); after it, the stage freed by the
// previous tile is refilled. No fence is used: a release fence would wait for
// every outstanding load and drain the pipeline.
//
// K order: the 32x32x32 MFMA takes 16 bytes per lane; lane group g = lane/32
// supplies logical chunk 2kc+g of the tile for A and for B alike, so the
// integer sum is the same whatever order the hardware reduces it in.
#include "internal.h"

namespace pcl {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int IG_BK = 128;  // bytes of K per tile

// s_waitcnt immediate for "vmcnt <= n", leaving expcnt and lgkmcnt unchecked.
constexpr int waitcnt_vm(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (15 << 8); }
constexpr int WAITCNT_LGKM0 = (15) | (3 << 14) | (7 << 4);  // lgkmcnt(0) only

__device__ __forceinline__ int swz_off(int r, int c) { return r * IG_BK + ((c ^ ((r >> 1) & 7)) << 4); }

// DMA of one operand tile (ROWS x 128 bytes) by NW waves: instruction j of
// wave w fills LDS rows 8*(j*NW + w) .. +7.
template <int ROWS, int NW>
struct DmaTile {
    static constexpr int SIZE = ROWS * IG_BK;
    static constexpr int INSTS = ROWS / (8 * NW);  // per wave
    static_assert(ROWS % (8 * NW) == 0, "tile rows must split over the waves");

    __device__ __forceinline__ static void issue(int8_t *lds, const int8_t *__restrict__ P, long ld,
                                                 int rows0, int nrows, int k0, int kmax, int wave,
                                                 int lane) {
#pragma unroll
        for (int j = 0; j < INSTS; j++) {
            const int rb = (j * NW + wave) * 8;   // first row of this instruction
            const int r = rb + (lane >> 3);
            const int c = (lane & 7) ^ ((r >> 1) & 7);
            const int grow = min(rows0 + r, nrows - 1);
            const int gk = min(k0 + c * 16, kmax);
            __builtin_amdgcn_global_load_lds((const void *)(P + (long)grow * ld + gk),
                                             (lds_void_t *)(lds + rb * IG_BK), 16, 0, 0);
        }
    }
};

template <int BM, int BN, int WM, int WN, int STAGES, int OUT>
__global__ __launch_bounds__(64 * WM * WN) void igemm_mfma_kernel(
    const uint8_t *__restrict__ A, long lda, const int8_t *__restrict__ B, long ldb,
    const int32_t *__restrict__ col_off, const float *__restrict__ sa,
    const float *__restrict__ sb, void *__restrict__ Cv, long ldc, int M, int N, int K) {
    constexpr int NW = WM * WN;
    using TA = DmaTile<BM, NW>;
    using TB = DmaTile<BN, NW>;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int KC = IG_BK / 32;                      // MFMA k-chunks per tile
    constexpr int STAGE = TA::SIZE + TB::SIZE;
    constexpr int LOADS = TA::INSTS + TB::INSTS;        // DMA instructions per tile per wave
    static_assert(TM >= 1 && TN >= 1 && STAGES >= 2, "bad tile configuration");
    static_assert((STAGES - 2) * LOADS <= 63, "vmcnt range");

    __shared__ __attribute__((aligned(1024))) int8_t lds[STAGES * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int r32 = lane & 31, g = lane >> 5;

    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int bm, bn;
    tile_coords(xcd_remap(blockIdx.x, nbm * nbn), nbm, nbn, 8, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;

    const int8_t *A8 = reinterpret_cast<const int8_t *>(A);
    const int nk = (K + IG_BK - 1) / IG_BK;
    const int ka_max = K - 16;           // K % 16 == 0 and K > 0 whenever nk > 0
    const int kb_max = nk * IG_BK - 16;  // inside the zero-padded weight row

    auto issue = [&](int t) {
        int8_t *st = lds + (t % STAGES) * STAGE;
        TA::issue(st, A8, lda, m0, M, t * IG_BK, ka_max, wave, lane);
        TB::issue(st + TA::SIZE, B, ldb, n0, N, t * IG_BK, kb_max, wave, lane);
    };

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0;

    // tile row read by this lane for each A / B fragment
    int rowa[TM], rowb[TN];
#pragma unroll
    for (int i = 0; i < TM; i++) rowa[i] = wm * WTM + i * 32 + r32;
#pragma unroll
    for (int j = 0; j < TN; j++) rowb[j] = wn * WTN + j * 32 + r32;

#pragma unroll
    for (int t = 0; t < STAGES - 1; t++)
        if (t < nk) issue(t);

    for (int kt = 0; kt < nk; kt++) {
        if (kt + STAGES - 2 < nk) __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 2) * LOADS));
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __builtin_amdgcn_s_barrier();
        if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1);

        const int8_t *la = lds + (kt % STAGES) * STAGE;
        const int8_t *lb = la + TA::SIZE;
        // Fragments are double-buffered by k-chunk, and the re-centred A
        // fragments get registers of their own: no register that an issued
        // MFMA still reads is rewritten by the next chunk's reads or XORs.
        v4i fa[2][TM], fb[2][TN], ax[2][TM];
#pragma unroll
        for (int i = 0; i < TM; i++) fa[0][i] = *reinterpret_cast<const v4i *>(la + swz_off(rowa[i], g));
#pragma unroll
        for (int j = 0; j < TN; j++) fb[0][j] = *reinterpret_cast<const v4i *>(lb + swz_off(rowb[j], g));
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            const int cu = kc & 1;
#pragma unroll
            for (int i = 0; i < TM; i++) ax[cu][i] = fa[cu][i] ^ (int)0x80808080u;
            if (kc + 1 < KC) {
#pragma unroll
                for (int i = 0; i < TM; i++)
                    fa[cu ^ 1][i] = *reinterpret_cast<const v4i *>(la + swz_off(rowa[i], 2 * kc + 2 + g));
#pragma unroll
                for (int j = 0; j < TN; j++)
                    fb[cu ^ 1][j] = *reinterpret_cast<const v4i *>(lb + swz_off(rowb[j], 2 * kc + 2 + g));
            }
            // keep the next chunk's reads ahead of this chunk's MFMAs (the
            // scheduler would otherwise sink them and serialise read -> MFMA)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int i = 0; i < TM; i++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ax[cu][i], fb[cu][j], acc[i][j], 0, 0, 0);
        }
        // every fragment read of this stage completes before the next
        // barrier, after which the stage may be refilled
        __builtin_amdgcn_s_waitcnt(WAITCNT_LGKM0);
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

template <int BM, int BN, int WM, int WN, int STAGES>
static hipError_t launch_icfg(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                              const int8_t *B, long ldb, const int32_t *col_off, const float *sa,
                              const float *sb, void *C, long ldc, hipStream_t stream) {
    const int nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (nblk == 0) return hipSuccess;
    dim3 grid(nblk), block(64 * WM * WN);
    switch (out_mode) {
        case 0:
            hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, WM, WN, STAGES, 0>), grid, block, 0,
                               stream, A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K);
            break;
        case 1:
            hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, WM, WN, STAGES, 1>), grid, block, 0,
                               stream, A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K);
            break;
        default:
            hipLaunchKernelGGL((igemm_mfma_kernel<BM, BN, WM, WN, STAGES, 2>), grid, block, 0,
                               stream, A, lda, B, ldb, col_off, sa, sb, C, ldc, M, N, K);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_igemm(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                        const int8_t *Bpk, long ldb, const int32_t *col_off, const float *sa,
                        const float *sb, void *C, long ldc, hipStream_t stream) {
    long big = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (big >= 256)
        return launch_icfg<128, 128, 2, 2, 4>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb,
                                              C, ldc, stream);
    return launch_icfg<64, 64, 2, 2, 4>(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C,
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
