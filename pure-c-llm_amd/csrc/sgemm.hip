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

constexpr int SG_PAD_K = 4;   // floats of padding per K-contiguous LDS row
constexpr int SG_PAD_MN = 4;  // floats of padding per MN-contiguous LDS row

template <int NTHR, int ROWS, int BK, bool KC>
struct OperandTile {
    // LDS footprint of one buffer, in floats
    static constexpr int LD = KC ? (BK + SG_PAD_K) : (ROWS + SG_PAD_MN);
    static constexpr int SIZE = KC ? ROWS * LD : BK * LD;
    // 4-float vectors per tile and per thread
    static constexpr int VECS = ROWS * BK / 4;
    static constexpr int PER_THREAD = VECS / NTHR;
    static_assert(VECS % NTHR == 0, "tile must split evenly over the workgroup");

    // global -> registers. rows0: first row (m or n) of the tile; k0: first k.
    template <bool VEC>
    __device__ __forceinline__ static void load(v4f (&r)[PER_THREAD], const float *__restrict__ P,
                                                long ld, int rows0, int nrows, int k0, int K,
                                                int tid) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            int e = tid + i * NTHR;
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
                // VEC guarantees the 4-vector lies entirely inside or outside.
                // The load is unconditional from a clamped (valid) address and
                // the value is zeroed afterwards: with no branch around it the
                // compiler can count loads in flight across the prefetch ring.
                // KC: the row is scalar and k a 4-vector (K % 4 == 0, K >= 4);
                // MN: k is scalar and the row a 4-vector (nrows % 4 == 0).
                const bool ok = grow < nrows && gk < K;
                const int gr = KC ? min(grow, nrows - 1) : min(grow, nrows - 4);
                const int gc = KC ? min(gk, K - 4) : min(gk, K - 1);
                const float *src = KC ? P + (long)gr * ld + gc : P + (long)gc * ld + gr;
                v = *reinterpret_cast<const v4f *>(src);
                if (!ok) v = v4f{0.f, 0.f, 0.f, 0.f};
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
            int e = tid + i * NTHR;
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

// BM x BN output tile per workgroup of 256*KG threads: 2x2 waves share the
// tile spatially, and KG groups of those 4 waves split every BK-deep K tile
// (group g multiplies chunks [g*BK/(8*KG), (g+1)*BK/(8*KG))), so a small grid
// still puts KG waves on every SIMD. The groups' partial sums are added
// through LDS at the end (group g finishes the accumulator registers
// v in [16g/KG, 16(g+1)/KG) of every 32x32 block).
// PF: global tiles in flight in registers ahead of the LDS tile being
// multiplied (a ring of PF register slots, refilled PF tiles ahead).
// Split K: workgroup row blockIdx.y multiplies k in [y*kchunk, (y+1)*kchunk)
// and writes its partial product to C + y*M*ldc (kchunk = K: no split).
template <int BM, int BN, int BK, int KG, int PF, bool A_KC, bool B_KC, bool VEC>
__global__ __launch_bounds__(256 * KG) void sgemm_mfma_kernel(
    const float *__restrict__ A, long lda, const float *__restrict__ B, long ldb,
    const float *__restrict__ bias, float *__restrict__ C, long ldc, int M, int N, int K,
    int accumulate, int kchunk) {
    constexpr int NTHR = 256 * KG;
    using TA = OperandTile<NTHR, BM, BK, A_KC>;
    using TB = OperandTile<NTHR, BN, BK, B_KC>;
    constexpr int WTM = BM / 2, WTN = BN / 2;   // wave tile
    constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 MFMA blocks per wave
    constexpr int KCH = BK / 8;                  // 8-deep k chunks per tile
    constexpr int KCG = KCH / KG;                // chunks per K group
    static_assert(BK % 8 == 0 && KCH % KG == 0, "K tile must split over the K groups");
    static_assert(KG == 1 || KG == 2 || KG == 4, "one, two or four K groups");
    static_assert(PF >= 1, "at least one tile in flight");

    // two buffers, each [A tile | B tile]; the K groups' exchange reuses them
    constexpr int BUF = TA::SIZE + TB::SIZE;
    constexpr int VH = 16 / KG;  // accumulator registers finished per group
    // exchange inboxes: [owner group][KG - 1 senders][4 waves][TM][TN][VH][64 lanes]
    constexpr int XCH = KG > 1 ? KG * (KG - 1) * 256 * TM * TN * VH : 0;
    constexpr int LDS_FLOATS = 2 * BUF > XCH ? 2 * BUF : XCH;
    __shared__ __attribute__((aligned(16))) float lds[LDS_FLOATS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int kg = wave >> 2, wq = wave & 3;
    const int wm = wq >> 1, wn = wq & 1;
    const int r32 = lane & 31, g = lane >> 5;

    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int bm, bn;
    tile_coords(xcd_remap(blockIdx.x, nbm * nbn), nbm, nbn, 8, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;
    {
        const int kbeg = blockIdx.y * kchunk;
        K = K - kbeg < kchunk ? K - kbeg : kchunk;
        A += A_KC ? kbeg : (long)kbeg * lda;
        B += B_KC ? kbeg : (long)kbeg * ldb;
        C += (long)blockIdx.y * M * ldc;
    }

    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    v4f ra[PF][TA::PER_THREAD], rb[PF][TB::PER_THREAD];
    const int nk = (K + BK - 1) / BK;
    // tile t's registers live in slot t % PF; tiles past the end re-read the
    // last tile (never stored), so every iteration issues the same loads
    auto fetch = [&](auto S, int t) {
        const int k0 = (t < nk ? t : nk - 1) * BK;
        TA::template load<VEC>(ra[S.value], A, lda, m0, M, k0, K, tid);
        TB::template load<VEC>(rb[S.value], B, ldb, n0, N, k0, K, tid);
    };
    auto put = [&](auto S, int buf) {
        TA::store(ra[S.value], lds + buf * BUF, tid);
        TB::store(rb[S.value], lds + buf * BUF + TA::SIZE, tid);
    };

    if (nk > 0) {
        static_for<0, PF>([&](auto S) { fetch(S, S.value); });
        put(IC<0>{}, 0);
    }
    __syncthreads();

    for (int kt0 = 0; kt0 < nk; kt0 += PF) {
        static_for<0, PF>([&](auto S) {
            const int kt = kt0 + S.value;
            if (kt < nk) {
                // slot S held tile kt, already in LDS: refill it PF tiles ahead
                fetch(S, kt + PF);
                const float *la = lds + (kt & 1) * BUF;
                const float *lb = la + TA::SIZE;
                // all of this group's fragments of the tile are requested
                // before the first MFMA, so LDS latency overlaps the chain
                v4f fa[KCG][TM], fb[KCG][TN];
#pragma unroll
                for (int c = 0; c < KCG; c++) {
                    const int kc = kg * KCG + c;
#pragma unroll
                    for (int i = 0; i < TM; i++) fa[c][i] = TA::frag(la, wm * WTM + i * 32 + r32, kc, g);
#pragma unroll
                    for (int j = 0; j < TN; j++) fb[c][j] = TB::frag(lb, wn * WTN + j * 32 + r32, kc, g);
                }
#pragma unroll
                for (int c = 0; c < KCG; c++)
#pragma unroll
                    for (int s = 0; s < 4; s++)
#pragma unroll
                        for (int i = 0; i < TM; i++)
#pragma unroll
                            for (int j = 0; j < TN; j++)
                                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                    fa[c][i][s], fb[c][j][s], acc[i][j], 0, 0, 0);
                if (kt + 1 < nk) put(IC<(S.value + 1) % PF>{}, (kt + 1) & 1);
                __syncthreads();
            }
        });
    }

    // K groups: group g finishes accumulator registers v in [g*VH, (g+1)*VH).
    // Every group posts the registers it does not finish to their owner's
    // inbox (lane-contiguous, conflict-free), then adds its senders' shares to
    // its own registers in sender order. Register indices stay compile-time
    // (a runtime index would move the accumulators out of registers). The last
    // loop barrier has retired every tile read.
    if constexpr (KG > 1) {
        auto slot = [&](int owner, int sender, int i, int j, int u) {
            const int s = sender < owner ? sender : sender - 1;
            return (((((owner * (KG - 1) + s) * 4 + wq) * TM + i) * TN + j) * VH + u) * 64 + lane;
        };
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
                static_for<0, 16>([&](auto V) {
                    constexpr int v = V.value, owner = v / VH;
                    if (owner != kg) lds[slot(owner, kg, i, j, v % VH)] = acc[i][j][v];
                });
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
                static_for<0, 16>([&](auto V) {
                    constexpr int v = V.value, owner = v / VH;
                    if (owner == kg) {
#pragma unroll
                        for (int sdr = 0; sdr < KG; sdr++)
                            if (sdr != kg) acc[i][j][v] += lds[slot(owner, sdr, i, j, v % VH)];
                    }
                });
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
            const int rb = m0 + wm * WTM + i * 32 + g * 4;
            // old C values (accumulate) are all requested before any is used,
            // from clamped rows; rows past M are never stored
            float old[16];
            if (accumulate) {
                static_for<0, 16>([&](auto V) {
                    constexpr int v = V.value;
                    if (KG == 1 || v / VH == kg)
                        old[v] = C[(long)min(rb + (v >> 2) * 8 + (v & 3), M - 1) * ldc + col];
                });
            }
            static_for<0, 16>([&](auto V) {
                constexpr int v = V.value;
                if (KG == 1 || v / VH == kg) {
                    const int row = rb + (v >> 2) * 8 + (v & 3);
                    if (row < M) {
                        float out = acc[i][j][v] + bv;
                        if (accumulate) out = old[v] + out;
                        C[(long)row * ldc + col] = out;
                    }
                }
            });
        }
    }
}

// Split-K epilogue: C = (accumulate ? C : 0) + (P_0 + P_1 + ... + bias), the
// partial products added in split order (deterministic).
__global__ void sgemm_splitk_reduce_kernel(const float *__restrict__ P, int splits, int M, int N,
                                           const float *__restrict__ bias, float *__restrict__ C,
                                           long ldc, int accumulate) {
    const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    const long MN = (long)M * N;
    if (i >= MN) return;
    const int m = (int)(i / N), n = (int)(i % N);
    float s = P[i];
    for (int z = 1; z < splits; z++) s += P[z * MN + i];
    float out = s + (bias ? bias[n] : 0.f);
    float *c = C + (long)m * ldc + n;
    if (accumulate) out = *c + out;
    *c = out;
}

template <int BM, int BN, int BK, int KG, int PF, bool A_KC, bool B_KC>
static hipError_t launch_cfg(bool vec, int M, int N, int K, int splits, int kchunk,
                             const float *A, long lda, const float *B, long ldb, const float *bias,
                             int accumulate, float *C, long ldc, hipStream_t stream) {
    const int nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (nblk == 0) return hipSuccess;
    dim3 grid(nblk, splits), block(256 * KG);
    if (vec)
        hipLaunchKernelGGL((sgemm_mfma_kernel<BM, BN, BK, KG, PF, A_KC, B_KC, true>), grid, block, 0,
                           stream, A, lda, B, ldb, bias, C, ldc, M, N, K, accumulate, kchunk);
    else
        hipLaunchKernelGGL((sgemm_mfma_kernel<BM, BN, BK, KG, PF, A_KC, B_KC, false>), grid, block,
                           0, stream, A, lda, B, ldb, bias, C, ldc, M, N, K, accumulate, kchunk);
    return hipGetLastError();
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Tile configurations (launch_cfg parameters), chosen by plan_sgemm.
enum SgemmCfg {
    SG_128_BK16 = 0,     // 128x128, BK 16, 4 waves: up to 4 workgroups per CU
    SG_128_BK32 = 1,     // 128x128, BK 32, 4 waves: 2 workgroups per CU
    SG_128_KG2 = 2,      // 128x128, BK 32, 8 waves in two K groups, 2 tiles in flight
    SG_64_KG2 = 3,       // 64x64, BK 64, 8 waves in two K groups, 2 tiles in flight
};

SgemmPlan plan_sgemm(int M, int N, int K) {
    SgemmPlan p{SG_64_KG2, 1, K > 0 ? K : 1, 0};
    const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    const long t64 = (long)((M + 63) / 64) * ((N + 63) / 64);
    if (t128 >= 512) {
        // whole rounds of 2 per CU take the deeper tile, otherwise 4 per CU
        // keep more of the grid resident at once
        p.cfg = t128 % 512 == 0 ? SG_128_BK32 : SG_128_BK16;
    } else if (t128 >= 256) {
        p.cfg = SG_128_KG2;
    } else if (t64 < 256 && K >= 128) {
        // too few tiles for 256 CUs: split K (chunks of whole 64-deep tiles)
        int splits = (int)(256 / (t64 > 0 ? t64 : 1));
        if (splits > K / 64) splits = K / 64;
        if (splits > 16) splits = 16;
        if (splits > 1) {
            const int kchunk = ((K + splits - 1) / splits + 63) / 64 * 64;
            p.splits = (K + kchunk - 1) / kchunk;
            p.kchunk = kchunk;
            if (p.splits > 1) p.part_bytes = (size_t)p.splits * M * N * sizeof(float);
            else p.kchunk = K;
        }
    }
    return p;
}

template <bool A_KC, bool B_KC>
static hipError_t dispatch_layout(const SgemmPlan &p, int M, int N, int K, const float *A,
                                  long lda, const float *B, long ldb, const float *bias,
                                  int accumulate, float *C, long ldc, const Workspace &ws,
                                  hipStream_t stream) {
    // 16-byte vector loads need the contiguous extent and leading dimension to
    // be multiples of 4 floats and 16-byte aligned bases (split-K chunks are
    // multiples of 64, so every chunk keeps that alignment).
    bool vec = aligned16(A) && aligned16(B) && lda % 4 == 0 && ldb % 4 == 0 &&
               (A_KC ? K % 4 == 0 : M % 4 == 0) && (B_KC ? K % 4 == 0 : N % 4 == 0);
    const bool split = p.splits > 1;
    if (split && (ws.buf == nullptr || ws.bytes_cap < p.part_bytes)) return hipErrorInvalidValue;
    float *out = split ? static_cast<float *>(ws.buf) : C;
    const long ldo = split ? N : ldc;
    const float *b = split ? nullptr : bias;
    const int acc = split ? 0 : accumulate;
    hipError_t e;
    switch (p.cfg) {
    case SG_128_BK16:
        e = launch_cfg<128, 128, 16, 1, 1, A_KC, B_KC>(vec, M, N, K, p.splits, p.kchunk, A, lda, B,
                                                       ldb, b, acc, out, ldo, stream);
        break;
    case SG_128_BK32:
        e = launch_cfg<128, 128, 32, 1, 1, A_KC, B_KC>(vec, M, N, K, p.splits, p.kchunk, A, lda, B,
                                                       ldb, b, acc, out, ldo, stream);
        break;
    case SG_128_KG2:
        e = launch_cfg<128, 128, 32, 2, 2, A_KC, B_KC>(vec, M, N, K, p.splits, p.kchunk, A, lda, B,
                                                       ldb, b, acc, out, ldo, stream);
        break;
    default:
        e = launch_cfg<64, 64, 64, 2, 2, A_KC, B_KC>(vec, M, N, K, p.splits, p.kchunk, A, lda, B,
                                                     ldb, b, acc, out, ldo, stream);
        break;
    }
    if (e != hipSuccess || !split) return e;
    const long MN = (long)M * N;
    hipLaunchKernelGGL(sgemm_splitk_reduce_kernel, dim3((unsigned)((MN + 255) / 256)), dim3(256), 0,
                       stream, static_cast<const float *>(ws.buf), p.splits, M, N, bias, C, ldc,
                       accumulate);
    return hipGetLastError();
}

hipError_t launch_sgemm(const SgemmPlan &p, bool a_kcontig, bool b_kcontig, int M, int N, int K,
                        const float *A, long lda, const float *B, long ldb, const float *bias,
                        int accumulate, float *C, long ldc, const Workspace &ws,
                        hipStream_t stream) {
    if (a_kcontig && !b_kcontig)
        return dispatch_layout<true, false>(p, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, ws,
                                            stream);
    if (a_kcontig && b_kcontig)
        return dispatch_layout<true, true>(p, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, ws,
                                           stream);
    if (!a_kcontig && !b_kcontig)
        return dispatch_layout<false, false>(p, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc,
                                             ws, stream);
    return dispatch_layout<false, true>(p, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, ws,
                                        stream);
}

}  // namespace pcl
