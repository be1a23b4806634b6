// sgemm.hip -- FP32 GEMM on the CDNA4 f32 matrix cores (v_mfma_f32_32x32x2f32,
// and v_mfma_f32_16x16x4f32 for grids of two or more workgroups per CU).
//
// Each kernel template covers every row-major layout the reference uses:
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

// ---------------------------------------------------------------------------
// Epilogues (train.c:314-333 and gpu_kernels.cu:228-243 tanh-GELU, the
// residual adds of train.c:522/527): applied to v = acc + bias.
constexpr float GELU_C = 0.7978845608028654f;  // sqrt(2/pi)
__device__ __forceinline__ float gelu_f(float x) {
    return 0.5f * x * (1.0f + tanhf(GELU_C * (x + 0.044715f * x * x * x)));
}
__device__ __forceinline__ float gelu_grad(float x) {
    const float t = tanhf(GELU_C * (x + 0.044715f * x * x * x));
    const float dudx = GELU_C * (1.0f + 3.0f * 0.044715f * x * x);
    return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * dudx;
}
// EPI_GELU: aux_out (if set) <- v, C <- gelu(v); EPI_RESID: C <- aux_in + v;
// EPI_GELU_BWD: C <- v * gelu'(aux_in)
template <int EPI>
__device__ __forceinline__ float apply_epi(float v, const float *aux_in, float *aux_out, long ai) {
    if constexpr (EPI == EPI_GELU) {
        if (aux_out) aux_out[ai] = v;
        return gelu_f(v);
    } else if constexpr (EPI == EPI_RESID) {
        return aux_in[ai] + v;
    } else if constexpr (EPI == EPI_GELU_BWD) {
        return v * gelu_grad(aux_in[ai]);
    }
    return v;
}

// The same epilogue as a separate pass over an M x N product already in C
// (operands the fused kernels do not take: unaligned, split K, other layouts).
// Grid (ceil(N / 256), M).
__global__ void sgemm_epilogue_kernel(int epi, int M, int N, float *__restrict__ C, long ldc,
                                      const float *__restrict__ aux_in,
                                      float *__restrict__ aux_out, long ld_aux) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    const long m = blockIdx.y;
    if (n >= N) return;
    float *c = C + m * ldc + n;
    const long ai = m * ld_aux + n;
    if (epi == EPI_GELU) *c = apply_epi<EPI_GELU>(*c, aux_in, aux_out, ai);
    else if (epi == EPI_RESID) *c = apply_epi<EPI_RESID>(*c, aux_in, aux_out, ai);
    else if (epi == EPI_GELU_BWD) *c = apply_epi<EPI_GELU_BWD>(*c, aux_in, aux_out, ai);
}

// Flat elementwise kernels of the reference GPU API (gpu_kernels.cu:228-251).
__global__ void gelu_fwd_kernel(float *__restrict__ Y, const float *__restrict__ X, long n) {
    const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i < n) Y[i] = gelu_f(X[i]);
}
__global__ void gelu_bwd_kernel(float *__restrict__ dX, const float *__restrict__ dY,
                                const float *__restrict__ X, long n) {
    const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i < n) dX[i] = dY[i] * gelu_grad(X[i]);
}
__global__ void vec_add_kernel(float *__restrict__ C, const float *__restrict__ A,
                               const float *__restrict__ B, long n) {
    const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i < n) C[i] = A[i] + B[i];
}

hipError_t launch_elementwise(int op, long n, float *out, const float *a, const float *b,
                              hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    if (op == 0) hipLaunchKernelGGL(gelu_fwd_kernel, grid, block, 0, stream, out, a, n);
    else if (op == 1) hipLaunchKernelGGL(gelu_bwd_kernel, grid, block, 0, stream, out, a, b, n);
    else hipLaunchKernelGGL(vec_add_kernel, grid, block, 0, stream, out, a, b, n);
    return hipGetLastError();
}

// Copy rows x cols floats from src (leading dimension lds, any 4-byte
// alignment) into dst (ldd a multiple of 4, 16-byte aligned): each thread
// gathers 4 consecutive floats with 4-byte loads (consecutive lanes read
// consecutive 16 bytes, so the reads stay coalesced) and writes them as one
// 16-byte store; a row's last partial vector is written element by element.
__global__ __launch_bounds__(256) void copy_rows_kernel(float *__restrict__ dst, long ldd,
                                                        const float *__restrict__ src, long lds,
                                                        int rows, int cols) {
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    const int nv = (cols + 3) / 4;
    for (int r = blockIdx.y; r < rows; r += gridDim.y) {
        const float *sr = src + (long)r * lds;
        float *dr = dst + (long)r * ldd;
        for (int v = blockIdx.x * 256 + threadIdx.x; v < nv; v += gridDim.x * 256) {
            const int c = 4 * v;
            if (c + 4 <= cols) {
                const v4f_t x = {__builtin_nontemporal_load(sr + c), __builtin_nontemporal_load(sr + c + 1),
                                 __builtin_nontemporal_load(sr + c + 2), __builtin_nontemporal_load(sr + c + 3)};
                *reinterpret_cast<v4f_t *>(dr + c) = x;
            } else {
                for (int e = c; e < cols; e++) dr[e] = sr[e];
            }
        }
    }
}

hipError_t launch_copy_rows(float *dst, long ldd, const float *src, long lds, int rows, int cols,
                            hipStream_t stream) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const int nv = (cols + 3) / 4;
    const dim3 grid((unsigned)((nv + 1023) / 1024), (unsigned)(rows < 4096 ? rows : 4096)), block(256);
    hipLaunchKernelGGL(copy_rows_kernel, grid, block, 0, stream, dst, ldd, src, lds, rows, cols);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// LDS-DMA pipeline. Operand tiles of SD_BK = 32 floats of K go from global
// memory straight into a STAGES-deep LDS ring with global_load_lds_dwordx4
// (no VGPR staging, no ds_write), issued by every wave; the wave's waits are
// explicit (s_waitcnt), as are its fragment reads (inline ds_read), so the
// compiler's loop-carried wait insertion cannot serialise the ring. Layouts
// in LDS, unpadded and swizzled so fragment reads are conflict-free:
//  * K-contiguous operand: ROWS rows of 128 bytes; logical 16-byte chunk c of
//    row r sits at chunk c ^ ((r >> 1) & 7);
//  * MN-contiguous operand: 32 k-rows of ROWS floats; logical chunk c of
//    k-row k sits at chunk c ^ (((k >> 2) & 1) << 3).
// A DMA instruction writes 1 KB of consecutive LDS; each lane picks the
// global chunk that lands in its swizzled slot. Per K tile: wait for this
// wave's fragment reads (issued during the previous tile's MFMAs) and for its
// DMA of the next tile, one barrier, refill the stage just read, read the
// next tile's fragments, then this tile's MFMAs. Requires K % 32 == 0 and the
// 16-byte vector conditions of the register-staged kernel.
constexpr int SD_BK = 32;

template <int OFF>
__device__ __forceinline__ void sd_read128(v4f &r, unsigned addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds_read offset field");
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
}
template <int OFF>
__device__ __forceinline__ void sd_read32(float &r, unsigned addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds_read offset field");
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
}
__device__ __forceinline__ void sd_fence(v4f &r) { asm volatile("" : "+v"(r)); }
__device__ __forceinline__ void sd_fence(float &r) { asm volatile("" : "+v"(r)); }
constexpr int sd_waitcnt_vm(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (15 << 8); }

// One operand's part of a ring stage: SUB consecutive K tiles of ROWS (M or
// N) x SD_BK (K) floats, tile s at byte SUBB * s of the stage.
template <int ROWS, bool KC, int NW, int SUB, int SUBB>
struct DmaTile {
    static constexpr int BYTES = ROWS * SD_BK * 4;  // ROWS * 128, one K tile
    static constexpr int INST = BYTES / 1024;        // DMA instructions per K tile
    static constexpr int PER_WAVE = SUB * INST / NW;
    static_assert((SUB * INST) % NW == 0, "DMA instructions must split over the waves");
    static constexpr int CHR = KC ? 8 : ROWS / 4;    // 16-byte chunks per LDS row
    static_assert(KC || CHR >= 16, "MN swizzle needs 16 chunks per k-row");

    // per-lane source offset (floats, at k = 0) and LDS byte offset of this
    // wave's instruction q; rows0: the tile's first row (m or n)
    __device__ __forceinline__ static void setup(long (&voff)[PER_WAVE], int (&ldso)[PER_WAVE],
                                                 int wave, int lane, int rows0, int nrows,
                                                 long ld) {
#pragma unroll
        for (int q = 0; q < PER_WAVE; q++) {
            const int sub = (q * NW + wave) / INST, inst = (q * NW + wave) % INST;
            if (KC) {
                const int r = inst * 8 + lane / 8;
                const int gc = (lane % 8) ^ ((r >> 1) & 7);
                voff[q] = (long)min(rows0 + r, nrows - 1) * ld + sub * SD_BK + gc * 4;
            } else {
                const int rpi = 64 / CHR;  // k-rows per instruction
                const int k = inst * rpi + lane / CHR;
                const int gc = (lane % CHR) ^ (((k >> 2) & 1) << 3);
                voff[q] = (long)(sub * SD_BK + k) * ld + min(rows0 + gc * 4, nrows - 4);
            }
            ldso[q] = sub * SUBB + inst * 1024;
        }
    }
    // issue this wave's DMA of the SUB tiles from k0 into the stage at lds_stage
    __device__ __forceinline__ static void dma(const float *P, long ld, int k0, const long (&voff)[PER_WAVE],
                                               const int (&ldso)[PER_WAVE], int8_t *lds_stage) {
        const float *base = KC ? P + k0 : P + (long)k0 * ld;
#pragma unroll
        for (int q = 0; q < PER_WAVE; q++)
            __builtin_amdgcn_global_load_lds((const void *)(base + voff[q]),
                                             (__attribute__((address_space(3))) void *)(lds_stage + ldso[q]),
                                             16, 0, 0);
    }
};

template <int BM, int BN, int KG, int STAGES, int SUB, bool A_KC, bool B_KC, int EPI = EPI_NONE>
__global__ __launch_bounds__(256 * KG) void sgemm_dma_kernel(
    const float *__restrict__ A, long lda, const float *__restrict__ B, long ldb,
    const float *__restrict__ bias, float *__restrict__ C, long ldc, int M, int N, int K,
    int accumulate, int kchunk, const float *__restrict__ aux_in, float *__restrict__ aux_out,
    long ld_aux) {
    constexpr int NW = 4 * KG;
    constexpr int SUBB = (BM + BN) * SD_BK * 4;  // one K tile of both operands
    using TA = DmaTile<BM, A_KC, NW, SUB, SUBB>;
    using TB = DmaTile<BN, B_KC, NW, SUB, SUBB>;
    constexpr int WTM = BM / 2, WTN = BN / 2, TM = WTM / 32, TN = WTN / 32;
    constexpr int KCH = SD_BK / 8;   // 8-deep k chunks per tile
    constexpr int KCG = KCH / KG;    // chunks per K group
    constexpr int STAGE = SUB * SUBB;
    constexpr int VH = 16 / KG;
    constexpr int XCH = KG > 1 ? KG * (KG - 1) * 256 * TM * TN * VH * 4 : 0;
    constexpr int LDS_BYTES = STAGES * STAGE > XCH ? STAGES * STAGE : XCH;
    constexpr int LOADS = TA::PER_WAVE + TB::PER_WAVE;
    static_assert(KCH % KG == 0 && STAGES >= 2, "tile configuration");
    static_assert((STAGES - 1) * LOADS <= 63, "vmcnt range");
    static_assert(STAGE <= 65536, "ds_read offset field");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget of a CU");
    __shared__ __attribute__((aligned(1024))) int8_t lds[LDS_BYTES];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = wave >> 2, wq = wave & 3, wm = wq >> 1, wn = wq & 1;
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
    const int nk = K / (SD_BK * SUB);  // ring stages (SUB K tiles each)

    long voa[TA::PER_WAVE], vob[TB::PER_WAVE];
    int lda_o[TA::PER_WAVE], ldb_o[TB::PER_WAVE];
    TA::setup(voa, lda_o, wave, lane, m0, M, lda);
    TB::setup(vob, ldb_o, wave, lane, n0, N, ldb);
    auto dma = [&](int t) {
        int8_t *st = lds + (t % STAGES) * STAGE;
        TA::dma(A, lda, t * SUB * SD_BK, voa, lda_o, st);
        TB::dma(B, ldb, t * SUB * SD_BK, vob, ldb_o, st + TA::BYTES);
    };

    // Fragment addresses (bytes within a stage). K-contiguous operand: row
    // rb + 32i + r32 at logical chunk 2kc + g (a 16-byte read gives the four
    // k of this lane's MFMA steps). MN-contiguous: element (k, n) with
    // k = 8kc + 4g + s, n = cb + 32j + r32 (four 4-byte reads).
    const unsigned lds0 = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)lds;
    unsigned a_addr[A_KC ? KCG : TM], b_addr[B_KC ? KCG : TN];
    if constexpr (A_KC) {
#pragma unroll
        for (int c = 0; c < KCG; c++)
            a_addr[c] = (wm * WTM + r32) * 128 + (((2 * (kg * KCG + c) + g) ^ ((r32 >> 1) & 7)) << 4);
    } else {
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int m = wm * WTM + i * 32 + r32;
            a_addr[i] = (kg * KCG * 8 + 4 * g) * BM * 4 + (((m >> 2) ^ (g << 3)) << 4) + (m & 3) * 4;
        }
    }
    if constexpr (B_KC) {
#pragma unroll
        for (int c = 0; c < KCG; c++)
            b_addr[c] = TA::BYTES + (wn * WTN + r32) * 128 +
                        (((2 * (kg * KCG + c) + g) ^ ((r32 >> 1) & 7)) << 4);
    } else {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = wn * WTN + j * 32 + r32;
            b_addr[j] = TA::BYTES + (kg * KCG * 8 + 4 * g) * BN * 4 + (((n >> 2) ^ (g << 3)) << 4) + (n & 3) * 4;
        }
    }
    // Fragments of one stage, two slots (current and next stage). A
    // K-contiguous operand fills one 16-byte register quad per block; an
    // MN-contiguous one four separate floats (each its own read, so no
    // register copy can run ahead of the wait).
    v4f fak[2][SUB][KCG][A_KC ? TM : 1], fbk[2][SUB][KCG][B_KC ? TN : 1];
    float fam[2][SUB][KCG][A_KC ? 1 : TM][4], fbm[2][SUB][KCG][B_KC ? 1 : TN][4];
    auto read_tile = [&](auto SL, int t) {
        constexpr int sl = decltype(SL)::value;
        const unsigned st = lds0 + (t % STAGES) * STAGE;
        static_for<0, SUB>([&](auto U) {
        constexpr int u = decltype(U)::value, uo = u * SUBB;
        static_for<0, KCG>([&](auto Cc) {
            constexpr int c = decltype(Cc)::value;
            static_for<0, TM>([&](auto I) {
                constexpr int i = decltype(I)::value;
                if constexpr (A_KC) {
                    sd_read128<uo + i * 32 * 128>(fak[sl][u][c][i], st + a_addr[c]);
                } else {
                    sd_read32<uo + (c * 8 + 0) * BM * 4>(fam[sl][u][c][i][0], st + a_addr[i]);
                    sd_read32<uo + (c * 8 + 1) * BM * 4>(fam[sl][u][c][i][1], st + a_addr[i]);
                    sd_read32<uo + (c * 8 + 2) * BM * 4>(fam[sl][u][c][i][2], st + a_addr[i]);
                    sd_read32<uo + (c * 8 + 3) * BM * 4>(fam[sl][u][c][i][3], st + a_addr[i]);
                }
            });
            static_for<0, TN>([&](auto J) {
                constexpr int j = decltype(J)::value;
                if constexpr (B_KC) {
                    sd_read128<uo + j * 32 * 128>(fbk[sl][u][c][j], st + b_addr[c]);
                } else {
                    sd_read32<uo + (c * 8 + 0) * BN * 4>(fbm[sl][u][c][j][0], st + b_addr[j]);
                    sd_read32<uo + (c * 8 + 1) * BN * 4>(fbm[sl][u][c][j][1], st + b_addr[j]);
                    sd_read32<uo + (c * 8 + 2) * BN * 4>(fbm[sl][u][c][j][2], st + b_addr[j]);
                    sd_read32<uo + (c * 8 + 3) * BN * 4>(fbm[sl][u][c][j][3], st + b_addr[j]);
                }
            });
        });
        });
    };
    // after the wait: order every later use of slot sl after it
    auto fence_slot = [&](auto SL) {
        constexpr int sl = decltype(SL)::value;
#pragma unroll
        for (int u = 0; u < SUB; u++)
#pragma unroll
        for (int c = 0; c < KCG; c++) {
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if constexpr (A_KC) {
                    sd_fence(fak[sl][u][c][i]);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; q++) sd_fence(fam[sl][u][c][i][q]);
                }
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if constexpr (B_KC) {
                    sd_fence(fbk[sl][u][c][j]);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; q++) sd_fence(fbm[sl][u][c][j][q]);
                }
            }
        }
    };

    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    // scalar arguments of the epilogue are materialised before the loop (a
    // scalar load in flight would also count in lgkmcnt)
    float *Cm = C;
    long ldcm = ldc;
    asm volatile("" : "+s"(Cm), "+s"(ldcm));

    if (nk > 0) {
#pragma unroll
        for (int t = 0; t < STAGES; t++)
            if (t < nk) dma(t);
        if (nk >= STAGES) __builtin_amdgcn_s_waitcnt(sd_waitcnt_vm((STAGES - 1) * LOADS));
        else __builtin_amdgcn_s_waitcnt(sd_waitcnt_vm(0));
        __builtin_amdgcn_s_barrier();
        read_tile(IC<0>{}, 0);
    }
    auto step = [&](auto SL, int kt) {
        constexpr int sl = decltype(SL)::value;
        // this wave's reads of tile kt have landed; its DMA of tile kt+1 too
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        fence_slot(SL);
        if (kt + STAGES - 1 < nk) __builtin_amdgcn_s_waitcnt(sd_waitcnt_vm((STAGES - 2) * LOADS));
        else __builtin_amdgcn_s_waitcnt(sd_waitcnt_vm(0));
        __builtin_amdgcn_s_barrier();
        if (kt + STAGES < nk) dma(kt + STAGES);  // into the stage of tile kt, read by every wave
        if (kt + 1 < nk) read_tile(IC<sl ^ 1>{}, kt + 1);
        static_for<0, SUB * KCG>([&](auto UC) {
            constexpr int u = decltype(UC)::value / KCG, c = decltype(UC)::value % KCG;
            static_for<0, 4>([&](auto S) {
                constexpr int s4 = decltype(S)::value;
                static_for<0, TM>([&](auto I) {
                    constexpr int i = decltype(I)::value;
                    static_for<0, TN>([&](auto J) {
                        constexpr int j = decltype(J)::value;
                        float av, bv;
                        if constexpr (A_KC) av = fak[sl][u][c][i][s4];
                        else av = fam[sl][u][c][i][s4];
                        if constexpr (B_KC) bv = fbk[sl][u][c][j][s4];
                        else bv = fbm[sl][u][c][j][s4];
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc[i][j], 0, 0, 0);
                    });
                });
            });
        });
    };
    for (int kt = 0; kt < nk; kt += 2) {
        step(IC<0>{}, kt);
        if (kt + 1 < nk) step(IC<1>{}, kt + 1);
    }
    __builtin_amdgcn_s_barrier();  // every wave is done with the ring (exchange reuses it)

    if constexpr (KG > 1) {
        float *xl = reinterpret_cast<float *>(lds);
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
                    if (owner != kg) xl[slot(owner, kg, i, j, v % VH)] = acc[i][j][v];
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
                            if (sdr != kg) acc[i][j][v] += xl[slot(owner, sdr, i, j, v % VH)];
                    }
                });
    }

#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int col = n0 + wn * WTN + j * 32 + r32;
        if (col >= N) continue;
        const float bv = bias ? bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int rb = m0 + wm * WTM + i * 32 + g * 4;
            // old C (accumulate) or the epilogue's input operand, loaded as a
            // batch before the stores
            constexpr bool AUX = EPI == EPI_RESID || EPI == EPI_GELU_BWD;
            float old[16];
            if (AUX || accumulate) {
                const auto src = gbl(AUX ? aux_in : Cm);
                const long lds_ = AUX ? ld_aux : ldcm;
                static_for<0, 16>([&](auto V) {
                    constexpr int v = V.value;
                    if (KG == 1 || v / VH == kg)
                        old[v] = src[(long)min(rb + (v >> 2) * 8 + (v & 3), M - 1) * lds_ + col];
                });
            }
            static_for<0, 16>([&](auto V) {
                constexpr int v = V.value;
                if (KG == 1 || v / VH == kg) {
                    const int row = rb + (v >> 2) * 8 + (v & 3);
                    if (row < M) {
                        float out = acc[i][j][v] + bv;
                        if constexpr (EPI == EPI_GELU) {
                            if (aux_out) aux_out[(long)row * ld_aux + col] = out;
                            out = gelu_f(out);
                        } else if constexpr (EPI == EPI_RESID) {
                            out = old[v] + out;
                        } else if constexpr (EPI == EPI_GELU_BWD) {
                            out = out * gelu_grad(old[v]);
                        } else if (accumulate) {
                            out = old[v] + out;
                        }
                        gbl(Cm)[(long)row * ldcm + col] = out;
                    }
                }
            });
        }
    }
}

template <int BM, int BN, int KG, int STAGES, int SUB, bool A_KC, bool B_KC, int EPI = EPI_NONE>
static hipError_t launch_dma(int M, int N, int K, int splits, int kchunk, const float *A, long lda,
                             const float *B, long ldb, const float *bias, int accumulate, float *C,
                             long ldc, hipStream_t stream, const float *aux_in = nullptr,
                             float *aux_out = nullptr, long ld_aux = 0) {
    const int nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL((sgemm_dma_kernel<BM, BN, KG, STAGES, SUB, A_KC, B_KC, EPI>), dim3(nblk, splits),
                       dim3(256 * KG), 0, stream, A, lda, B, ldb, bias, C, ldc, M, N, K, accumulate,
                       kchunk, aux_in, aux_out, ld_aux);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The same products on v_mfma_f32_16x16x4f32, which sustains a higher f32
// rate on this part than the 32x32x2 form (145 against ~135 TFLOP/s for a
// loop of nothing but MFMAs), with a ring small enough for two workgroups
// per CU (their barriers are independent, so a SIMD always has a second wave
// to issue from).
//
// Tile: BM x BN per workgroup of WM x WN waves (2 x 2 in every launch here;
// OCC workgroups per CU size the LDS budget); a wave owns (BM/WM) x (BN/WN)
// as TM x TN blocks of 16x16. A ring stage holds BK = 16 SUB
// k (SUB = 1 or 2), used as SUB sub-steps of 16: lane (r16, q) = (lane % 16,
// lane / 16) feeds k = 16u + 4q + s at MFMA step s of sub-step u (the same
// for A and B, so the sum over k is unchanged) and holds outputs (4q + v,
// r16) of a block. LDS layouts, unpadded and swizzled (SQ_LDS_BANK_CONFLICT
// reads zero):
//  * K-contiguous operand: rows of 4 BK bytes (4 SUB pieces of 16 bytes);
//    logical piece p of row r sits at p ^ ((r >> 1) & (4 SUB - 1)). A lane
//    reads one piece (its four k) per block per sub-step. (For 64-byte rows
//    the map (r >> 2) & 3 conflicts; for 128-byte rows (r >> 1) & 3 and
//    ((r >> 1) & 3) | ((r & 1) << 2) do.)
//  * MN-contiguous operand: BK k-rows of ROWS floats; logical 16-byte chunk
//    c of k-row k sits at c ^ (((k >> 2) & 3) << 2). A lane reads four floats
//    (k = 16u + 4q .. + 3) per block per sub-step.
// Per sub-step: wait for this wave's reads of the sub-step's fragments; on
// the last sub-step of a stage also wait for this wave's DMA of the next
// stage and cross the stage's one barrier (after it every wave has read this
// stage and every DMA of the next has landed); read the next sub-step's
// fragments (the next stage's first after the barrier) while this
// sub-step's MFMAs run; on the last sub-step refill this stage (tile kt +
// STAGES) with the DMA instructions spread among the MFMAs (issued together
// they stall the wave). Every stage issues one tile's DMA (clamped to the
// last tile past the end, into a stage no one reads again), so the wait is
// always vmcnt((STAGES - 2) * LOADS). What decides between the shapes is
// how far ahead the DMA runs, (STAGES - 1) * BK k: 128x128 tiles take a
// 4-stage ring of 16-deep stages (48 k ahead in 64 KB; 32-deep stages fit
// only two, 32 k ahead, 3-5% slower), 128x64 tiles a 3-stage ring of
// 32-deep stages (64 k ahead in 72 KB).
template <int ROWS, bool KC, int NW, int BK>
struct Dma16 {
    static constexpr int PC = BK / 4;                // 16-byte pieces per K-contiguous row
    static constexpr int BYTES = ROWS * BK * 4;      // one ring stage of this operand
    static constexpr int INST = BYTES / 1024;
    static constexpr int PER_WAVE = INST / NW;
    static_assert(INST % NW == 0, "DMA instructions must split over the waves");
    static constexpr int CHR = ROWS / 4;  // 16-byte chunks per MN-contiguous k-row
    static_assert(KC || CHR % 16 == 0, "MN swizzle needs a multiple of 16 chunks per k-row");
    __device__ __forceinline__ static void setup(long (&voff)[PER_WAVE], int (&ldso)[PER_WAVE], int wave,
                                                 int lane, int rows0, int nrows, long ld) {
#pragma unroll
        for (int q = 0; q < PER_WAVE; q++) {
            const int inst = q * NW + wave;
            if (KC) {
                const int r = inst * (64 / PC) + lane / PC;
                const int gp = (lane % PC) ^ ((r >> 1) & (PC - 1));
                voff[q] = (long)min(rows0 + r, nrows - 1) * ld + gp * 4;
            } else {
                const int e = inst * 64 + lane, k = e / CHR, c = e % CHR;
                const int gc = c ^ (((k >> 2) & 3) << 2);
                voff[q] = (long)k * ld + min(rows0 + gc * 4, nrows - 4);
            }
            ldso[q] = inst * 1024;
        }
    }
    __device__ __forceinline__ static void dma(const float *P, long ld, int k0, const long (&voff)[PER_WAVE],
                                               const int (&ldso)[PER_WAVE], int8_t *lds_stage) {
        const float *base = KC ? P + k0 : P + (long)k0 * ld;
#pragma unroll
        for (int q = 0; q < PER_WAVE; q++)
            __builtin_amdgcn_global_load_lds((const void *)(base + voff[q]),
                                             (__attribute__((address_space(3))) void *)(lds_stage + ldso[q]),
                                             16, 0, 0);
    }
};

template <int BM, int BN, int STAGES, int SUB, bool A_KC, bool B_KC, int EPI = EPI_NONE, int WM = 2,
          int WN = 2, int OCC = 2>
__global__ __launch_bounds__(64 * WM * WN, OCC) void sgemm16_kernel(
    const float *__restrict__ A, long lda, const float *__restrict__ B, long ldb,
    const float *__restrict__ bias, float *__restrict__ C, long ldc, int M, int N, int K,
    int accumulate, int kchunk, const float *__restrict__ aux_in, float *__restrict__ aux_out,
    long ld_aux) {
    constexpr int NW = WM * WN;
    constexpr int BK = 16 * SUB, PC = 4 * SUB;
    static_assert(SUB == 1 || SUB == 2, "16- or 32-deep stages");
    using TA = Dma16<BM, A_KC, NW, BK>;
    using TB = Dma16<BN, B_KC, NW, BK>;
    constexpr int STAGE = TA::BYTES + TB::BYTES;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 16, TN = WTN / 16;
    constexpr int LOADS = TA::PER_WAVE + TB::PER_WAVE;
    static_assert(STAGES >= 2 && (STAGES - 1) * LOADS <= 63, "vmcnt range");
    static_assert(STAGE <= 65536 && STAGES * STAGE <= 160 * 1024 / OCC, "OCC workgroups per CU");
    static_assert(WTM % 16 == 0 && WTN % 16 == 0, "tile");
    __shared__ __attribute__((aligned(1024))) int8_t lds[STAGES * STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int r16 = lane & 15, q = lane >> 4;

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
    const int nk = K / BK;

    long voa[TA::PER_WAVE], vob[TB::PER_WAVE];
    int lda_o[TA::PER_WAVE], ldb_o[TB::PER_WAVE];
    TA::setup(voa, lda_o, wave, lane, m0, M, lda);
    TB::setup(vob, ldb_o, wave, lane, n0, N, ldb);
    auto dma = [&](int t) {
        int8_t *st = lds + (t % STAGES) * STAGE;
        const int tk = min(t, nk - 1);
        TA::dma(A, lda, tk * BK, voa, lda_o, st);
        TB::dma(B, ldb, tk * BK, vob, ldb_o, st + TA::BYTES);
    };
    // fragment addresses within a stage (block offsets as immediates; the
    // K-contiguous swizzle depends only on r16 since row bases are multiples
    // of 16)
    const unsigned lds0 = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)lds;
    unsigned a_addr[A_KC ? SUB : TM], b_addr[B_KC ? SUB : TN];
    if constexpr (A_KC) {
#pragma unroll
        for (int u = 0; u < SUB; u++)
            a_addr[u] = (wm * WTM + r16) * (4 * BK) + (((4 * u + q) ^ ((r16 >> 1) & (PC - 1))) << 4);
    } else {
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int m = wm * WTM + i * 16 + r16;
            a_addr[i] = 4 * q * BM * 4 + (((m >> 2) ^ (q << 2)) << 4) + (m & 3) * 4;
        }
    }
    if constexpr (B_KC) {
#pragma unroll
        for (int u = 0; u < SUB; u++)
            b_addr[u] = TA::BYTES + (wn * WTN + r16) * (4 * BK) + (((4 * u + q) ^ ((r16 >> 1) & (PC - 1))) << 4);
    } else {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = wn * WTN + j * 16 + r16;
            b_addr[j] = TA::BYTES + 4 * q * BN * 4 + (((n >> 2) ^ (q << 2)) << 4) + (n & 3) * 4;
        }
    }
    v4f fak[2][A_KC ? TM : 1], fbk[2][B_KC ? TN : 1];
    float fam[2][A_KC ? 1 : TM][4], fbm[2][B_KC ? 1 : TN][4];
    // sub-step u of the stage at st into slot sl
    auto read_sub = [&](auto SL, auto U, unsigned st) {
        constexpr int sl = decltype(SL)::value, u = decltype(U)::value;
        static_for<0, TM>([&](auto I) {
            constexpr int i = decltype(I)::value;
            if constexpr (A_KC) {
                sd_read128<i * 16 * 4 * BK>(fak[sl][i], st + a_addr[u]);
            } else {
                sd_read32<(16 * u + 0) * BM * 4>(fam[sl][i][0], st + a_addr[i]);
                sd_read32<(16 * u + 1) * BM * 4>(fam[sl][i][1], st + a_addr[i]);
                sd_read32<(16 * u + 2) * BM * 4>(fam[sl][i][2], st + a_addr[i]);
                sd_read32<(16 * u + 3) * BM * 4>(fam[sl][i][3], st + a_addr[i]);
            }
        });
        static_for<0, TN>([&](auto J) {
            constexpr int j = decltype(J)::value;
            if constexpr (B_KC) {
                sd_read128<j * 16 * 4 * BK>(fbk[sl][j], st + b_addr[u]);
            } else {
                sd_read32<(16 * u + 0) * BN * 4>(fbm[sl][j][0], st + b_addr[j]);
                sd_read32<(16 * u + 1) * BN * 4>(fbm[sl][j][1], st + b_addr[j]);
                sd_read32<(16 * u + 2) * BN * 4>(fbm[sl][j][2], st + b_addr[j]);
                sd_read32<(16 * u + 3) * BN * 4>(fbm[sl][j][3], st + b_addr[j]);
            }
        });
    };
    auto fence_slot = [&](auto SL) {
        constexpr int sl = decltype(SL)::value;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            if constexpr (A_KC) {
                sd_fence(fak[sl][i]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) sd_fence(fam[sl][i][e]);
            }
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if constexpr (B_KC) {
                sd_fence(fbk[sl][j]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) sd_fence(fbm[sl][j][e]);
            }
        }
    };
    v4f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    auto mfma_sub = [&](auto SL) {
        constexpr int sl = decltype(SL)::value;
        static_for<0, 4>([&](auto S) {
            constexpr int s4 = decltype(S)::value;
            static_for<0, TM>([&](auto I) {
                constexpr int i = decltype(I)::value;
                static_for<0, TN>([&](auto J) {
                    constexpr int j = decltype(J)::value;
                    float av, bv;
                    if constexpr (A_KC) av = fak[sl][i][s4];
                    else av = fam[sl][i][s4];
                    if constexpr (B_KC) bv = fbk[sl][j][s4];
                    else bv = fbm[sl][j][s4];
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[i][j], 0, 0, 0);
                });
            });
        });
    };

    float *Cm = C;
    long ldcm = ldc;
    asm volatile("" : "+s"(Cm), "+s"(ldcm));

    constexpr int NMF = 4 * TM * TN, NRD = (A_KC ? TM : 4 * TM) + (B_KC ? TN : 4 * TN);
    constexpr int PER = NMF / LOADS > 0 ? NMF / LOADS : 1;
    constexpr int REST = NMF - PER * LOADS > 0 ? NMF - PER * LOADS : 0;
    if (nk > 0) {
#pragma unroll
        for (int t = 0; t < STAGES; t++) dma(t);
        __builtin_amdgcn_s_waitcnt(sd_waitcnt_vm((STAGES - 1) * LOADS));
        __builtin_amdgcn_s_barrier();
        read_sub(IC<0>{}, IC<0>{}, lds0);
        // sub-step U of stage kt, its fragments in slot SL
        auto sub = [&](auto SL, auto U, int kt) {
            constexpr int sl = decltype(SL)::value, u = decltype(U)::value;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            fence_slot(SL);
            if constexpr (u + 1 < SUB) {
                __builtin_amdgcn_sched_barrier(0);
                read_sub(IC<sl ^ 1>{}, IC<u + 1>{}, lds0 + (kt % STAGES) * STAGE);
                __builtin_amdgcn_sched_barrier(0);
                mfma_sub(SL);
                __builtin_amdgcn_sched_barrier(0);
            } else {
                __builtin_amdgcn_s_waitcnt(sd_waitcnt_vm((STAGES - 2) * LOADS));
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                read_sub(IC<sl ^ 1>{}, IC<0>{}, lds0 + ((kt + 1) % STAGES) * STAGE);
                mfma_sub(SL);
                dma(kt + STAGES);
                __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);  // LDS reads
                static_for<0, LOADS>([&](auto) {
                    __builtin_amdgcn_sched_group_barrier(0x008, PER, 0);  // MFMAs
                    __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);    // one DMA
                });
                if constexpr (REST > 0) __builtin_amdgcn_sched_group_barrier(0x008, REST, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        if constexpr (SUB == 2) {
            for (int kt = 0; kt < nk; kt++) {
                sub(IC<0>{}, IC<0>{}, kt);
                sub(IC<1>{}, IC<1>{}, kt);
            }
        } else {
            // one sub-step per stage: the slot alternates with the stage
            int kt = 0;
            for (; kt + 1 < nk; kt += 2) {
                sub(IC<0>{}, IC<0>{}, kt);
                sub(IC<1>{}, IC<0>{}, kt + 1);
            }
            if (kt < nk) sub(IC<0>{}, IC<0>{}, kt);
        }
        // no DMA or fragment read in flight past the loop
        __builtin_amdgcn_s_waitcnt(sd_waitcnt_vm(0));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }

    // Epilogue. A tile wholly inside C takes the form without bounds checks.
    // One address per output row (row * ldc once per row, the TN columns at
    // immediate offsets); C is stored through a global pointer (the asm above
    // hides its provenance, which would otherwise give flat stores).
    typedef __attribute__((address_space(1))) float gfloat;
    gfloat *Cg = (gfloat *)Cm;
    constexpr bool AUX = EPI == EPI_RESID || EPI == EPI_GELU_BWD;
    const int row0 = m0 + wm * WTM + 4 * q, col0 = n0 + wn * WTN + r16;
    auto store = [&](auto CHECK) {
        constexpr bool chk = decltype(CHECK)::value != 0;
        float bv[TN];
        int cj[TN];  // column of block j (clamped into C when checking)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            cj[j] = chk ? min(col0 + j * 16, N - 1) : col0 + j * 16;
            bv[j] = bias ? bias[cj[j]] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < TM; i++) {
            float old[4][TN];
            if (AUX || accumulate) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int row = chk ? min(row0 + i * 16 + v, M - 1) : row0 + i * 16 + v;
                    if constexpr (AUX) {
                        const float *src = aux_in + (long)row * ld_aux;
#pragma unroll
                        for (int j = 0; j < TN; j++) old[v][j] = src[cj[j]];
                    } else {
                        const gfloat *src = Cg + (long)row * ldcm;
#pragma unroll
                        for (int j = 0; j < TN; j++) old[v][j] = src[cj[j]];
                    }
                }
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int row = row0 + i * 16 + v;
                if (chk && row >= M) continue;
                gfloat *dst = Cg + (long)row * ldcm;
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    if (chk && col0 + j * 16 >= N) continue;
                    float out = acc[i][j][v] + bv[j];
                    if constexpr (EPI == EPI_GELU) {
                        if (aux_out) aux_out[(long)row * ld_aux + cj[j]] = out;
                        out = gelu_f(out);
                    } else if constexpr (EPI == EPI_RESID) {
                        out = old[v][j] + out;
                    } else if constexpr (EPI == EPI_GELU_BWD) {
                        out = out * gelu_grad(old[v][j]);
                    } else if (accumulate) {
                        out = old[v][j] + out;
                    }
                    dst[cj[j]] = out;
                }
            }
        }
    };
    if (m0 + BM <= M && n0 + BN <= N)
        store(IC<0>{});
    else
        store(IC<1>{});
}

template <int BM, int BN, int STAGES, int SUB, bool A_KC, bool B_KC, int EPI = EPI_NONE, int WM = 2, int WN = 2,
          int OCC = 2>
static hipError_t launch_s16(int M, int N, int K, int splits, int kchunk, const float *A, long lda,
                             const float *B, long ldb, const float *bias, int accumulate, float *C,
                             long ldc, hipStream_t stream, const float *aux_in = nullptr,
                             float *aux_out = nullptr, long ld_aux = 0) {
    const int nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL((sgemm16_kernel<BM, BN, STAGES, SUB, A_KC, B_KC, EPI, WM, WN, OCC>), dim3(nblk, splits),
                       dim3(64 * WM * WN), 0,
                       stream, A, lda, B, ldb, bias, C, ldc, M, N, K, accumulate, kchunk, aux_in, aux_out,
                       ld_aux);
    return hipGetLastError();
}

// Split-K epilogue: C = (accumulate ? C : 0) + (P_0 + P_1 + ... + bias), the
// partial products added in split order (deterministic).
// Grid (ceil(N / 256), M); applies the epilogue (accumulate only with EPI_NONE).
__global__ void sgemm_splitk_reduce_kernel(const float *__restrict__ P, int splits, int M, int N,
                                           const float *__restrict__ bias, float *__restrict__ C,
                                           long ldc, int accumulate, int epi,
                                           const float *__restrict__ aux_in,
                                           float *__restrict__ aux_out, long ld_aux) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    const long m = blockIdx.y;
    if (n >= N) return;
    const long MN = (long)M * N, i = m * N + n;
    float s = P[i];
    for (int z = 1; z < splits; z++) s += P[z * MN + i];
    float out = s + (bias ? bias[n] : 0.f);
    float *c = C + m * ldc + n;
    const long ai = m * ld_aux + n;
    if (epi == EPI_GELU) out = apply_epi<EPI_GELU>(out, aux_in, aux_out, ai);
    else if (epi == EPI_RESID) out = apply_epi<EPI_RESID>(out, aux_in, aux_out, ai);
    else if (epi == EPI_GELU_BWD) out = apply_epi<EPI_GELU_BWD>(out, aux_in, aux_out, ai);
    else if (accumulate) out = *c + out;
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
    SG_32x64 = 4,        // 32x64 on the 16x16x4 kernel, no split (A K-contiguous, K <= 512)
};

SgemmPlan plan_sgemm(int M, int N, int K, bool a_kcontig) {
    SgemmPlan p{SG_64_KG2, 1, K > 0 ? K : 1, 0};
    const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    const long t64 = (long)((M + 63) / 64) * ((N + 63) / 64);
    // Grids too small for 256 CUs with a short K (the grown model's prefill
    // products, M = 256): 32x64 tiles in one launch -- twice the workgroups of
    // 64x64 and no split-K sum pass (256 x 1536 x 512: 12.0 -> 8.6 us, the NT
    // head 11.0 -> 7.5, 256 x 512 x 512: 9.9 -> 8.5; with K = 2048 the split
    // stays ahead, 13.1 against 26.9 us).
    if (a_kcontig && t64 < 256 && K >= 32 && K <= 512) {
        p.cfg = SG_32x64;
        return p;
    }
    if (t128 >= 512) {
        // whole rounds of 2 per CU take the deeper tile, otherwise 4 per CU
        // keep more of the grid resident at once
        p.cfg = t128 % 512 == 0 ? SG_128_BK32 : SG_128_BK16;
    } else if (t128 >= 256) {
        p.cfg = SG_128_KG2;
    } else if (t64 < 256 && K >= 128) {
        // too few tiles for 256 CUs: split K (chunks of whole 64-deep tiles);
        // grids of 129-255 tiles with a long K take 2+ workgroups per CU
        int splits = (int)(256 / (t64 > 0 ? t64 : 1));
        if (splits < 2 && K >= 2048) splits = (int)((512 + t64 - 1) / t64);
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

// Grids of at least two workgroups per CU take the 16x16x4 kernel (its
// workgroups pair up on a CU): 1 = 128x128 tiles, 2 = grids that have only one
// 128x128 tile per CU: one 128x128 workgroup of 8 waves (32x64 each; 16-deep
// stages, 32-deep for NT) per CU, or for TT two 128x64 workgroups of 4 waves,
// 3 = 64x64 tiles (two per CU only at that size, e.g. 2048 x 1024), 0 = the
// 32x32x2 kernel (smaller grids, where its two K groups keep two waves on
// every SIMD). Measured on the 350M-class shapes: 128x128 +8-11% where it
// applies; the 8-wave 128x128 workgroup +3-7% over two 128x64 ones (the
// attention projection, FF2 and dW); 64x64 on 2048 x 1024 x 1024: +11% (with
// one 64x64 tile per CU, 1024^3, it is not ahead).
static int s16_tile(int M, int N) {
    const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    const long t64 = (long)((M + 127) / 128) * ((N + 63) / 64);
    const long t6464 = (long)((M + 63) / 64) * ((N + 63) / 64);
    if (t128 >= 512) return 1;
    if (t64 >= 512) return 2;
    if (t6464 >= 512) return 3;
    return 0;
}

// Route 1 of s16_tile: two 4-wave 128x128 workgroups per CU (192-wide tiles
// where those fill the chip better, below); for NN, one
// 8-wave 128x256 workgroup per CU (a quarter less LDS fill per CU) where its
// tiles fill whole rounds of 256 CUs (at least two, at most 1/16 of the last
// round idle): +2.6-3.2% on 4096 x 4096 x 1024 and three other NN grids of
// 512-768 such tiles; on 4096 x 3072 (384 tiles, half a round idle) it was
// 21% slower, and on NT and TN grids slower or level.
static bool s16_wide_nn(int M, int N) {
    const long t = (long)((M + 127) / 128) * ((N + 255) / 256);
    const long slots = (t + 255) / 256 * 256;
    return t >= 512 && (slots - t) * 16 <= 256;
}

// Share of the launched tile area that lies inside C when tiles of BM x BN
// run `per_round` at a time (rounds of the whole chip).
static double s16_fill(int M, int N, int BM, int BN, int per_round) {
    const long t = (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const long slots = (t + per_round - 1) / per_round * per_round;
    return (double)M * N / ((double)slots * BM * BN);
}

// 192-wide tiles where they fill the chip's rounds clearly better than
// 128x128 (4096 x 3072: 512 tiles of 128x192, one round, against 768 of
// 128x128, a round and a half): two 4-wave 128x192 workgroups per CU, or for
// NT one 8-wave 256x192 workgroup on 32-deep stages when that fills as well.
// Measured on 4096 x 3072 x 1024: NN +3.7%, TN +2.6%, NT +4.8% (+2.7% with
// 128x192).
static int s16_wide192(int M, int N, bool nt) {
    const double f128 = s16_fill(M, N, 128, 128, 512), f192 = s16_fill(M, N, 128, 192, 512);
    if (f192 <= f128 + 0.05) return 0;
    return nt && s16_fill(M, N, 256, 192, 256) >= f192 ? 2 : 1;
}

template <bool A_KC, bool B_KC, int EPI = EPI_NONE>
static hipError_t launch_s16_two_per_cu(int M, int N, int K, const float *A, long lda, const float *B,
                                        long ldb, const float *bias, int accumulate, float *C, long ldc,
                                        hipStream_t stream, const float *aux_in = nullptr,
                                        float *aux_out = nullptr, long ld_aux = 0) {
    if constexpr (A_KC && !B_KC) {
        if (s16_wide_nn(M, N))
            return launch_s16<128, 256, 4, 1, A_KC, B_KC, EPI, 2, 4, 1>(M, N, K, 1, K, A, lda, B, ldb, bias,
                                                                      accumulate, C, ldc, stream, aux_in, aux_out,
                                                                      ld_aux);
    }
    const int w192 = s16_wide192(M, N, A_KC && B_KC);
    if constexpr (A_KC && B_KC) {
        if (w192 == 2)
            return launch_s16<256, 192, 2, 2, A_KC, B_KC, EPI, 4, 2, 1>(M, N, K, 1, K, A, lda, B, ldb, bias,
                                                                      accumulate, C, ldc, stream, aux_in, aux_out,
                                                                      ld_aux);
    }
    if (w192)
        return launch_s16<128, 192, 4, 1, A_KC, B_KC, EPI>(M, N, K, 1, K, A, lda, B, ldb, bias, accumulate, C, ldc,
                                                         stream, aux_in, aux_out, ld_aux);
    return launch_s16<128, 128, 4, 1, A_KC, B_KC, EPI>(M, N, K, 1, K, A, lda, B, ldb, bias, accumulate, C, ldc,
                                                     stream, aux_in, aux_out, ld_aux);
}

// Route 2 of s16_tile: one 8-wave 128x128 workgroup per CU (NT on 32-deep
// stages), two 4-wave 128x64 workgroups for TT.
template <bool A_KC, bool B_KC, int EPI = EPI_NONE>
static hipError_t launch_s16_one_per_cu(int M, int N, int K, const float *A, long lda, const float *B,
                                        long ldb, const float *bias, int accumulate, float *C, long ldc,
                                        hipStream_t stream, const float *aux_in = nullptr,
                                        float *aux_out = nullptr, long ld_aux = 0) {
    if constexpr (!A_KC && B_KC)
        return launch_s16<128, 64, 3, 2, A_KC, B_KC, EPI>(M, N, K, 1, K, A, lda, B, ldb, bias, accumulate, C,
                                                        ldc, stream, aux_in, aux_out, ld_aux);
    else if constexpr (A_KC && B_KC)
        return launch_s16<128, 128, 4, 2, A_KC, B_KC, EPI, 4, 2, 1>(M, N, K, 1, K, A, lda, B, ldb, bias,
                                                                  accumulate, C, ldc, stream, aux_in, aux_out,
                                                                  ld_aux);
    else
        return launch_s16<128, 128, 4, 1, A_KC, B_KC, EPI, 4, 2, 1>(M, N, K, 1, K, A, lda, B, ldb, bias,
                                                                  accumulate, C, ldc, stream, aux_in, aux_out,
                                                                  ld_aux);
}

// Fused epilogues exist for the layouts the trainer uses them in: NN
// (forward FF1 + GELU, O / FF2 + residual) and NT (dX of FF2 times GELU').
template <bool A_KC, bool B_KC>
constexpr bool epi_fused(int epi) {
    return (A_KC && !B_KC && (epi == EPI_GELU || epi == EPI_RESID)) ||
           (A_KC && B_KC && epi == EPI_GELU_BWD);
}

template <bool A_KC, bool B_KC, int EPI>
static hipError_t launch_dma_epi(const SgemmPlan &p, int M, int N, int K, const float *A, long lda,
                                 const float *B, long ldb, const float *bias, float *C, long ldc,
                                 const float *aux_in, float *aux_out, long ld_aux,
                                 hipStream_t stream) {
    const int s16 = s16_tile(M, N);
    if (s16 == 1)
        return launch_s16_two_per_cu<A_KC, B_KC, EPI>(M, N, K, A, lda, B, ldb, bias, 0, C, ldc, stream, aux_in,
                                                      aux_out, ld_aux);
    if (s16 == 2)
        return launch_s16_one_per_cu<A_KC, B_KC, EPI>(M, N, K, A, lda, B, ldb, bias, 0, C, ldc, stream, aux_in,
                                                      aux_out, ld_aux);
    if (s16 == 3)
        return launch_s16<64, 64, 4, 1, A_KC, B_KC, EPI>(M, N, K, 1, K, A, lda, B, ldb, bias, 0, C, ldc,
                                                       stream, aux_in, aux_out, ld_aux);
    if constexpr (A_KC) {
        if (p.cfg == SG_32x64)
            return launch_s16<32, 64, 3, 2, A_KC, B_KC, EPI, 2, 2, 4>(M, N, K, 1, K, A, lda, B, ldb, bias, 0, C,
                                                                    ldc, stream, aux_in, aux_out, ld_aux);
    }
    if (p.cfg == SG_64_KG2)
        return launch_dma<64, 64, 2, 2, 1, A_KC, B_KC, EPI>(M, N, K, 1, K, A, lda, B, ldb, bias, 0, C,
                                                            ldc, stream, aux_in, aux_out, ld_aux);
    return launch_dma<128, 128, 2, 2, 1, A_KC, B_KC, EPI>(M, N, K, 1, K, A, lda, B, ldb, bias, 0, C,
                                                          ldc, stream, aux_in, aux_out, ld_aux);
}

template <bool A_KC, bool B_KC>
static hipError_t dispatch_layout(const SgemmPlan &p, int M, int N, int K, const float *A,
                                  long lda, const float *B, long ldb, const float *bias,
                                  int accumulate, float *C, long ldc, const Workspace &ws,
                                  hipStream_t stream, int epi, const float *aux_in,
                                  float *aux_out, long ld_aux) {
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
    // Aligned operands with K a multiple of 32 (per split as well: split
    // chunks are multiples of 64) take the LDS-DMA pipeline.
    const bool dma_ok = vec && K % SD_BK == 0;
    // With a K split the reduce pass applies the epilogue (below); otherwise the
    // GEMM kernel does (fused layouts) or one elementwise pass after the product.
    if (epi != EPI_NONE && !split) {
        if (dma_ok && epi_fused<A_KC, B_KC>(epi)) {
            if constexpr (A_KC && !B_KC) {
                if (epi == EPI_GELU)
                    return launch_dma_epi<A_KC, B_KC, EPI_GELU>(p, M, N, K, A, lda, B, ldb, bias, C, ldc,
                                                                aux_in, aux_out, ld_aux, stream);
                return launch_dma_epi<A_KC, B_KC, EPI_RESID>(p, M, N, K, A, lda, B, ldb, bias, C, ldc,
                                                             aux_in, aux_out, ld_aux, stream);
            } else if constexpr (A_KC && B_KC) {
                return launch_dma_epi<A_KC, B_KC, EPI_GELU_BWD>(p, M, N, K, A, lda, B, ldb, bias, C,
                                                                ldc, aux_in, aux_out, ld_aux, stream);
            }
        }
        e = dispatch_layout<A_KC, B_KC>(p, M, N, K, A, lda, B, ldb, bias, 0, C, ldc, ws, stream,
                                        EPI_NONE, nullptr, nullptr, 0);
        if (e != hipSuccess) return e;
        if ((long)M * N == 0) return hipSuccess;
        hipLaunchKernelGGL(sgemm_epilogue_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)M),
                           dim3(256), 0, stream, epi, M, N, C, ldc, aux_in, aux_out, ld_aux);
        return hipGetLastError();
    }
    const int s16 = split ? 0 : s16_tile(M, N);
    if (dma_ok && s16 == 1) {
        e = launch_s16_two_per_cu<A_KC, B_KC>(M, N, K, A, lda, B, ldb, b, acc, out, ldo, stream);
    } else if (dma_ok && s16 == 2) {
        e = launch_s16_one_per_cu<A_KC, B_KC>(M, N, K, A, lda, B, ldb, b, acc, out, ldo, stream);
    } else if (dma_ok && s16 == 3) {
        e = launch_s16<64, 64, 4, 1, A_KC, B_KC>(M, N, K, 1, K, A, lda, B, ldb, b, acc, out, ldo, stream);
    } else if (A_KC && dma_ok && p.cfg == SG_32x64) {
        // 16x16 blocks of 16 x 32 per wave (2 x 2 waves), 32-deep stages, a
        // 3-stage ring sized for four workgroups per CU
        if constexpr (A_KC)
            e = launch_s16<32, 64, 3, 2, A_KC, B_KC, EPI_NONE, 2, 2, 4>(M, N, K, 1, K, A, lda, B, ldb, b, acc,
                                                                      out, ldo, stream);
    } else if (dma_ok) {
        if (p.cfg == SG_64_KG2)
            e = launch_dma<64, 64, 2, 2, 1, A_KC, B_KC>(M, N, K, p.splits, p.kchunk, A, lda, B, ldb, b,
                                                     acc, out, ldo, stream);
        else
            e = launch_dma<128, 128, 2, 2, 1, A_KC, B_KC>(M, N, K, p.splits, p.kchunk, A, lda, B, ldb, b,
                                                       acc, out, ldo, stream);
    } else switch (p.cfg) {
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
    hipLaunchKernelGGL(sgemm_splitk_reduce_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)M),
                       dim3(256), 0, stream, static_cast<const float *>(ws.buf), p.splits, M, N, bias,
                       C, ldc, accumulate, epi, aux_in, aux_out, ld_aux);
    return hipGetLastError();
}

hipError_t launch_sgemm(const SgemmPlan &p, bool a_kcontig, bool b_kcontig, int M, int N, int K,
                        const float *A, long lda, const float *B, long ldb, const float *bias,
                        int accumulate, float *C, long ldc, const Workspace &ws,
                        hipStream_t stream, int epi, const float *aux_in, float *aux_out,
                        long ld_aux) {
    if (a_kcontig && !b_kcontig)
        return dispatch_layout<true, false>(p, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, ws,
                                            stream, epi, aux_in, aux_out, ld_aux);
    if (a_kcontig && b_kcontig)
        return dispatch_layout<true, true>(p, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, ws,
                                           stream, epi, aux_in, aux_out, ld_aux);
    if (!a_kcontig && !b_kcontig)
        return dispatch_layout<false, false>(p, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc,
                                             ws, stream, epi, aux_in, aux_out, ld_aux);
    return dispatch_layout<false, true>(p, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, ws,
                                        stream, epi, aux_in, aux_out, ld_aux);
}

}  // namespace pcl
