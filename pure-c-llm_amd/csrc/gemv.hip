// gemv.hip -- decode-shaped products (M <= 8 token rows), bound by HBM.
//
//   sgemv_n: Y = X.W + bias, W K x N row-major (N-contiguous):
//            generate.c:95-107 matvec, transformer.c:174-195 proj_token.
//   sgemv_t: Y = X.W^T + bias, W N x K (K-contiguous): the tied head,
//            model.c:64-77 lm_head, generate.c:176-182.
//   igemv:   u8 x s8 -> int32 over the packed N x Kp weights, with the same
//            dequant epilogue as the INT8 GEMM (gemm_bench.c:260-285).
//   bias_bwd (gpu_kernels.cu:102-108) is sgemv_n with X = ones.
//
// Every weight byte is read exactly once, with 16-byte loads along the
// contiguous dimension; the few activation rows are staged in LDS per block.
// Each thread issues a batch of independent weight loads (clamped to valid
// addresses, no branches) before it consumes any of them, so a block keeps
// 16-32 KB of HBM reads in flight; the arithmetic on the batch is guarded.
// To fill 256 CUs when N alone gives too few blocks, K is split across
// blocks: each block writes its partial sums to a workspace and a second,
// small kernel adds the splits in split order (plus bias / accumulate /
// dequant), so results are deterministic run to run. The kernel boundary
// orders the two; no block ever waits on another, and no cross-XCD cache
// maintenance is issued inside a kernel.
#include "internal.h"

namespace pcl {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int GV_THREADS = 256;
constexpr int GV_TARGET_BLOCKS = 1024;   // ~4 per CU
// Activation rows staged in LDS per block: MR rows x KCH elements, sized so
// the staging takes 16 KB (sgemv_n), 32 KB (sgemv_t) or 16 KB (igemv).
template <int MR> struct Kch {
    static constexpr int SGN = 4096 / MR;   // floats
    static constexpr int SGT = 8192 / MR;   // floats
    static constexpr int IGV = 16384 / MR;  // bytes
};
constexpr int SGT_RPL = 2;               // sgemv_t / igemv rows per 16-lane group
constexpr int SGT_ROWS = 16 * SGT_RPL;   // rows of W per block

static int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

// Lane reductions on the DPP network (VALU operands from other lanes: no LDS
// crossbar round trip per step as a shuffle takes). An inclusive scan of
// row_shr 1, 2, 4, 8 leaves each 16-lane row's total in its last lane;
// row_bcast15 adds row 0's total into row 1 and row 2's into row 3, and
// row_bcast31 adds lane 31 into rows 2 and 3. The total (or, for values >= 0,
// the maximum) of each aligned group of W = 16, 32 or 64 lanes lands in the
// group's last lane; the other lanes hold partial results. Sources outside a
// row read 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xF, true);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, true));
}
template <int W>
__device__ __forceinline__ int dpp_sum_last(int v) {
    v += dpp_i<0x111, 0xF>(v);
    v += dpp_i<0x112, 0xF>(v);
    v += dpp_i<0x114, 0xF>(v);
    v += dpp_i<0x118, 0xF>(v);
    if constexpr (W >= 32) v += dpp_i<0x142, 0xA>(v);
    if constexpr (W >= 64) v += dpp_i<0x143, 0xC>(v);
    return v;
}
template <int W>
__device__ __forceinline__ float dpp_sum_last(float v) {
    v += dpp_f<0x111, 0xF>(v);
    v += dpp_f<0x112, 0xF>(v);
    v += dpp_f<0x114, 0xF>(v);
    v += dpp_f<0x118, 0xF>(v);
    if constexpr (W >= 32) v += dpp_f<0x142, 0xA>(v);
    if constexpr (W >= 64) v += dpp_f<0x143, 0xC>(v);
    return v;
}
__device__ __forceinline__ float dpp_max_last64(float v) {  // v >= 0
    v = fmaxf(v, dpp_f<0x111, 0xF>(v));
    v = fmaxf(v, dpp_f<0x112, 0xF>(v));
    v = fmaxf(v, dpp_f<0x114, 0xF>(v));
    v = fmaxf(v, dpp_f<0x118, 0xF>(v));
    v = fmaxf(v, dpp_f<0x142, 0xA>(v));
    v = fmaxf(v, dpp_f<0x143, 0xC>(v));
    return v;
}


// Stage MR activation rows of one split (elements [0, kchunk) of row m start
// at X0 + m*ldx; elements at or past kvalid, and rows m >= M, stage as zero)
// into LDS rows of stride ld. Each thread issues up to 16 independent loads
// (at most JUMAX per row) before it writes any of them, so the staging costs
// one memory latency rather than one per element; JUMAX caps the registers
// the batch holds (16 16-byte loads take 64 of them, which set the
// occupancy of the GEMVs with one or two rows). With 16-byte aligned rows the loads are
// 16-byte vectors (the chunk that straddles kvalid is assembled element by
// element); otherwise single elements. RECENTRE: u8 activations are stored
// as x ^ 0x80 (= x - 128 as s8), padding stays 0.
template <int MR, bool RECENTRE, typename T, int JUMAX = 4>
__device__ __forceinline__ void stage_rows(T *xs, int ld, int kchunk, int kvalid, int M,
                                           const T *X0, long ldx) {
    typedef T vec_t __attribute__((ext_vector_type(16 / sizeof(T))));
    constexpr int V = 16 / sizeof(T);
    const int tid = (int)threadIdx.x;
    auto fix = [](T x) -> T {
        if constexpr (RECENTRE) return (T)(x ^ (T)0x80);
        else return x;
    };
    const auto Xg = gbl(X0);
    const bool vec = ((reinterpret_cast<uintptr_t>(X0) | (uintptr_t)(ldx * sizeof(T))) & 15) == 0;
    if (vec) {
        const int nch = kchunk / V;                  // kchunk is a multiple of 64 elements
        if (MR > 1 && nch < GV_THREADS) {
            // Rows shorter than one chunk per thread: thread t takes chunk t % nch
            // of rows t / nch, t / nch + rp, ... (rp rows side by side), so every
            // wave shares the loads instead of the first nch threads holding
            // MR each while the others wait at the block's barrier.
            const int rp = GV_THREADS / nch, m0 = tid / nch, kk = (tid - m0 * nch) * V;
            if (m0 < rp) {
                vec_t v[MR];
#pragma unroll
                for (int s = 0; s < MR; s++) {
                    const int m = m0 + s * rp;
                    vec_t x = (T)0;
                    if (m < M) {
                        const auto src = Xg + (long)m * ldx + kk;
                        if (kk + V <= kvalid) {
                            x = *gvec<vec_t>(src);
                            if constexpr (RECENTRE) x ^= (T)0x80;
                        } else {
#pragma unroll
                            for (int e = 0; e < V; e++)
                                if (kk + e < kvalid) x[e] = fix(src[e]);
                        }
                    }
                    v[s] = x;
                }
#pragma unroll
                for (int s = 0; s < MR; s++) {
                    const int m = m0 + s * rp;
                    if (m < MR) *reinterpret_cast<vec_t *>(xs + m * ld + kk) = v[s];
                }
            }
            return;
        }
        constexpr int JU0 = MR >= 16 ? 1 : 16 / MR, JU = JU0 < JUMAX ? JU0 : JUMAX;  // vector loads per row per round
        for (int c0 = 0; c0 * GV_THREADS < nch; c0 += JU) {
            vec_t v[MR][JU];
#pragma unroll
            for (int m = 0; m < MR; m++)
#pragma unroll
                for (int ju = 0; ju < JU; ju++) {
                    const int kk = (tid + (c0 + ju) * GV_THREADS) * V;
                    vec_t x = (T)0;
                    if (m < M && kk < kchunk) {
                        const auto src = Xg + (long)m * ldx + kk;
                        if (kk + V <= kvalid) {
                            x = *gvec<vec_t>(src);
                            if constexpr (RECENTRE) x ^= (T)0x80;
                        } else {
#pragma unroll
                            for (int e = 0; e < V; e++)
                                if (kk + e < kvalid) x[e] = fix(src[e]);
                        }
                    }
                    v[m][ju] = x;
                }
#pragma unroll
            for (int m = 0; m < MR; m++)
#pragma unroll
                for (int ju = 0; ju < JU; ju++) {
                    const int kk = (tid + (c0 + ju) * GV_THREADS) * V;
                    if (kk < kchunk) *reinterpret_cast<vec_t *>(xs + m * ld + kk) = v[m][ju];
                }
        }
    } else {
        constexpr int JU0 = MR >= 16 ? 1 : 16 / MR, JU = JU0 < JUMAX ? JU0 : JUMAX;  // element loads per row per round
        for (int j0 = 0; j0 * GV_THREADS < kchunk; j0 += JU) {
            T v[MR][JU];
#pragma unroll
            for (int m = 0; m < MR; m++)
#pragma unroll
                for (int ju = 0; ju < JU; ju++) {
                    const int kk = tid + (j0 + ju) * GV_THREADS;
                    v[m][ju] = (m < M && kk < kvalid) ? fix(Xg[(long)m * ldx + kk]) : (T)0;
                }
#pragma unroll
            for (int m = 0; m < MR; m++)
#pragma unroll
                for (int ju = 0; ju < JU; ju++) {
                    const int kk = tid + (j0 + ju) * GV_THREADS;
                    if (kk < kchunk) xs[m * ld + kk] = v[m][ju];
                }
        }
    }
}

// Input transforms of the decode step applied to a staged activation row
// (M = 1): XF_LN = LayerNorm over the whole row X[0..K) (generate.c:106-114:
// mean, mean square deviation, (x - mu) * (1/sqrtf(var + 1e-5)) * g + b), of
// which this block holds elements [kb, kb + klen); XF_GELU = tanh-GELU
// (train.c:314-322) elementwise. Every block of a launch computes the same
// statistics in the same order, so all see identical values.
constexpr int XF_NONE = 0, XF_LN = 1, XF_GELU = 2;

__device__ __forceinline__ float gv_block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

template <int XF>
__device__ __forceinline__ void gv_xform(float *xs, int klen, int kb, int K,
                                         const float *__restrict__ X,
                                         const float *__restrict__ g,
                                         const float *__restrict__ b) {
    if constexpr (XF == XF_LN) {
        __shared__ float red[GV_THREADS / 64];
        float s = 0.f;
        for (int k = threadIdx.x; k < K; k += GV_THREADS) s += X[k];
        const float mu = gv_block_sum(s, red) / K;
        float q = 0.f;
        for (int k = threadIdx.x; k < K; k += GV_THREADS) {
            const float d = X[k] - mu;
            q += d * d;
        }
        const float var = gv_block_sum(q, red) / K;
        const float rs = 1.0f / sqrtf(var + 1e-5f);
        for (int k = threadIdx.x; k < klen; k += GV_THREADS)
            xs[k] = (xs[k] - mu) * rs * g[kb + k] + b[kb + k];
    } else if constexpr (XF == XF_GELU) {
        for (int k = threadIdx.x; k < klen; k += GV_THREADS) {
            const float v = xs[k];
            xs[k] = 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
        }
    }
    __syncthreads();
}

// Second pass of a split-K GEMV: Y[m,n] = sum over splits in order (+ bias,
// + Y when accumulating). part is [splits][M][nround]. Partials are loaded
// eight at a time before they are added (in split order), so a thread waits
// for one memory round trip per eight splits rather than per split: these
// grids are a few workgroups (a bias gradient of 1024 columns: four), so the
// loads' latency, not bandwidth, sets the time.
__global__ void sgemv_reduce_kernel(const float *__restrict__ part, int splits, int M, int N,
                                    int nround, const float *__restrict__ bias,
                                    float *__restrict__ Y, long ldy, int accumulate) {
    const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i >= (long)M * N) return;
    const int m = (int)(i / N), n = (int)(i % N);
    const long stride = (long)M * nround;
    const float *p = part + (long)m * nround + n;
    float s = 0.f;
    int q = 0;
    for (; q + 8 <= splits; q += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = p[(q + u) * stride];
#pragma unroll
        for (int u = 0; u < 8; u++) s += v[u];
    }
    for (; q < splits; q++) s += p[q * stride];
    float y = s + (bias ? bias[n] : 0.f);
    float *dst = Y + (long)m * ldy + n;
    *dst = accumulate ? *dst + y : y;
}

// ------------------------------------------------------------- sgemv_n ----
// Block = CW columns x kchunk rows of W. Thread (c4 = tid%(CW/4),
// rg = tid/(CW/4)) owns columns 4*c4..4*c4+3 and a contiguous run of
// kchunk/RG rows (RG = row groups per block). Narrow strips (CW = 16) give
// enough blocks without splitting K when N is small.
template <int MR, bool VEC, bool XONES, int CW>
__global__ __launch_bounds__(GV_THREADS) void sgemv_n_kernel(
    const float *__restrict__ X, long ldx, const float *__restrict__ W, long ldw,
    const float *__restrict__ bias, float *__restrict__ Y, long ldy, int M, int N, int K,
    int kchunk, int splits, float *__restrict__ part, int accumulate) {
    constexpr int CQ = CW / 4;             // threads across a strip row
    constexpr int RG = GV_THREADS / CQ;    // row groups
    __shared__ float red[RG][MR][CW];
    // activation rows of this split, MR x kchunk (dynamic: sized at launch)
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_dyn[];
    float *xs = reinterpret_cast<float *>(gv_dyn);

    const int tid = threadIdx.x;
    const int c4 = tid % CQ, rg = tid / CQ;
    const int strip = blockIdx.x, sp = blockIdx.y;
    const int n0 = strip * CW, col = n0 + 4 * c4;
    const int kb = sp * kchunk;
    const int run = kchunk / RG;  // multiple of 8

    const int r0 = rg * run;
    // column clamp keeps the vector loads in bounds; clamped lanes only feed
    // columns >= N, which are never stored. Rows past K are clamped for the
    // load and skipped in the arithmetic (the host never launches K == 0).
    const int colc = VEC ? min(col, N - 4) : col;
    constexpr int UR = 8;  // rows per load batch (run is a multiple of 8)
    auto load_batch = [&](v4f (&w)[UR], int i) {
#pragma unroll
        for (int u = 0; u < UR; u++) {
            const int k = min(kb + r0 + i + u, K - 1);
            const float *src = W + (long)k * ldw + colc;
            if (VEC) {
                w[u] = *reinterpret_cast<const v4f *>(src);
            } else {
                w[u] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (col + j < N) w[u][j] = src[j];
            }
        }
    };
    // the first weight batch is in flight while the activations are staged,
    // and so are the bias and old output of this thread's first output
    v4f wn[UR];
    load_batch(wn, 0);
    const int pn = n0 + tid % CW;
    const bool pown = splits == 1 && tid < M * CW && pn < N;
    const float pbias = pown && bias ? bias[pn] : 0.f;
    const float pold = pown && accumulate ? Y[(long)(tid / CW) * ldy + pn] : 0.f;

    if (!XONES) {
        stage_rows<MR, false>(xs, kchunk, kchunk, min(kchunk, K - kb), M, X + kb, ldx);
        __syncthreads();
    }

    float acc[MR][4];
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[m][j] = 0.f;

    for (int i = 0; i < run; i += UR) {
        v4f w[UR];
#pragma unroll
        for (int u = 0; u < UR; u++) w[u] = wn[u];
        if (i + UR < run) load_batch(wn, i + UR);
#pragma unroll
        for (int u = 0; u < UR; u++) {
            if (kb + r0 + i + u < K) {
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const float xv = XONES ? 1.f : xs[m * kchunk + r0 + i + u];
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[m][j] += xv * w[u][j];
                }
            }
        }
    }

#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int j = 0; j < 4; j++) red[rg][m][4 * c4 + j] = acc[m][j];
    __syncthreads();

    const int nround = gridDim.x * CW;
    for (int o = tid; o < M * CW; o += GV_THREADS) {
        const int m = o / CW, c = o % CW, n = n0 + c;
        float s = 0.f;
#pragma unroll 16
        for (int r = 0; r < RG; r++) s += red[r][m][c];
        if (splits == 1) {
            if (n < N) {
                float y = s + (o == tid ? pbias : (bias ? bias[n] : 0.f));
                float *dst = Y + (long)m * ldy + n;
                *dst = accumulate ? (o == tid ? pold : *dst) + y : y;
            }
        } else {
            part[((long)sp * M + m) * nround + n] = s;
        }
    }
}

// ------------------------------------------------------------- sgemv_t ----
// Block = SGT_ROWS rows of W (N x K) x kchunk columns. Thread (j = tid%16,
// rs = tid/16) reads 16-byte vectors k = 4j + 64i of rows rs + 16r.
template <int MR, bool VEC, int XF = XF_NONE>
__global__ __launch_bounds__(GV_THREADS) void sgemv_t_kernel(
    const float *__restrict__ X, long ldx, const float *__restrict__ W, long ldw,
    const float *__restrict__ bias, float *__restrict__ Y, long ldy, int M, int N, int K,
    int kchunk, int splits, float *__restrict__ part, int accumulate,
    const float *__restrict__ xg = nullptr, const float *__restrict__ xb = nullptr) {
    __shared__ float res[MR][SGT_ROWS];
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_dyn[];
    float *xs = reinterpret_cast<float *>(gv_dyn);  // MR x kchunk, sized at launch

    const int tid = threadIdx.x;
    const int j = tid & 15, rs = tid >> 4;
    const int strip = blockIdx.x, sp = blockIdx.y;
    const int n0 = strip * SGT_ROWS;
    const int kb = sp * kchunk;
    const int klen = min(kchunk, K - kb);

    // rows past N are clamped (their sums are never stored); k past klen is
    // clamped for the load and skipped in the arithmetic (klen >= 1: the
    // host never launches K == 0)
    const float *wrow[SGT_RPL];
#pragma unroll
    for (int r = 0; r < SGT_RPL; r++) wrow[r] = W + (long)min(n0 + rs + 16 * r, N - 1) * ldw + kb;
    constexpr int UK = 4;  // 64-element k steps per load batch
    // weight rows are streamed once per call: non-temporal loads (5.5 against
    // 4.8-5.0 TB/s on the 206 MB tied head)
    auto load_batch = [&](v4f (&w)[UK][SGT_RPL], int k0) {
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < SGT_RPL; r++) {
                const int k = k0 + 64 * u;
                if (VEC) {
                    w[u][r] = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(wrow[r] + min(k, klen - 4)));
                } else {
                    w[u][r] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (k + e < klen) w[u][r][e] = wrow[r][k + e];
                }
            }
    };
    // the first weight batch is in flight while the activations are staged,
    // and so are the bias and old output of this thread's output (one per
    // thread: M * SGT_ROWS <= 256)
    v4f wn[UK][SGT_RPL];
    load_batch(wn, 4 * j);
    const int pn = n0 + tid % SGT_ROWS;
    const bool pown = splits == 1 && tid < M * SGT_ROWS && pn < N;
    const float pbias = pown && bias ? bias[pn] : 0.f;
    const float pold = pown && accumulate ? Y[(long)(tid / SGT_ROWS) * ldy + pn] : 0.f;

    stage_rows<MR, false>(xs, kchunk, kchunk, klen, M, X + kb, ldx);
    __syncthreads();
    if constexpr (XF != XF_NONE) gv_xform<XF>(xs, klen, kb, K, X, xg, xb);

    float acc[SGT_RPL][MR];
#pragma unroll
    for (int r = 0; r < SGT_RPL; r++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r][m] = 0.f;

    for (int k0 = 4 * j; k0 < klen; k0 += 64 * UK) {
        v4f w[UK][SGT_RPL];
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < SGT_RPL; r++) w[u][r] = wn[u][r];
        if (k0 + 64 * UK < klen) load_batch(wn, k0 + 64 * UK);
#pragma unroll
        for (int u = 0; u < UK; u++) {
            const int k = k0 + 64 * u;
            if (k < klen) {
                v4f xv[MR];
#pragma unroll
                for (int m = 0; m < MR; m++) xv[m] = *reinterpret_cast<const v4f *>(&xs[m * kchunk + k]);
#pragma unroll
                for (int r = 0; r < SGT_RPL; r++)
#pragma unroll
                    for (int m = 0; m < MR; m++)
                        acc[r][m] += xv[m][0] * w[u][r][0] + xv[m][1] * w[u][r][1] +
                                     xv[m][2] * w[u][r][2] + xv[m][3] * w[u][r][3];
            }
        }
    }

    // reduce over the 16 lanes of each row group (DPP, into the group's last lane)
#pragma unroll
    for (int r = 0; r < SGT_RPL; r++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r][m] = dpp_sum_last<16>(acc[r][m]);
    if (j == 15) {
#pragma unroll
        for (int r = 0; r < SGT_RPL; r++)
#pragma unroll
            for (int m = 0; m < MR; m++) res[m][rs + 16 * r] = acc[r][m];
    }
    __syncthreads();

    const int nround = gridDim.x * SGT_ROWS;
    for (int o = tid; o < M * SGT_ROWS; o += GV_THREADS) {
        const int m = o / SGT_ROWS, c = o % SGT_ROWS, n = n0 + c;
        const float s = res[m][c];
        if (splits == 1) {
            if (n < N) {
                const float y = s + pbias;
                float *dst = Y + (long)m * ldy + n;
                *dst = accumulate ? pold + y : y;
            }
        } else {
            part[((long)sp * M + m) * nround + n] = s;
        }
    }
}

// --------------------------------------------------------------- igemv ----
// Same geometry as sgemv_t over bytes: thread reads 16 weight bytes
// (k = 16j + 256i) of rows rs + 16r; activations are staged re-centred
// (x ^ 0x80 = x - 128) so v_dot4_i32_i8 accumulates sum (x-128)*w exactly.
__device__ __forceinline__ int32_t epi_int(int32_t v, const int32_t *col_off, int n) {
    return col_off ? (int32_t)((unsigned)v + (unsigned)gbl(col_off)[n]) : v;
}

template <int OUT>
__device__ __forceinline__ void igemv_write(void *Yv, long ldy, int m, int n, int32_t v,
                                            const int32_t *col_off, const float *sa,
                                            const float *sb) {
    v = epi_int(v, col_off, n);
    if (OUT == 0) {
        gbl(reinterpret_cast<int32_t *>(Yv))[(long)m * ldy + n] = v;
    } else {
        const float dq = (OUT == 2) ? gbl(sa)[m] * gbl(sb)[n] : gbl(sb)[n];
        gbl(reinterpret_cast<float *>(Yv))[(long)m * ldy + n] = (float)v * dq;
    }
}

// Outputs n .. n+3 of row m (n + 3 < N) in one 16-byte store, each value as
// igemv_write gives it. The store is only 4-byte aligned when ldy is not a
// multiple of 4 (a vocabulary-wide logits row); global accesses on this target
// may be unaligned, and the compiler still emits one dwordx4 store.
template <int OUT>
__device__ __forceinline__ void igemv_write4(void *Yv, long ldy, int m, int n, v4i v,
                                             const int32_t *col_off, const float *sa,
                                             const float *sb) {
    typedef int32_t v4i_u __attribute__((ext_vector_type(4), aligned(4)));
    typedef float v4f_u __attribute__((ext_vector_type(4), aligned(4)));
    v4i_u r;
#pragma unroll
    for (int e = 0; e < 4; e++) r[e] = epi_int(v[e], col_off, n + e);
    if (OUT == 0) {
        *reinterpret_cast<__attribute__((address_space(1))) v4i_u *>(
            gbl(reinterpret_cast<int32_t *>(Yv)) + (long)m * ldy + n) = r;
    } else {
        v4f_u f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float dq = (OUT == 2) ? gbl(sa)[m] * gbl(sb)[n + e] : gbl(sb)[n + e];
            f[e] = (float)r[e] * dq;
        }
        *reinterpret_cast<__attribute__((address_space(1))) v4f_u *>(
            gbl(reinterpret_cast<float *>(Yv)) + (long)m * ldy + n) = f;
    }
}

// Second pass of a split-K INT8 GEMV: exact int32 sum of the splits, then the
// epilogue of the single-pass kernel.
template <int OUT>
__global__ void igemv_reduce_kernel(const int32_t *__restrict__ part, int splits, int M, int N,
                                    int nround, const int32_t *__restrict__ col_off,
                                    const float *__restrict__ sa, const float *__restrict__ sb,
                                    void *__restrict__ Yv, long ldy) {
    const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i >= (long)M * N) return;
    const int m = (int)(i / N), n = (int)(i % N);
    unsigned s = 0;
    for (int q = 0; q < splits; q++) s += (unsigned)part[((long)q * M + m) * nround + n];
    igemv_write<OUT>(Yv, ldy, m, n, (int32_t)s, col_off, sa, sb);
}

template <int MR, int OUT>
__global__ __launch_bounds__(GV_THREADS) void igemv_kernel(
    const uint8_t *__restrict__ X, long ldx, const int8_t *__restrict__ B, long ldb,
    const int32_t *__restrict__ col_off, const float *__restrict__ sa,
    const float *__restrict__ sb, void *__restrict__ Yv, long ldy, int M, int N, int K,
    int kchunk, int splits, int32_t *__restrict__ part) {
    __shared__ int32_t res[MR][SGT_ROWS];
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_dyn[];
    int8_t *xs = reinterpret_cast<int8_t *>(gv_dyn);  // MR x kchunk, sized at launch

    const int tid = threadIdx.x;
    const int j = tid & 15, rs = tid >> 4;
    const int strip = blockIdx.x, sp = blockIdx.y;
    const int n0 = strip * SGT_ROWS;
    const int kb = sp * kchunk;
    // bytes of this split inside the packed rows (ldb >= roundup(K,16), zero pad)
    const int kend = min(kb + kchunk, (K + 15) & ~15);
    const int klen = kend - kb;

    // rows past N are clamped (never stored); k past klen is clamped for the
    // load and skipped in the arithmetic (klen >= 16: the host never launches
    // K == 0)
    const int8_t *brow[SGT_RPL];
#pragma unroll
    for (int r = 0; r < SGT_RPL; r++) brow[r] = B + (long)min(n0 + rs + 16 * r, N - 1) * ldb + kb;
    // 256-byte k steps per load batch; with 4-8 rows of X a batch's dot
    // products take long enough that half-size batches overlap better
    constexpr int UK = MR >= 4 ? 2 : 4;
    auto load_batch = [&](v4i (&w)[UK][SGT_RPL], int k0) {
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < SGT_RPL; r++)
                w[u][r] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(brow[r] + min(k0 + 256 * u, klen - 16)));
    };
    // the first weight batch is in flight while the activations are staged,
    // and so are the epilogue operands of this thread's output (o = tid, one
    // per thread: M * SGT_ROWS <= 256), so the block's life holds one memory
    // latency rather than two
    v4i wn[UK][SGT_RPL];
    load_batch(wn, 16 * j);
    const int om = tid / SGT_ROWS, on = min(n0 + tid % SGT_ROWS, N - 1);
    const bool owns = splits == 1 && tid < M * SGT_ROWS;
    const float dq_pre = (OUT == 0 || !owns) ? 0.f
                         : (OUT == 2 ? gbl(sa)[om] * gbl(sb)[on] : gbl(sb)[on]);
    const unsigned off_pre = (owns && col_off) ? (unsigned)gbl(col_off)[on] : 0u;

    stage_rows<MR, true>(reinterpret_cast<uint8_t *>(xs), kchunk, kchunk, min(kchunk, K - kb), M,
                         X + kb, ldx);
    __syncthreads();

    int32_t acc[SGT_RPL][MR];
#pragma unroll
    for (int r = 0; r < SGT_RPL; r++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r][m] = 0;

    for (int k0 = 16 * j; k0 < klen; k0 += 256 * UK) {
        v4i w[UK][SGT_RPL];
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < SGT_RPL; r++) w[u][r] = wn[u][r];
        if (k0 + 256 * UK < klen) load_batch(wn, k0 + 256 * UK);
#pragma unroll
        for (int u = 0; u < UK; u++) {
            const int k = k0 + 256 * u;
            if (k < klen) {
                v4i xv[MR];
#pragma unroll
                for (int m = 0; m < MR; m++) xv[m] = *reinterpret_cast<const v4i *>(&xs[m * kchunk + k]);
#pragma unroll
                for (int r = 0; r < SGT_RPL; r++)
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        int a = acc[r][m];
                        a = __builtin_amdgcn_sdot4(xv[m][0], w[u][r][0], a, false);
                        a = __builtin_amdgcn_sdot4(xv[m][1], w[u][r][1], a, false);
                        a = __builtin_amdgcn_sdot4(xv[m][2], w[u][r][2], a, false);
                        a = __builtin_amdgcn_sdot4(xv[m][3], w[u][r][3], a, false);
                        acc[r][m] = a;
                    }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < SGT_RPL; r++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r][m] = dpp_sum_last<16>(acc[r][m]);  // exact in any order
    if (j == 15) {
#pragma unroll
        for (int r = 0; r < SGT_RPL; r++)
#pragma unroll
            for (int m = 0; m < MR; m++) res[m][rs + 16 * r] = acc[r][m];
    }
    __syncthreads();

    const int nround = gridDim.x * SGT_ROWS;
    if (tid < M * SGT_ROWS) {
        const int m = tid / SGT_ROWS, c = tid % SGT_ROWS, n = n0 + c;
        if (splits == 1) {
            // igemv_write with the operands loaded at the start
            if (n < N) {
                const int32_t v = (int32_t)((unsigned)res[m][c] + off_pre);
                if (OUT == 0) gbl(reinterpret_cast<int32_t *>(Yv))[(long)m * ldy + n] = v;
                else gbl(reinterpret_cast<float *>(Yv))[(long)m * ldy + n] = (float)v * dq_pre;
            }
        } else {
            part[((long)sp * M + m) * nround + n] = res[m][c];
        }
    }
}

// ------------------------------------------------------------- planning ----
static int mr_of(int M) { return M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8)); }

// strips: blocks along N; want: blocks wanted in all; kstep: K granularity
// of a split; kmin: least K per split worth a second kernel; kmax: most K a
// block can stage.
static GemvPlan make_plan(int strips, int want, int M, int K, int kstep, int kmin, int kmax,
                          int rows_per_strip) {
    GemvPlan p;
    p.strips = strips;
    int splits = cdiv(want, strips > 0 ? strips : 1);
    int most = cdiv(K, kmin);
    if (splits > most) splits = most;
    if (splits < cdiv(K, kmax)) splits = cdiv(K, kmax);  // staging limit
    if (splits < 1) splits = 1;
    int kchunk = cdiv(cdiv(K, splits), kstep) * kstep;
    if (kchunk > kmax) kchunk = kmax;
    if (kchunk < kstep) kchunk = kstep;
    splits = K > 0 ? cdiv(K, kchunk) : 1;
    p.splits = splits;
    p.kchunk = kchunk;
    p.part_bytes = splits > 1 ? (size_t)splits * M * strips * rows_per_strip * 4 : 0;
    p.cw = rows_per_strip;
    return p;
}

// A GEMV launch costs ~3 us before any weight arrives, so a second (reduce)
// kernel only pays when a single pass would leave each thread several
// dependent load batches on a small grid. Weights of K x N (N-contiguous)
// take 16-column strips and stay unsplit up to K = 1024 (two 8-row batches
// per thread); deeper K splits into 512-row chunks (one batch each) until the
// grid has ~1024 blocks. Weights of N x K (K-contiguous rows: the tied head,
// INT8 packed rows) split only when the grid has under 256 blocks and a split
// still covers 1024 floats or 2048 bytes. bias_bwd (a K-deep column sum)
// keeps 64-column strips.
GemvPlan plan_sgemv(int w_trans, int M, int N, int K) {
    const int mr = mr_of(M);
    if (w_trans) return make_plan(cdiv(N, SGT_ROWS), 256, M, K, 64, 1024, 8192 / mr, SGT_ROWS);
    if (K <= 1024 && K <= 4096 / mr) return make_plan(cdiv(N, 16), 1, M, K, 512, 1 << 30, 4096 / mr, 16);
    return make_plan(cdiv(N, 16), GV_TARGET_BLOCKS, M, K, 512, 512, 4096 / mr, 16);
}

GemvPlan plan_bias_bwd(int N, int M) {
    return make_plan(cdiv(N, 64), GV_TARGET_BLOCKS, 1, M, 128, 128, 4096, 64);
}

GemvPlan plan_igemv(int M, int N, int K) {
    return make_plan(cdiv(N, SGT_ROWS), 256, M, K, 256, 2048, 16384 / mr_of(M), SGT_ROWS);
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int reduce_grid(int M, int N) { return cdiv((long)M * N, 256); }

template <int MR>
static void launch_sgemv_mr(const GemvPlan &p, int w_trans, bool vec, bool x_ones, int M, int N,
                            int K, const float *X, long ldx, const float *W, long ldw,
                            const float *bias, int accumulate, float *Y, long ldy,
                            const Workspace &ws, hipStream_t s) {
    dim3 grid(p.strips, p.splits), block(GV_THREADS);
    float *part = (float *)ws.buf;
    const size_t xsb = (size_t)MR * p.kchunk * sizeof(float);  // staged activation rows
    if (w_trans) {
        if (vec)
            hipLaunchKernelGGL((sgemv_t_kernel<MR, true>), grid, block, xsb, s, X, ldx, W, ldw, bias,
                               Y, ldy, M, N, K, p.kchunk, p.splits, part, accumulate);
        else
            hipLaunchKernelGGL((sgemv_t_kernel<MR, false>), grid, block, xsb, s, X, ldx, W, ldw, bias,
                               Y, ldy, M, N, K, p.kchunk, p.splits, part, accumulate);
    } else if (x_ones) {
        if (vec)
            hipLaunchKernelGGL((sgemv_n_kernel<1, true, true, 64>), grid, block, 0, s, X, ldx, W,
                               ldw, bias, Y, ldy, M, N, K, p.kchunk, p.splits, part, accumulate);
        else
            hipLaunchKernelGGL((sgemv_n_kernel<1, false, true, 64>), grid, block, 0, s, X, ldx, W,
                               ldw, bias, Y, ldy, M, N, K, p.kchunk, p.splits, part, accumulate);
    } else if (p.cw == 16) {
        if (vec)
            hipLaunchKernelGGL((sgemv_n_kernel<MR, true, false, 16>), grid, block, xsb, s, X, ldx, W,
                               ldw, bias, Y, ldy, M, N, K, p.kchunk, p.splits, part, accumulate);
        else
            hipLaunchKernelGGL((sgemv_n_kernel<MR, false, false, 16>), grid, block, xsb, s, X, ldx,
                               W, ldw, bias, Y, ldy, M, N, K, p.kchunk, p.splits, part, accumulate);
    } else {
        if (vec)
            hipLaunchKernelGGL((sgemv_n_kernel<MR, true, false, 64>), grid, block, xsb, s, X, ldx, W,
                               ldw, bias, Y, ldy, M, N, K, p.kchunk, p.splits, part, accumulate);
        else
            hipLaunchKernelGGL((sgemv_n_kernel<MR, false, false, 64>), grid, block, xsb, s, X, ldx,
                               W, ldw, bias, Y, ldy, M, N, K, p.kchunk, p.splits, part, accumulate);
    }
    if (p.splits > 1) {
        const int nround = p.strips * (w_trans ? SGT_ROWS : p.cw);
        hipLaunchKernelGGL(sgemv_reduce_kernel, dim3(reduce_grid(M, N)), dim3(256), 0, s, part,
                           p.splits, M, N, nround, bias, Y, ldy, accumulate);
    }
}

hipError_t launch_sgemv(const GemvPlan &p, int w_trans, int M, int N, int K, const float *X,
                        long ldx, bool x_ones, const float *W, long ldw, const float *bias,
                        int accumulate, float *Y, long ldy, const Workspace &ws,
                        hipStream_t stream) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (K <= 0) {  // Y = (accumulate ? Y : 0) + bias: the reduce pass over zero splits
        hipLaunchKernelGGL(sgemv_reduce_kernel, dim3(reduce_grid(M, N)), dim3(256), 0, stream,
                           nullptr, 0, M, N, N, bias, Y, ldy, accumulate);
        return hipGetLastError();
    }
    if (p.splits > 1 && (ws.buf == nullptr || ws.bytes_cap < p.part_bytes)) return hipErrorInvalidValue;
    bool vec = aligned16(W) && ldw % 4 == 0 && (w_trans ? K % 4 == 0 : N % 4 == 0);
    if (x_ones) {
        launch_sgemv_mr<1>(p, w_trans, vec, true, M, N, K, X, ldx, W, ldw, bias, accumulate, Y,
                           ldy, ws, stream);
    } else if (M == 1) {
        launch_sgemv_mr<1>(p, w_trans, vec, false, M, N, K, X, ldx, W, ldw, bias, accumulate, Y,
                           ldy, ws, stream);
    } else if (M <= 2) {
        launch_sgemv_mr<2>(p, w_trans, vec, false, M, N, K, X, ldx, W, ldw, bias, accumulate, Y,
                           ldy, ws, stream);
    } else if (M <= 4) {
        launch_sgemv_mr<4>(p, w_trans, vec, false, M, N, K, X, ldx, W, ldw, bias, accumulate, Y,
                           ldy, ws, stream);
    } else {
        launch_sgemv_mr<8>(p, w_trans, vec, false, M, N, K, X, ldx, W, ldw, bias, accumulate, Y,
                           ldy, ws, stream);
    }
    return hipGetLastError();
}

// One row (M = 1) with an input transform, over N x K weights (sgemv_t's
// plans and kernel).
template <int XF>
static void launch_sgemv_xf_t(const GemvPlan &p, bool vec, int N, int K, const float *X,
                              const float *W, long ldw, const float *g, const float *b,
                              const float *bias, int accumulate, float *Y, const Workspace &ws,
                              hipStream_t s) {
    dim3 grid(p.strips, p.splits), block(GV_THREADS);
    float *part = (float *)ws.buf;
    const size_t xsb = (size_t)p.kchunk * sizeof(float);
    const long ldx = K, ldy = N;
    if (vec)
        hipLaunchKernelGGL((sgemv_t_kernel<1, true, XF>), grid, block, xsb, s, X, ldx, W, ldw, bias, Y,
                           ldy, 1, N, K, p.kchunk, p.splits, part, accumulate, g, b);
    else
        hipLaunchKernelGGL((sgemv_t_kernel<1, false, XF>), grid, block, xsb, s, X, ldx, W, ldw, bias, Y,
                           ldy, 1, N, K, p.kchunk, p.splits, part, accumulate, g, b);
    if (p.splits > 1)
        hipLaunchKernelGGL(sgemv_reduce_kernel, dim3(reduce_grid(1, N)), dim3(256), 0, s, part,
                           p.splits, 1, N, p.strips * SGT_ROWS, bias, Y, ldy, accumulate);
}

hipError_t launch_sgemv_xf(const GemvPlan &p, int xf, int N, int K, const float *X,
                           const float *W, long ldw, const float *g, const float *b,
                           const float *bias, int accumulate, float *Y, const Workspace &ws,
                           hipStream_t stream) {
    if (N <= 0 || K <= 0) return hipErrorInvalidValue;
    if (xf == XF_LN && (!g || !b)) return hipErrorInvalidValue;
    if (p.splits > 1 && (ws.buf == nullptr || ws.bytes_cap < p.part_bytes)) return hipErrorInvalidValue;
    const bool vec = aligned16(W) && ldw % 4 == 0 && K % 4 == 0;
    if (xf == XF_LN)
        launch_sgemv_xf_t<XF_LN>(p, vec, N, K, X, W, ldw, g, b, bias, accumulate, Y, ws, stream);
    else if (xf == XF_GELU)
        launch_sgemv_xf_t<XF_GELU>(p, vec, N, K, X, W, ldw, g, b, bias, accumulate, Y, ws, stream);
    else
        launch_sgemv_xf_t<XF_NONE>(p, vec, N, K, X, W, ldw, g, b, bias, accumulate, Y, ws, stream);
    return hipGetLastError();
}

// ---------------------------------------------------- decode INT8 row ----
// One fp32 activation row through an input transform, quantised per row in
// LDS (the rule of quant.hip: amax from 1e-8, scale = amax * fl(1/127),
// q = clamp(roundf(x / scale)), padding past K is 0 after recentring), times
// the packed s8 weights (N rows of Kp bytes), dequantised by scale * sb[n]:
//   QX_NONE: the row as is; QX_LN: LayerNorm (g, b; two passes, mean then
//   the mean square of the deviations); QX_BIAS_GELU: tanh-GELU(x + b).
//   EPI 0: Y[n] = v * dq;  EPI 1: Y[n] = Y[n] + (v * dq + bias[n]).
// Every block computes the same row, scale and bytes. No K split.
constexpr int QX_NONE = 0, QX_LN = 1, QX_BIAS_GELU = 2;

__device__ __forceinline__ float gv_sum4(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// The input transform of the decode rows. A thread owns elements tid + 256 e;
// the transform's per-element vectors of its first QPF elements are loaded
// into registers up front (qx_prefetch), the rest when they are used.
constexpr int QPF = 8;

template <int QX>
__device__ __forceinline__ void qx_prefetch(const float *__restrict__ g, const float *__restrict__ b, int K,
                                            float (&gpf)[QPF], float (&bpf)[QPF]) {
#pragma unroll
    for (int e = 0; e < QPF; e++) {
        const int i = (int)threadIdx.x + 256 * e;
        gpf[e] = QX == QX_LN && i < K ? g[i] : 0.f;
        bpf[e] = QX != QX_NONE && i < K ? b[i] : 0.f;
    }
}

__device__ __forceinline__ float qx_gelu(float v) {
    return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
}

// xf[0..K) = transform(X): QX_LN LayerNorm (mean, then the mean square of the
// deviations, each a sum over the thread's elements in order and then over the
// four waves; (x - mu) * rsd * g + b), QX_BIAS_GELU tanh-GELU(x + b), QX_NONE
// x. The row is read once into LDS; each thread revisits only its own
// elements. Ends with the block's barrier.
template <int QX>
__device__ __forceinline__ void qx_row(const float *__restrict__ X, const float *__restrict__ g,
                                       const float *__restrict__ b, int K, const float (&gpf)[QPF],
                                       const float (&bpf)[QPF], float *xf, float *red) {
    const int tid = threadIdx.x;
    if constexpr (QX == QX_LN) {
        float s0 = 0.f;
        for (int i = tid; i < K; i += 256) {
            const float v = X[i];
            xf[i] = v;
            s0 += v;
        }
        const float mu = gv_sum4(s0, red) / K;
        float q = 0.f;
        for (int i = tid; i < K; i += 256) {
            const float d = xf[i] - mu;
            q += d * d;
        }
        const float var = gv_sum4(q, red) / K;
        const float rsd = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
        for (int e = 0; e < QPF; e++) {
            const int i = tid + 256 * e;
            if (i < K) xf[i] = (xf[i] - mu) * rsd * gpf[e] + bpf[e];
        }
        for (int i = tid + 256 * QPF; i < K; i += 256) xf[i] = (xf[i] - mu) * rsd * g[i] + b[i];
    } else if constexpr (QX == QX_BIAS_GELU) {
#pragma unroll
        for (int e = 0; e < QPF; e++) {
            const int i = tid + 256 * e;
            if (i < K) xf[i] = qx_gelu(X[i] + bpf[e]);
        }
        for (int i = tid + 256 * QPF; i < K; i += 256) xf[i] = qx_gelu(X[i] + b[i]);
    } else {
        for (int i = tid; i < K; i += 256) xf[i] = X[i];
    }
    __syncthreads();
}

// Sum over the block of one value per thread: each wave's total (DPP, in its
// last lane), then the four waves in order, into a red[4] used once per
// launch (no barrier before the writes).
__device__ __forceinline__ float gv_sum4_once(float v, float *red) {
    v = dpp_sum_last<64>(v);
    if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// Two block sums in one barrier: a and b on the DPP network (two independent
// chains), lane 63 of wave w leaves them in red[w] and red[4 + w].
__device__ __forceinline__ void gv_sum4x2_once(float &a, float &b, float *red) {
    a = dpp_sum_last<64>(a);
    b = dpp_sum_last<64>(b);
    if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = a, red[4 + (threadIdx.x >> 6)] = b;
    __syncthreads();
    a = red[0] + red[1] + red[2] + red[3];
    b = red[4] + red[5] + red[6] + red[7];
}

// qx_row for rows of at most 256 * QPF elements, kept in registers: v[e] =
// transform(X)[tid + 256 e] (0 past K). The same per-thread partial sums as
// qx_row; a wave's partials are added on the DPP network (another
// association than qx_row's shuffles, so LayerNorm statistics may differ in
// the last bit); no LDS round trips, one barrier per LayerNorm sum. red: 8
// floats, each half used once.
template <int QX>
__device__ __forceinline__ void qx_regs(const float *__restrict__ X, int K, const float (&gpf)[QPF],
                                        const float (&bpf)[QPF], float (&v)[QPF], float *red) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int e = 0; e < QPF; e++) {
        const int i = tid + 256 * e;
        v[e] = i < K ? X[i] : 0.f;
    }
    if constexpr (QX == QX_LN) {
        // mean and variance from one reduction, shifted by the row's first
        // element (so the difference of the two sums does not cancel when the
        // mean is large against the spread): with d = x - x0,
        // mu = x0 + sum(d) / K, var = sum(d^2) / K - (sum(d) / K)^2
        const float x0 = X[0];
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int e = 0; e < QPF; e++) {
            if (tid + 256 * e < K) {
                const float d = v[e] - x0;
                s0 += d;
                s1 += d * d;
            }
        }
        gv_sum4x2_once(s0, s1, red);
        const float dm = s0 / K, mu = x0 + dm;
        const float var = fmaxf(s1 / K - dm * dm, 0.f);
        const float rsd = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
        for (int e = 0; e < QPF; e++)
            if (tid + 256 * e < K) v[e] = (v[e] - mu) * rsd * gpf[e] + bpf[e];
    } else if constexpr (QX == QX_BIAS_GELU) {
#pragma unroll
        for (int e = 0; e < QPF; e++)
            if (tid + 256 * e < K) v[e] = qx_gelu(v[e] + bpf[e]);
    }
}

// Thread layout: LPR lanes per weight row (16-byte pieces k = 16*lane +
// 16*LPR*u), 256/LPR row groups of RPL = 2 rows: RPB = 512/LPR rows per block,
// so shallow products spread over more blocks; UK 16-byte loads per row per
// batch, chosen so a batch spans the whole row when it is short.
template <int QX, int EPI, int LPR, int UK>
__global__ __launch_bounds__(GV_THREADS) void igemv_q_kernel(
    const float *__restrict__ X, const float *__restrict__ g, const float *__restrict__ b, int K,
    const int8_t *__restrict__ B, long ldb, const float *__restrict__ sb,
    const float *__restrict__ bias, float *__restrict__ Y, int N, GemvTap tap) {
    static_assert(GV_THREADS == 256, "the reductions assume four waves");
    constexpr int RPL = 2, RG = GV_THREADS / LPR, RPB = RG * RPL;
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_dyn[];
    const int Kp = (int)ldb;
    float *xf = reinterpret_cast<float *>(gv_dyn);          // [Kp]
    int8_t *xs = reinterpret_cast<int8_t *>(xf + Kp);        // [Kp]
    __shared__ float red[4], mred[4], red8[8];
    __shared__ int32_t res[RPB];

    const int tid = threadIdx.x;
    const int j = tid % LPR, rs = tid / LPR;
    const int n0 = blockIdx.x * RPB;
    const int klen = min(Kp, (K + 15) & ~15);
    const int8_t *brow[RPL];
#pragma unroll
    for (int r = 0; r < RPL; r++) brow[r] = B + (long)min(n0 + rs + RG * r, N - 1) * ldb;
    auto load_batch = [&](v4i (&w)[UK][RPL], int k0) {
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < RPL; r++)
                w[u][r] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(brow[r] + min(k0 + 16 * LPR * u, klen - 16)));
    };
    v4i wn[UK][RPL];
    load_batch(wn, 16 * j);  // in flight while the row is made
    // what does not depend on the row loads with the weights, so the block's
    // chain holds one dependent global read (the row) instead of three: the
    // transform's vectors for a thread's first QPF elements, the epilogue's
    // scale, bias and residual of output n0 + tid
    float gpf[QPF], bpf[QPF];
    qx_prefetch<QX>(g, b, K, gpf, bpf);
    float esb = 0.f, ebias = 0.f, ey = 0.f;
    if (tid < RPB && n0 + tid < N) {
        esb = sb[n0 + tid];
        if (EPI == 1) ebias = bias[n0 + tid], ey = Y[n0 + tid];
    }
    // rows of at most 256 * QPF bytes (Kp <= 256 * QPF) stay in registers
    // from the load to the quantised bytes; longer rows go through LDS
    const bool regs = Kp <= 256 * QPF;
    float v[QPF];
    float mx = 0.f;
    if (regs) {
        qx_regs<QX>(X, K, gpf, bpf, v, red8);
#pragma unroll
        for (int e = 0; e < QPF; e++)
            if (tid + 256 * e < K) mx = fmaxf(mx, fabsf(v[e]));
    } else {
        qx_row<QX>(X, g, b, K, gpf, bpf, xf, red);
        for (int i = tid; i < K; i += 256) mx = fmaxf(mx, fabsf(xf[i]));
    }
    mx = dpp_max_last64(mx);
    if ((tid & 63) == 63) mred[tid >> 6] = mx;
    __syncthreads();
    const float amax = fmaxf(fmaxf(fmaxf(mred[0], mred[1]), fmaxf(mred[2], mred[3])), AMAX_INIT);
    const float scale = amax * RCP127, inv = 1.0f / scale;
    if (regs) {
#pragma unroll
        for (int e = 0; e < QPF; e++) {
            const int k = tid + 256 * e;
            if (k < Kp) xs[k] = (int8_t)(k < K ? quant_q(v[e], inv) : 0);
        }
    } else {
        for (int k = tid; k < Kp; k += 256) xs[k] = (int8_t)(k < K ? quant_q(xf[k], inv) : 0);
    }
    __syncthreads();
    if (tap.xq && blockIdx.x == 0) {  // every block makes the same row; block 0 records it
        for (int k = tid; k < Kp; k += 256) tap.xq[k] = (uint8_t)(xs[k] + 128);
        if (tid == 0) tap.sa[0] = scale;
    }

    int32_t acc[RPL] = {};
    for (int k0 = 16 * j; k0 < klen; k0 += 16 * LPR * UK) {
        v4i w[UK][RPL];
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < RPL; r++) w[u][r] = wn[u][r];
        if (k0 + 16 * LPR * UK < klen) load_batch(wn, k0 + 16 * LPR * UK);
#pragma unroll
        for (int u = 0; u < UK; u++) {
            const int k = k0 + 16 * LPR * u;
            if (k < klen) {
                const v4i xv = *reinterpret_cast<const v4i *>(&xs[k]);
#pragma unroll
                for (int r = 0; r < RPL; r++) {
                    int a = acc[r];
                    a = __builtin_amdgcn_sdot4(xv[0], w[u][r][0], a, false);
                    a = __builtin_amdgcn_sdot4(xv[1], w[u][r][1], a, false);
                    a = __builtin_amdgcn_sdot4(xv[2], w[u][r][2], a, false);
                    a = __builtin_amdgcn_sdot4(xv[3], w[u][r][3], a, false);
                    acc[r] = a;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPL; r++) {  // the row's LPR lanes, exact in any order
        const int v = dpp_sum_last<LPR>(acc[r]);
        if (j == LPR - 1) res[rs + RG * r] = v;
    }
    __syncthreads();
    if (tid < RPB) {
        const int n = n0 + tid;
        if (n < N) {
            const float dq = scale * esb;
            const float y = (float)res[tid] * dq;
            if (tap.y) tap.y[n] = y;
            if (EPI == 1) Y[n] = ey + (y + ebias);
            else Y[n] = y;
        }
    }
}

template <int QX, int EPI>
static void launch_igemv_q_shape(const float *X, const float *g, const float *b, int K,
                                 const int8_t *B, int Kp, const float *sb, const float *bias,
                                 float *Y, int N, hipStream_t s, const GemvTap &tap) {
    const size_t lds = (size_t)Kp * (sizeof(float) + 1);
    const dim3 block(GV_THREADS);
#define IGQ(LPRV, UKV)                                                                       \
    hipLaunchKernelGGL((igemv_q_kernel<QX, EPI, LPRV, UKV>), dim3((unsigned)cdiv(N, 512 / LPRV)), \
                       block, lds, s, X, g, b, K, B, (long)Kp, sb, bias, Y, N, tap)
    if (Kp <= 256) IGQ(16, 1);
    else if (Kp <= 512) IGQ(32, 1);
    else if (Kp <= 1024) IGQ(64, 1);
    else if (Kp <= 2048) IGQ(64, 2);
    else IGQ(64, 4);
#undef IGQ
}

hipError_t launch_igemv_q(int qx, int epi, const float *X, const float *g, const float *b, int K,
                          const int8_t *B, int Kp, const float *sb, const float *bias, float *Y,
                          int N, hipStream_t s, const GemvTap &tap) {
    if (N <= 0 || K <= 0 || K > Kp || Kp % 256 != 0 || Kp > IGEMV_Q_MAX_K) return hipErrorInvalidValue;
    if ((tap.xq != nullptr) != (tap.sa != nullptr)) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(B) & 15) != 0) return hipErrorInvalidValue;
    if ((qx == QX_LN && (!g || !b)) || (qx == QX_BIAS_GELU && !b) || (epi == 1 && !bias))
        return hipErrorInvalidValue;
    if (qx == QX_LN) {
        if (epi) launch_igemv_q_shape<QX_LN, 1>(X, g, b, K, B, Kp, sb, bias, Y, N, s, tap);
        else launch_igemv_q_shape<QX_LN, 0>(X, g, b, K, B, Kp, sb, bias, Y, N, s, tap);
    } else if (qx == QX_BIAS_GELU) {
        if (epi) launch_igemv_q_shape<QX_BIAS_GELU, 1>(X, g, b, K, B, Kp, sb, bias, Y, N, s, tap);
        else launch_igemv_q_shape<QX_BIAS_GELU, 0>(X, g, b, K, B, Kp, sb, bias, Y, N, s, tap);
    } else {
        if (epi) launch_igemv_q_shape<QX_NONE, 1>(X, g, b, K, B, Kp, sb, bias, Y, N, s, tap);
        else launch_igemv_q_shape<QX_NONE, 0>(X, g, b, K, B, Kp, sb, bias, Y, N, s, tap);
    }
    return hipGetLastError();
}

// ------------------------------------------------------ decode fp32 row ----
// The fp32 twin of igemv_q_kernel: one activation row through the same input
// transform (staged in LDS), times fp32 weights stored N x K (a row per output,
// 16-byte loads along K), + bias; EPI 0: Y[n] = s + bias[n]; EPI 1: Y[n] =
// Y[n] + (s + bias[n]). LPR lanes per weight row, RPL = 2 rows per lane group.
template <int QX, int EPI, int LPR, int UK>
__global__ __launch_bounds__(GV_THREADS) void sgemv_q_kernel(
    const float *__restrict__ X, const float *__restrict__ g, const float *__restrict__ b, int K,
    const float *__restrict__ W, long ldw, const float *__restrict__ bias, float *__restrict__ Y,
    int N) {
    static_assert(GV_THREADS == 256, "the reductions assume four waves");
    // LPR 128 / 256: a row spans two / four waves (the products with few rows
    // spread over more workgroups); the wave sums are added through LDS in wave order
    static_assert(LPR == 16 || LPR == 32 || LPR == 64 || LPR == 128 || LPR == 256, "lanes per row");
    constexpr int RPL = 2, RG = GV_THREADS / LPR, RPB = RG * RPL, LW = LPR < 64 ? LPR : 64;
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_dyn[];
    float *xf = reinterpret_cast<float *>(gv_dyn);  // [K]
    __shared__ float red[4], red8[8], res[RPB], wsum[LPR > 64 ? 4 : 1][RPL];

    const int tid = threadIdx.x;
    const int j = tid % LPR, rs = tid / LPR;
    const int n0 = blockIdx.x * RPB;
    const float *wrow[RPL];
#pragma unroll
    for (int r = 0; r < RPL; r++) wrow[r] = W + (long)min(n0 + rs + RG * r, N - 1) * ldw;
    auto load_batch = [&](v4f (&w)[UK][RPL], int k0) {
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < RPL; r++)
                w[u][r] = *reinterpret_cast<const v4f *>(wrow[r] + min(k0 + 4 * LPR * u, K - 4));
    };
    v4f wn[UK][RPL];
    load_batch(wn, 4 * j);  // in flight while the row is made
    // loaded with the weights: the transform's vectors, the epilogue's bias
    // and residual (one dependent global read in the block's chain, the row)
    float gpf[QPF], bpf[QPF];
    qx_prefetch<QX>(g, b, K, gpf, bpf);
    float ebias = 0.f, ey = 0.f;
    if (tid < RPB && n0 + tid < N) {
        if (bias) ebias = bias[n0 + tid];
        if (EPI == 1) ey = Y[n0 + tid];
    }
    if (K <= 256 * QPF) {
        float v[QPF];
        qx_regs<QX>(X, K, gpf, bpf, v, red8);
#pragma unroll
        for (int e = 0; e < QPF; e++)
            if (tid + 256 * e < K) xf[tid + 256 * e] = v[e];
        __syncthreads();
    } else {
        qx_row<QX>(X, g, b, K, gpf, bpf, xf, red);
    }

    float acc[RPL] = {};
    for (int k0 = 4 * j; k0 < K; k0 += 4 * LPR * UK) {
        v4f w[UK][RPL];
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < RPL; r++) w[u][r] = wn[u][r];
        if (k0 + 4 * LPR * UK < K) load_batch(wn, k0 + 4 * LPR * UK);
#pragma unroll
        for (int u = 0; u < UK; u++) {
            const int k = k0 + 4 * LPR * u;
            if (k < K) {
                const v4f xv = *reinterpret_cast<const v4f *>(&xf[k]);
#pragma unroll
                for (int r = 0; r < RPL; r++)
                    acc[r] += xv[0] * w[u][r][0] + xv[1] * w[u][r][1] + xv[2] * w[u][r][2] +
                              xv[3] * w[u][r][3];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPL; r++) {
        const float v = dpp_sum_last<LW>(acc[r]);
        if constexpr (LPR > 64) {
            if ((tid & 63) == 63) wsum[tid >> 6][r] = v;
        } else {
            if (j == LW - 1) res[rs + RG * r] = v;
        }
    }
    if constexpr (LPR > 64) {
        // row rs + RG*r of the block: waves rs*(LPR/64) .. +LPR/64-1, added in order
        __syncthreads();
        if (tid < RPB) {
            const int g0 = tid % RG, r = tid / RG;
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < LPR / 64; w++) v += wsum[g0 * (LPR / 64) + w][r];
            res[tid] = v;
        }
    }
    __syncthreads();
    if (tid < RPB) {
        const int n = n0 + tid;
        if (n < N) {
            const float y = res[tid] + ebias;
            if (EPI == 1) Y[n] = ey + y;
            else Y[n] = y;
        }
    }
}

template <int QX, int EPI>
static void launch_sgemv_q_shape(const float *X, const float *g, const float *b, int K,
                                 const float *W, const float *bias, float *Y, int N, hipStream_t s) {
    const size_t lds = (size_t)K * sizeof(float);
    const dim3 block(GV_THREADS);
#define SGQ(LPRV, UKV)                                                                       \
    hipLaunchKernelGGL((sgemv_q_kernel<QX, EPI, LPRV, UKV>), dim3((unsigned)cdiv(N, 512 / LPRV)), \
                       block, lds, s, X, g, b, K, W, (long)K, bias, Y, N)
    // Products with few rows (N <= 1024: at most 128 workgroups of 8 rows)
    // spread each row over two or four waves instead: 2-4 rows per workgroup,
    // 256-512 workgroups.
    if (N <= 1024 && K >= 1024) {
        if (K <= 1024) SGQ(256, 1);
        else if (K <= 2048) SGQ(256, 2);
        else SGQ(256, 4);
    } else if (N <= 1024 && K >= 512) {
        SGQ(128, 1);
    } else if (K <= 64) SGQ(16, 1);
    else if (K <= 128) SGQ(32, 1);
    else if (K <= 256) SGQ(64, 1);
    else if (K <= 512) SGQ(64, 2);
    else SGQ(64, 4);
#undef SGQ
}

hipError_t launch_sgemv_q(int qx, int epi, const float *X, const float *g, const float *b, int K,
                          const float *W, const float *bias, float *Y, int N, hipStream_t s) {
    if (N <= 0 || K <= 0 || K % 4 != 0 || K > SGEMV_Q_MAX_K) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(W) & 15) != 0) return hipErrorInvalidValue;
    if ((qx == QX_LN && (!g || !b)) || (qx == QX_BIAS_GELU && !b)) return hipErrorInvalidValue;
    if (qx == QX_LN) {
        if (epi) launch_sgemv_q_shape<QX_LN, 1>(X, g, b, K, W, bias, Y, N, s);
        else launch_sgemv_q_shape<QX_LN, 0>(X, g, b, K, W, bias, Y, N, s);
    } else if (qx == QX_BIAS_GELU) {
        if (epi) launch_sgemv_q_shape<QX_BIAS_GELU, 1>(X, g, b, K, W, bias, Y, N, s);
        else launch_sgemv_q_shape<QX_BIAS_GELU, 0>(X, g, b, K, W, bias, Y, N, s);
    } else {
        if (epi) launch_sgemv_q_shape<QX_NONE, 1>(X, g, b, K, W, bias, Y, N, s);
        else launch_sgemv_q_shape<QX_NONE, 0>(X, g, b, K, W, bias, Y, N, s);
    }
    return hipGetLastError();
}

template <int MR>
static void launch_igemv_mr(const GemvPlan &p, int out_mode, int M, int N, int K,
                            const uint8_t *X, long ldx, const int8_t *B, long ldb,
                            const int32_t *col_off, const float *sa, const float *sb, void *Y,
                            long ldy, const Workspace &ws, hipStream_t s) {
    dim3 grid(p.strips, p.splits), block(GV_THREADS);
    int32_t *part = (int32_t *)ws.buf;
    const size_t xsb = (size_t)MR * p.kchunk;  // staged activation rows
    const int nround = p.strips * SGT_ROWS;
    const dim3 rg(reduce_grid(M, N)), rb(256);
    if (out_mode == 0) {
        hipLaunchKernelGGL((igemv_kernel<MR, 0>), grid, block, xsb, s, X, ldx, B, ldb, col_off, sa,
                           sb, Y, ldy, M, N, K, p.kchunk, p.splits, part);
        if (p.splits > 1)
            hipLaunchKernelGGL((igemv_reduce_kernel<0>), rg, rb, 0, s, part, p.splits, M, N,
                               nround, col_off, sa, sb, Y, ldy);
    } else if (out_mode == 1) {
        hipLaunchKernelGGL((igemv_kernel<MR, 1>), grid, block, xsb, s, X, ldx, B, ldb, col_off, sa,
                           sb, Y, ldy, M, N, K, p.kchunk, p.splits, part);
        if (p.splits > 1)
            hipLaunchKernelGGL((igemv_reduce_kernel<1>), rg, rb, 0, s, part, p.splits, M, N,
                               nround, col_off, sa, sb, Y, ldy);
    } else {
        hipLaunchKernelGGL((igemv_kernel<MR, 2>), grid, block, xsb, s, X, ldx, B, ldb, col_off, sa,
                           sb, Y, ldy, M, N, K, p.kchunk, p.splits, part);
        if (p.splits > 1)
            hipLaunchKernelGGL((igemv_reduce_kernel<2>), rg, rb, 0, s, part, p.splits, M, N,
                               nround, col_off, sa, sb, Y, ldy);
    }
}

hipError_t launch_igemv(const GemvPlan &p, int out_mode, int M, int N, int K, const uint8_t *X,
                        long ldx, const int8_t *Bpk, long ldb, const int32_t *col_off,
                        const float *sa, const float *sb, void *Y, long ldy, const Workspace &ws,
                        hipStream_t stream) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (K <= 0) {  // v = 0: the reduce pass over zero splits applies the epilogue
        const dim3 rg(reduce_grid(M, N)), rb(256);
        if (out_mode == 0)
            hipLaunchKernelGGL((igemv_reduce_kernel<0>), rg, rb, 0, stream, nullptr, 0, M, N, N,
                               col_off, sa, sb, Y, ldy);
        else if (out_mode == 1)
            hipLaunchKernelGGL((igemv_reduce_kernel<1>), rg, rb, 0, stream, nullptr, 0, M, N, N,
                               col_off, sa, sb, Y, ldy);
        else
            hipLaunchKernelGGL((igemv_reduce_kernel<2>), rg, rb, 0, stream, nullptr, 0, M, N, N,
                               col_off, sa, sb, Y, ldy);
        return hipGetLastError();
    }
    if (p.splits > 1 && (ws.buf == nullptr || ws.bytes_cap < p.part_bytes)) return hipErrorInvalidValue;
    if (M == 1)
        launch_igemv_mr<1>(p, out_mode, M, N, K, X, ldx, Bpk, ldb, col_off, sa, sb, Y, ldy, ws, stream);
    else if (M <= 2)
        launch_igemv_mr<2>(p, out_mode, M, N, K, X, ldx, Bpk, ldb, col_off, sa, sb, Y, ldy, ws, stream);
    else if (M <= 4)
        launch_igemv_mr<4>(p, out_mode, M, N, K, X, ldx, Bpk, ldb, col_off, sa, sb, Y, ldy, ws, stream);
    else
        launch_igemv_mr<8>(p, out_mode, M, N, K, X, ldx, Bpk, ldb, col_off, sa, sb, Y, ldy, ws, stream);
    return hipGetLastError();
}

// ------------------------------------------------------- grouped GEMV ----
// Many independent decode products in one launch (pcl_gemv_group_*). The
// launch's blocks are a host-built list of (product, strip) work items,
// largest first, so the weights of every product stream at once instead of
// one short launch per product. A block owns a strip of outputs over the
// whole K (no split, no second pass), stages its product's activation rows in
// LDS while its first weight batch is in flight, and reads every weight byte
// once with non-temporal 16-byte loads.
//   GG_F32_N: W K x N (N-contiguous; generate.c:95-107 matvec), 64-column
//             strips; lane (c4 = lane%16, rr = lane/16) of wave w owns 4
//             columns and the contiguous run of rows of group 4w + rr; the 16
//             group sums of a column are added across lanes, then waves, in a
//             fixed order.
//   GG_F32_T: W N x K (K-contiguous rows; the tied head, model.c:64-77),
//             32-row strips: 16 lanes per row, 16-byte pieces k = 4j + 64i.
//   GG_U8S8:  packed N x Kp s8 rows (the INT8 GEMM's layout), 32-row strips,
//             exact int32 dot products of the re-centred activations, then
//             the dequant epilogue of the INT8 GEMM (gemm_bench.c:272-275).

template <int MR>
__device__ __forceinline__ void gg_f32_n(const GgDesc &d, int strip, float *xs, float (*red)[MR][64]) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int c4 = lane & 15, rr = lane >> 4;
    const int M = d.M, N = d.N, K = d.K, ld = d.xld;
    const int run = ld >> 4;  // rows per group, a multiple of 8
    const int n0 = strip * 64, col = n0 + 4 * c4;
    const int colc = min(col, N - 4);  // N % 4 == 0: clamped lanes feed columns >= N only
    const auto W = gbl(static_cast<const float *>(d.W));
    const long ldw = d.ldw;
    const int r0 = (wv * 4 + rr) * run;
    constexpr int UR = 8;  // rows per load batch
    // rows past K load row K-1 and are zeroed, so they add exactly nothing
    auto load_batch = [&](v4f (&w)[UR], int i) {
#pragma unroll
        for (int u = 0; u < UR; u++) {
            const int k = r0 + i + u;
            v4f v = __builtin_nontemporal_load(gvec<v4f>(W + (long)min(k, K - 1) * ldw + colc));
            w[u] = k < K ? v : v4f{0.f, 0.f, 0.f, 0.f};
        }
    };
    v4f wn[UR];
    load_batch(wn, 0);
    stage_rows<MR, false, float, 16>(xs, ld, ld, K, M, static_cast<const float *>(d.X), d.ldx);
    __syncthreads();

    float acc[MR][4];
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[m][j] = 0.f;
    for (int i = 0; i < run; i += UR) {
        v4f w[UR];
#pragma unroll
        for (int u = 0; u < UR; u++) w[u] = wn[u];
        if (i + UR < run) load_batch(wn, i + UR);
#pragma unroll
        for (int m = 0; m < MR; m++) {
            const v4f xa = *reinterpret_cast<const v4f *>(&xs[m * ld + r0 + i]);
            const v4f xb = *reinterpret_cast<const v4f *>(&xs[m * ld + r0 + i + 4]);
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[m][j] += xa[u] * w[u][j];
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[m][j] += xb[u] * w[4 + u][j];
        }
    }
    // groups 4w .. 4w+3 of a column sit in lanes l, l^16, l^32, l^48: the
    // butterfly's sums (l + l^16, then + the other pair) by permlane swaps
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[m][j]), __float_as_uint(acc[m][j]), false, false);
            const float v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
            const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            acc[m][j] = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
        }
    if (rr == 0) {
#pragma unroll
        for (int m = 0; m < MR; m++)
#pragma unroll
            for (int j = 0; j < 4; j++) red[wv][m][4 * c4 + j] = acc[m][j];
    }
    __syncthreads();
    const auto Y = gbl(static_cast<float *>(d.Y));
    for (int o = tid; o < M * 64; o += GV_THREADS) {
        const int m = o >> 6, c = o & 63, n = n0 + c;
        if (n < N) {
            const float sum = ((red[0][m][c] + red[1][m][c]) + red[2][m][c]) + red[3][m][c];
            const float y = sum + (d.bias ? gbl(d.bias)[n] : 0.f);
            const auto dst = Y + (long)m * d.ldy + n;
            *dst = d.accumulate ? *dst + y : y;
        }
    }
}

template <int MR>
__device__ __forceinline__ void gg_f32_t(const GgDesc &d, int strip, float *xs) {
    const int tid = threadIdx.x, j = tid & 15, rs = tid >> 4;
    constexpr int RPL = 2, UK = 4;
    const int M = d.M, N = d.N, K = d.K, ld = d.xld;
    const int n0 = strip * 32;
    const auto W = gbl(static_cast<const float *>(d.W));
    const __attribute__((address_space(1))) float *wrow[RPL];
#pragma unroll
    for (int r = 0; r < RPL; r++) wrow[r] = W + (long)min(n0 + rs + 16 * r, N - 1) * d.ldw;
    // K % 4 == 0; k past K is clamped for the load and skipped in the sums
    auto load_batch = [&](v4f (&w)[UK][RPL], int k0) {
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < RPL; r++)
                w[u][r] = __builtin_nontemporal_load(gvec<v4f>(wrow[r] + min(k0 + 64 * u, K - 4)));
    };
    v4f wn[UK][RPL];
    load_batch(wn, 4 * j);
    stage_rows<MR, false, float, 16>(xs, ld, ld, K, M, static_cast<const float *>(d.X), d.ldx);
    __syncthreads();

    float acc[RPL][MR];
#pragma unroll
    for (int r = 0; r < RPL; r++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r][m] = 0.f;
    for (int k0 = 4 * j; k0 < K; k0 += 64 * UK) {
        v4f w[UK][RPL];
#pragma unroll
        for (int u = 0; u < UK; u++)
#pragma unroll
            for (int r = 0; r < RPL; r++) w[u][r] = wn[u][r];
        if (k0 + 64 * UK < K) load_batch(wn, k0 + 64 * UK);
#pragma unroll
        for (int u = 0; u < UK; u++) {
            const int k = k0 + 64 * u;
            if (k < K) {
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const v4f xv = *reinterpret_cast<const v4f *>(&xs[m * ld + k]);
#pragma unroll
                    for (int r = 0; r < RPL; r++)
                        acc[r][m] += xv[0] * w[u][r][0] + xv[1] * w[u][r][1] + xv[2] * w[u][r][2] +
                                     xv[3] * w[u][r][3];
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPL; r++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r][m] = dpp_sum_last<16>(acc[r][m]);  // the row's 16 lanes, into lane 15
    if (j == 15) {
        const auto Y = gbl(static_cast<float *>(d.Y));
#pragma unroll
        for (int r = 0; r < RPL; r++) {
            const int n = n0 + rs + 16 * r;
#pragma unroll
            for (int m = 0; m < MR; m++) {
                if (m < M && n < N) {
                    const float y = acc[r][m] + (d.bias ? gbl(d.bias)[n] : 0.f);
                    const auto dst = Y + (long)m * d.ldy + n;
                    *dst = d.accumulate ? *dst + y : y;
                }
            }
        }
    }
}

// GG_U8S8 through the matrix cores. A block owns 64 weight rows (16 per
// wave, one tile of v_mfma_i32_16x16x64_i8) over the whole K, walked in
// 256-byte K slices. A slice of a wave's 16 rows is read with four fully
// coalesced loads (4 rows x 256 contiguous bytes each), the next slice's
// loads issued before the current one is used, then turned into the
// A-operand layout through a 4 KB LDS region private to the wave: chunk q of
// row r is written at chunk q ^ r and read back by lane (i, g) as logical
// chunk 4c + g of row i (16 rows at one logical chunk: 16 distinct bank
// groups, both ways). A wave's LDS operations execute in order, so the
// region needs no barrier between a slice's reads and the next slice's
// writes. The activation rows are staged once per block in LDS, re-centred
// (x ^ 0x80 = x - 128 as s8) and zero past K; lane (m, g) of the B operand
// reads the same bytes of row m % MR, so every integer product pairs the
// same k whatever order the hardware sums in. D[i][m] lands in lane
// 16*(i/4) + m, register i % 4. Rows past N load row N-1 and columns m >= M
// come from a repeated row; neither is stored.
constexpr int GGQ_RB = 64;      // rows per block
constexpr int GGQ_SL = 256;     // bytes of K per slice
constexpr int GGQ_WREG = 16 * GGQ_SL;  // LDS bytes per wave

__host__ __device__ inline int ggq_x_bytes(int mr, int K) { return (mr * ((K + 255) / 256 * 256 + 16) + 15) / 16 * 16; }
int ggq_lds_bytes(int mr, int K) { return ggq_x_bytes(mr, K) + 4 * GGQ_WREG; }

template <int MR, bool TWO = (MR >= 8)>
__device__ __forceinline__ void gg_u8s8(const GgDesc &d, int strip, int8_t *lds) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int ri = lane & 15, g = lane >> 4;
    const int M = d.M, N = d.N;
    const int Kp = (d.K + 255) & ~255;  // packed rows are zero from K to Kp (ldw >= Kp)
    const int nsl = Kp / GGQ_SL;
    const int xld = Kp + 16;
    const int n0 = strip * GGQ_RB;
    int8_t *xs = lds;
    int8_t *wreg = lds + ggq_x_bytes(MR, d.K) + wv * GGQ_WREG;
    const auto B = gbl(static_cast<const int8_t *>(d.W));
    // load u of a slice: row 4u + lane/16 of the wave's tile, bytes 16*(lane%16)
    const __attribute__((address_space(1))) int8_t *src[4];
    int8_t *wdst[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int r = 4 * u + g;
        src[u] = B + (long)min(n0 + 16 * wv + r, N - 1) * d.ldw + 16 * ri;
        wdst[u] = wreg + r * GGQ_SL + ((ri ^ r) << 4);
    }
    auto load = [&](v4i (&w)[4], int t) {
#pragma unroll
        for (int u = 0; u < 4; u++) w[u] = __builtin_nontemporal_load(gvec<v4i>(src[u] + t * GGQ_SL));
    };
    // the first slice is in flight while the activations are staged (the
    // epilogue's scales load at the end: loading them here as well takes 12
    // more registers, one wave less per SIMD, and was slower)
    // TWO: two slices in flight per wave (8 KB), slice t + 2 loading into
    // the registers slice t has just handed to LDS; else one
    v4i wa[4], wb[4];
    load(wa, 0);
    if (TWO && nsl > 1) load(wb, 1);
    // one 16-byte load per row per thread and round: rows up to 4 KB stage in one
    // round, and the staging holds MR vector registers instead of 16
    stage_rows<MR, true, uint8_t, 1>(reinterpret_cast<uint8_t *>(xs), xld, Kp, d.K, M,
                                     static_cast<const uint8_t *>(d.X), d.ldx);
    __syncthreads();
    const int8_t *xr = xs + (ri % MR) * xld + 16 * g;
    v4i acc = {0, 0, 0, 0};
    auto step = [&](v4i (&w)[4], int t) {
#pragma unroll
        for (int u = 0; u < 4; u++) *reinterpret_cast<v4i *>(wdst[u]) = w[u];
        if (t + 2 < nsl) load(w, t + 2);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const v4i a = *reinterpret_cast<const v4i *>(wreg + ri * GGQ_SL + (((4 * c + g) ^ ri) << 4));
            const v4i b = *reinterpret_cast<const v4i *>(xr + t * GGQ_SL + 64 * c);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
        }
    };
    if constexpr (TWO) {
        for (int t = 0; t < nsl; t += 2) {
            step(wa, t);
            if (t + 1 < nsl) step(wb, t + 1);
        }
    } else {
        for (int t = 0; t < nsl; t++) {
#pragma unroll
            for (int u = 0; u < 4; u++) wb[u] = wa[u];
            if (t + 1 < nsl) load(wa, t + 1);
#pragma unroll
            for (int u = 0; u < 4; u++) *reinterpret_cast<v4i *>(wdst[u]) = wb[u];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const v4i a = *reinterpret_cast<const v4i *>(wreg + ri * GGQ_SL + (((4 * c + g) ^ ri) << 4));
                const v4i b = *reinterpret_cast<const v4i *>(xr + t * GGQ_SL + 64 * c);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
            }
        }
    }
    // a lane's four results are outputs nb .. nb+3 of row m: one 16-byte store
    const int m = lane & 15, nb = n0 + 16 * wv + 4 * g;
    if (m < M) {
        if (nb + 4 <= N) {
            if (d.out_mode == 0) igemv_write4<0>(d.Y, d.ldy, m, nb, acc, d.col_off, d.sa, d.sb);
            else if (d.out_mode == 1) igemv_write4<1>(d.Y, d.ldy, m, nb, acc, d.col_off, d.sa, d.sb);
            else igemv_write4<2>(d.Y, d.ldy, m, nb, acc, d.col_off, d.sa, d.sb);
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int n = nb + r;
                if (n < N) {
                    if (d.out_mode == 0) igemv_write<0>(d.Y, d.ldy, m, n, acc[r], d.col_off, d.sa, d.sb);
                    else if (d.out_mode == 1) igemv_write<1>(d.Y, d.ldy, m, n, acc[r], d.col_off, d.sa, d.sb);
                    else igemv_write<2>(d.Y, d.ldy, m, n, acc[r], d.col_off, d.sa, d.sb);
                }
            }
        }
    }
}

// Work item b is flat[b]: its product's descriptor with the strip index in
// `strip`, so a block reaches its operands' addresses with one lookup.
template <int MR>
__global__ __launch_bounds__(GV_THREADS) void gemv_group_kernel(const GgDesc *__restrict__ flat) {
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_dyn[];
    __shared__ float red[4][MR][64];
    const GgDesc d = flat[blockIdx.x];
    if (d.kind == GG_F32_N) gg_f32_n<MR>(d, d.strip, reinterpret_cast<float *>(gv_dyn), red);
    else if (d.kind == GG_F32_T) gg_f32_t<MR>(d, d.strip, reinterpret_cast<float *>(gv_dyn));
    else gg_u8s8<MR, (MR >= 4)>(d, d.strip, reinterpret_cast<int8_t *>(gv_dyn));
}

// A group whose products are all INT8: the same work items through the
// matrix-core path alone, so the kernel holds only that path's registers
// (58-86 against 124 for the kernel that also carries the fp32 paths) and a
// SIMD takes five or more of its waves instead of four.
template <int MR>
__global__ __launch_bounds__(GV_THREADS) void gemv_group_u8s8_kernel(const GgDesc *__restrict__ flat) {
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_dyn[];
    const GgDesc d = flat[blockIdx.x];
    gg_u8s8<MR, (MR >= 4)>(d, d.strip, reinterpret_cast<int8_t *>(gv_dyn));
}

// GG_U8S8 with one or two activation rows through dot products: the same
// 64-row strips, 16 lanes per weight row and four rows per 16-lane group;
// lane j reads bytes 16j + 256u of each row (fully coalesced: a 16-lane group
// covers 256 contiguous bytes of a row), 512 bytes of K per batch, the next
// batch in flight while the current one is multiplied, the first one (and
// the epilogue's scales) before the activations are staged. Products with
// v_dot4_i32_i8 of the re-centred activations (x ^ 0x80 = x - 128, zero from
// K to Kp as the packed weights are) are exact in any order; the 16 lanes of
// a row are then summed by shuffles. With one or two rows the matrix-core
// path spends more LDS traffic (a transposing round trip of every weight
// byte) than the products need. (Strips sized to ~32 KB per product -- 16
// rows at K = 2048 -- were slower on the grown decode sweep: the extra work
// items no longer fit the chip in one round.)
constexpr int GGD_RPL = 4;  // rows per 16-lane group
constexpr int GGD_UK = 2;   // 256-byte K steps per batch
static_assert(16 * GGD_RPL == GGQ_RB, "the dot path uses the matrix-core path's strips");

template <int MR>
__device__ __forceinline__ void gg_u8s8_dot(const GgDesc &d, int strip, int8_t *xs) {
    const int tid = threadIdx.x, j = tid & 15, rs = tid >> 4;
    const int M = d.M, N = d.N;
    const int Kp = (d.K + 255) & ~255;  // packed rows are zero from K to Kp (ldw >= Kp)
    const int xld = Kp + 16;
    const int n0 = strip * GGQ_RB;
    const auto B = gbl(static_cast<const int8_t *>(d.W));
    const __attribute__((address_space(1))) int8_t *wrow[GGD_RPL];
#pragma unroll
    for (int r = 0; r < GGD_RPL; r++) wrow[r] = B + (long)min(n0 + rs + 16 * r, N - 1) * d.ldw + 16 * j;
    // steps k = 256u past Kp are clamped to the last step for the load and
    // skipped in the products
    auto load_batch = [&](v4i (&w)[GGD_UK][GGD_RPL], int k0) {
#pragma unroll
        for (int u = 0; u < GGD_UK; u++)
#pragma unroll
            for (int r = 0; r < GGD_RPL; r++)
                w[u][r] = __builtin_nontemporal_load(gvec<v4i>(wrow[r] + min(k0 + 256 * u, Kp - 256)));
    };
    v4i wn[GGD_UK][GGD_RPL];
    load_batch(wn, 0);
    // the epilogue's operands load with the first batch (a block's life is
    // then one memory latency, not two): column scale and offset of the
    // group's four rows, row scales
    float sbv[GGD_RPL], sav[MR];
    unsigned offv[GGD_RPL];
#pragma unroll
    for (int r = 0; r < GGD_RPL; r++) {
        const int n = min(n0 + rs + 16 * r, N - 1);
        sbv[r] = d.out_mode != 0 ? gbl(d.sb)[n] : 0.f;
        offv[r] = d.col_off ? (unsigned)gbl(d.col_off)[n] : 0u;
    }
#pragma unroll
    for (int m = 0; m < MR; m++) sav[m] = d.out_mode == 2 ? gbl(d.sa)[min(m, M - 1)] : 1.f;
    stage_rows<MR, true, uint8_t, 1>(reinterpret_cast<uint8_t *>(xs), xld, Kp, d.K, M,
                                     static_cast<const uint8_t *>(d.X), d.ldx);
    __syncthreads();
    int32_t acc[GGD_RPL][MR];
#pragma unroll
    for (int r = 0; r < GGD_RPL; r++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r][m] = 0;
    for (int k0 = 0; k0 < Kp; k0 += 256 * GGD_UK) {
        v4i w[GGD_UK][GGD_RPL];
#pragma unroll
        for (int u = 0; u < GGD_UK; u++)
#pragma unroll
            for (int r = 0; r < GGD_RPL; r++) w[u][r] = wn[u][r];
        if (k0 + 256 * GGD_UK < Kp) load_batch(wn, k0 + 256 * GGD_UK);
#pragma unroll
        for (int u = 0; u < GGD_UK; u++) {
            const int k = k0 + 256 * u;
            if (k < Kp) {
                v4i xv[MR];
#pragma unroll
                for (int m = 0; m < MR; m++) xv[m] = *reinterpret_cast<const v4i *>(xs + m * xld + k + 16 * j);
#pragma unroll
                for (int r = 0; r < GGD_RPL; r++)
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        int a = acc[r][m];
                        a = __builtin_amdgcn_sdot4(xv[m][0], w[u][r][0], a, false);
                        a = __builtin_amdgcn_sdot4(xv[m][1], w[u][r][1], a, false);
                        a = __builtin_amdgcn_sdot4(xv[m][2], w[u][r][2], a, false);
                        a = __builtin_amdgcn_sdot4(xv[m][3], w[u][r][3], a, false);
                        acc[r][m] = a;
                    }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GGD_RPL; r++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r][m] = dpp_sum_last<16>(acc[r][m]);  // into lane 15, exact
    // lane 15 of a group writes its four outputs of each row m (rows past M and
    // outputs past N are not stored), as igemv_write: v + col_off, then
    // float(v) * dq with dq = sb[n] or sa[m] * sb[n]
#pragma unroll
    for (int m = 0; m < MR; m++) {
        if (j == 15 && m < M) {
#pragma unroll
            for (int r = 0; r < GGD_RPL; r++) {
                const int n = n0 + rs + 16 * r;
                if (n < N) {
                    const int32_t v = (int32_t)((unsigned)acc[r][m] + offv[r]);
                    const long o = (long)m * d.ldy + n;
                    if (d.out_mode == 0) {
                        gbl(reinterpret_cast<int32_t *>(d.Y))[o] = v;
                    } else {
                        const float dq = d.out_mode == 2 ? sav[m] * sbv[r] : sbv[r];
                        gbl(reinterpret_cast<float *>(d.Y))[o] = (float)v * dq;
                    }
                }
            }
        }
    }
}

template <int MR>
__global__ __launch_bounds__(GV_THREADS) void gemv_group_dot_kernel(const GgDesc *__restrict__ flat) {
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_dyn[];
    const GgDesc d = flat[blockIdx.x];
    gg_u8s8_dot<MR>(d, d.strip, reinterpret_cast<int8_t *>(gv_dyn));
}

// One product, descriptor by value (no device table): block b = strip b.
template <int MR>
__global__ __launch_bounds__(GV_THREADS) void gemv_one_u8s8_kernel(GgDesc d) {
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_dyn[];
    gg_u8s8<MR>(d, blockIdx.x, reinterpret_cast<int8_t *>(gv_dyn));
}

bool igemv_mfma_fits(int M, int N, int K, long ldb) {
    const int mr = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8));
    return M >= 1 && M <= 8 && K >= 1 && (long)N * ldb < (1L << 31) && ldb >= ((K + 255) & ~255) &&
           ggq_lds_bytes(mr, K) <= 65536;
}

hipError_t launch_igemv_mfma(int out_mode, int M, int N, int K, const uint8_t *X, long ldx,
                             const int8_t *Bpk, long ldb, const int32_t *col_off, const float *sa,
                             const float *sb, void *Y, long ldy, hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (!igemv_mfma_fits(M, N, K, ldb)) return hipErrorInvalidValue;
    GgDesc d = {};
    d.kind = GG_U8S8, d.M = M, d.N = N, d.K = K;
    d.X = X, d.ldx = ldx, d.W = Bpk, d.ldw = ldb;
    d.col_off = col_off, d.sa = sa, d.sb = sb, d.Y = Y, d.ldy = ldy;
    d.out_mode = out_mode;
    d.xld = gg_stage_ld(GG_U8S8, K);
    const dim3 grid(cdiv(N, GGQ_RB)), block(GV_THREADS);
    const int mr = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8));
    const size_t lds = (size_t)ggq_lds_bytes(mr, K);
    switch (mr) {
        case 1: hipLaunchKernelGGL(gemv_one_u8s8_kernel<1>, grid, block, lds, s, d); break;
        case 2: hipLaunchKernelGGL(gemv_one_u8s8_kernel<2>, grid, block, lds, s, d); break;
        case 4: hipLaunchKernelGGL(gemv_one_u8s8_kernel<4>, grid, block, lds, s, d); break;
        default: hipLaunchKernelGGL(gemv_one_u8s8_kernel<8>, grid, block, lds, s, d); break;
    }
    return hipGetLastError();
}

int gg_strip_rows(int kind) { return kind == GG_F32_T ? 32 : (kind == GG_F32_N ? 64 : GGQ_RB); }

int gg_stage_ld(int kind, int K) {
    if (kind == GG_F32_N) return 16 * ((cdiv(K, 16) + 7) / 8 * 8);
    if (kind == GG_F32_T) return (K + 63) / 64 * 64;
    return (K + 255) / 256 * 256 + 16;
}

size_t gg_lds_bytes(int kind, int K, int mr) {
    if (kind == GG_U8S8) return (size_t)ggq_lds_bytes(mr, K);
    return (size_t)mr * gg_stage_ld(kind, K) * 4;
}

hipError_t launch_gemv_group(const GgDesc *flat, int n_items, int mr,
                             size_t lds_bytes, bool all_u8s8, hipStream_t s) {
    if (n_items <= 0) return hipSuccess;
    const dim3 grid(n_items), block(GV_THREADS);
    if (all_u8s8) {
        // one or two rows: dot products (the staging is the same as the
        // matrix-core path's, without its 16 KB of per-wave regions)
        const size_t dot_lds = lds_bytes > 4 * (size_t)GGQ_WREG ? lds_bytes - 4 * (size_t)GGQ_WREG : lds_bytes;
        switch (mr) {
            case 1: hipLaunchKernelGGL(gemv_group_dot_kernel<1>, grid, block, dot_lds, s, flat); break;
            case 2: hipLaunchKernelGGL(gemv_group_dot_kernel<2>, grid, block, dot_lds, s, flat); break;
            case 4: hipLaunchKernelGGL(gemv_group_u8s8_kernel<4>, grid, block, lds_bytes, s, flat); break;
            default: hipLaunchKernelGGL(gemv_group_u8s8_kernel<8>, grid, block, lds_bytes, s, flat); break;
        }
        return hipGetLastError();
    }
    switch (mr) {
        case 1: hipLaunchKernelGGL(gemv_group_kernel<1>, grid, block, lds_bytes, s, flat); break;
        case 2: hipLaunchKernelGGL(gemv_group_kernel<2>, grid, block, lds_bytes, s, flat); break;
        case 4: hipLaunchKernelGGL(gemv_group_kernel<4>, grid, block, lds_bytes, s, flat); break;
        default: hipLaunchKernelGGL(gemv_group_kernel<8>, grid, block, lds_bytes, s, flat); break;
    }
    return hipGetLastError();
}

// ---------------------------------------------- allocation-free scratch ----
// The split-K partial sums of pcl_sgemv_noalloc live in this file-scope device
// array: one copy per GPU, held until the process ends, shared by every such
// call on that GPU (calls that overlap on one GPU race on it). In host code
// the name `scratch` is only a host-side stand-in for the symbol; its device
// address comes from hipGetSymbolAddress (gemv_noalloc_scratch), once per
// device, and only that address is ever handed to a kernel.
static __device__ __align__(256) unsigned char scratch[GEMV_NOALLOC_SCRATCH_BYTES];

hipError_t gemv_noalloc_scratch(void **dev_ptr) {
    return hipGetSymbolAddress(dev_ptr, HIP_SYMBOL(scratch));
}

}  // namespace pcl
