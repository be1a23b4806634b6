// attn.hip -- causal multi-head attention on the fp32 matrix cores (gfx950).
//
// Forward (train.c:339-370 attention_forward; gpu_kernels.cu:403-432 attn_fwd):
// per (batch, head) and query i, p_ij = softmax_j<=i(scale * q_i . k_j) and
// att_i = sum_j p_ij v_j, with the probabilities optionally stored for the
// backward ([B*H][T][T], zero above the diagonal as gpu_kernels.cu:279 does).
//
// One launch, no score matrix in HBM: a workgroup of four waves owns 128
// queries of one head (32 per wave) and streams 32-key blocks of K (and V)
// through double-buffered LDS. Each wave keeps its queries' Q in registers and
// computes the transposed score block S^T = K_blk . Q^T with
// v_mfma_f32_32x32x2f32, so a lane holds 16 scores of ONE query (its column)
// and a row reduction is 16 lane-local values plus one exchange with lane^32.
// Pass 1 accumulates the row maximum and exp-sum; pass 2 recomputes S^T, forms
// the normalised p (the reference's p = exp(s - max) / sum, computed in base 2
// as 2^(s' - (max' + log2 sum)) with Q pre-scaled by scale * log2 e, then
// att = sum_j p_j v_j), stores p when asked, and accumulates
// O^T = V^T . P^T where P^T is exactly the register layout S^T left behind
// (B operand), V^T comes from LDS one float per lane (A operand).
#include "internal.h"

#include <math.h>

namespace pcl {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int AT_QB = 128;  // queries per workgroup (4 waves x 32)
constexpr int AT_KB = 32;   // keys per block

// LDS rows padded so fragment reads are bank-conflict-free: K rows are read
// as 16-byte pieces by 16 lanes on 16 rows (stride DH + 4 floats puts row r
// at bank 4r mod 64 for DH a multiple of 64, a distinct 4-bank group for DH =
// 32 too); V rows j and j + 4 are read by the two lane halves (stride DH + 8
// puts them 32 banks apart).
template <int DH>
struct AttnTile {
    static constexpr int KS = DH + 4, VS = DH + 8;
    static constexpr int KFL = AT_KB * KS, VFL = AT_KB * VS;  // floats per block
    static constexpr int PT = AT_KB * DH / 4 / 256;           // float4 loads per thread per block
    static_assert(DH % 32 == 0 && PT >= 1, "head size");
};

// 32 x DH block of rows [r0, r0 + 32) of a (rows x ld) operand at column c0,
// rows >= T read as zero: this thread's float4 pieces.
template <int DH>
__device__ __forceinline__ void at_load(v4f (&r)[AttnTile<DH>::PT], const float *__restrict__ X,
                                        long ld, long row0, int r0, int T, int tid) {
    constexpr int C4 = DH / 4;
#pragma unroll
    for (int u = 0; u < AttnTile<DH>::PT; u++) {
        const int idx = u * 256 + tid, rr = idx / C4, c4 = idx % C4;
        v4f v = {0.f, 0.f, 0.f, 0.f};
        if (r0 + rr < T) v = *reinterpret_cast<const v4f *>(X + (row0 + r0 + rr) * ld + c4 * 4);
        r[u] = v;
    }
}
template <int DH, int STRIDE>
__device__ __forceinline__ void at_store(float *lds, const v4f (&r)[AttnTile<DH>::PT], int tid) {
    constexpr int C4 = DH / 4;
#pragma unroll
    for (int u = 0; u < AttnTile<DH>::PT; u++) {
        const int idx = u * 256 + tid, rr = idx / C4, c4 = idx % C4;
        *reinterpret_cast<v4f *>(lds + rr * STRIDE + c4 * 4) = r[u];
    }
}

// max(v, the value of lane ^ 32) through v_permlane32_swap (a VALU exchange
// of the wave's halves, no LDS crossbar round trip)
__device__ __forceinline__ float at_max_halves(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// S^T block (keys x queries) of this wave: A = K rows from LDS (16-byte piece
// 8q + 4lg of row r32, element e at MFMA step 4q + e), B = the wave's Q in the
// same k order (registers).
// key offset (within the block) of accumulator element v for lane half lg
__device__ __forceinline__ constexpr int at_key(int v, int lg) { return (v >> 2) * 8 + lg * 4 + (v & 3); }

// All of a block's fragment reads are issued before its MFMAs (in groups of
// up to 8 pieces), so the waits between them count down instead of draining
// the LDS queue before every MFMA.
template <int DH>
__device__ __forceinline__ v16f at_scores(const float *Ks, const v4f (&qf)[DH / 8], int r32, int lg) {
    constexpr int G = DH >= 128 ? 2 : (DH / 8 < 8 ? DH / 8 : 8);  // pieces per read group
    v16f s;
#pragma unroll
    for (int v = 0; v < 16; v++) s[v] = 0.f;
    const float *krow = Ks + r32 * AttnTile<DH>::KS + 4 * lg;
#pragma unroll
    for (int q0 = 0; q0 < DH / 8; q0 += G) {
        v4f kf[G];
#pragma unroll
        for (int q = 0; q < G; q++) kf[q] = *reinterpret_cast<const v4f *>(krow + 8 * (q0 + q));
        __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
        for (int q = 0; q < G; q++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[q][e], qf[q0 + q][e], s, 0, 0, 0);
    }
    return s;
}

// acc[nb] += X^T . W^T over one 32-key block: A = X rows (keys in the score
// layout's order, one float per lane from LDS, row stride VS), B = w[s4]
// (this lane's 16 key weights). Reads go out 8 key steps at a time (2 for
// 128-wide heads, whose accumulators leave fewer registers).
template <int DH>
__device__ __forceinline__ void at_accum(v16f (&acc)[DH / 32], const float *Xs, const float (&w)[16],
                                         int r32, int lg) {
    constexpr int S8 = DH >= 128 ? 2 : 8;  // key steps per read group
    const float *xcol = Xs + r32;
#pragma unroll
    for (int h8 = 0; h8 < 16; h8 += S8) {
        float xa[S8][DH / 32];
#pragma unroll
        for (int s4 = 0; s4 < S8; s4++)
#pragma unroll
            for (int nb = 0; nb < DH / 32; nb++)
                xa[s4][nb] = xcol[at_key(h8 + s4, lg) * AttnTile<DH>::VS + nb * 32];
        __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
        for (int s4 = 0; s4 < S8; s4++)
#pragma unroll
            for (int nb = 0; nb < DH / 32; nb++)
                acc[nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[s4][nb], w[h8 + s4], acc[nb], 0, 0, 0);
    }
}


// The online-softmax step of one key block in the log2 domain: the wave's Q
// fragments carry scale * log2(e), so s is already the exponent base 2 and
// p = 2^(s - m). Only a block holding keys past a query of the wave or past T
// (the diagonal block, the tail) is masked. The running maximum m moves only
// when a row's block maximum exceeds it by more than AT_LAZY (then the row's
// O^T and l are rescaled by 2^(m_old - m_new)); otherwise p = 2^(s - m) stays
// below 2^AT_LAZY. O / l and m + log2(l) do not depend on which m was used.
// The caller guarantees a visible key in every block it passes (so m is
// finite after the first).
constexpr float AT_LAZY = 8.f;
constexpr float AT_LOG2E = 1.44269504088896341f, AT_LN2 = 0.693147180559945309f;

// x = the block's scores with keys j > qi or j >= T set to -inf (only when
// the wave-uniform masked is set; keys k0 + at_key(v, lg)); returns max x.
__device__ __forceinline__ float at_mask(const v16f &s, bool masked, int k0, int qi, int T, int lg,
                                         float (&x)[16]) {
    if (masked) {
        const int lim = min(qi, T - 1) - k0;
#pragma unroll
        for (int v = 0; v < 16; v++) x[v] = at_key(v, lg) <= lim ? s[v] : -INFINITY;
    } else {
#pragma unroll
        for (int v = 0; v < 16; v++) x[v] = s[v];
    }
    float bm = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; v++) bm = fmaxf(bm, x[v]);
    return bm;
}

template <int DH>
__device__ __forceinline__ void at_online(const v16f &s, bool masked, int k0, int qi, int T, int lg, float &m,
                                          float &l, v16f (&oacc)[DH / 32], float (&p)[16]) {
    float x[16];
    const float bm = at_mask(s, masked, k0, qi, T, lg, x);
    const float mn = fmaxf(m, at_max_halves(bm));  // lanes i and i ^ 32 agree
    const bool grow = mn > m + AT_LAZY;
    if (__any(grow)) {
        const float mu = grow ? mn : m;
        const float alpha = __builtin_amdgcn_exp2f(m - mu);  // 1 where m stays, 0 on the first block
        l *= alpha;
#pragma unroll
        for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
            for (int v = 0; v < 16; v++) oacc[nb][v] *= alpha;
        m = mu;
    }
    float ps = 0.f;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        p[v] = __builtin_amdgcn_exp2f(x[v] - m);
        ps += p[v];
    }
    l += ps;
}

template <int DH>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(const float *__restrict__ Q,
                                                          const float *__restrict__ K,
                                                          const float *__restrict__ V, long ld,
                                                          float *__restrict__ O, long ldo,
                                                          float *__restrict__ P, int T, int H,
                                                          int BH, float scale) {
    using TL = AttnTile<DH>;
    __shared__ __attribute__((aligned(16))) float lds[2 * (TL::KFL + TL::VFL)];
    const int tid = threadIdx.x, lane = tid & 63, r32 = lane & 31, lg = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Causal work grows with the query block. The first half of the grid takes
    // the heavy blocks (descending), the second half the light ones
    // (ascending): the two workgroups a CU receives in the two dispatch rounds
    // then sum to about the same work (nqb - 1 + 1 blocks' worth).
    const int nqb = (T + AT_QB - 1) / AT_QB, half = (nqb + 1) / 2;
    const int L = (int)(blockIdx.x / BH), bh = (int)(blockIdx.x % BH);
    const int qblk = L < half ? nqb - 1 - L : L - half;
    const int b = bh / H, h = bh % H;
    const long row0 = (long)b * T;  // first token row of this sequence
    const int hc = h * DH;          // first column of this head
    // the light half takes its 32-query slices in reverse wave order, so the
    // waves sharing a SIMD (one from each half) sum to the same work
    const int wslot = L < half ? wave : 3 - wave;
    const int q0 = qblk * AT_QB, q0w = q0 + wslot * 32;
    const int qi = q0w + r32;              // this lane's query
    const int qlast = min(T - 1, q0 + AT_QB - 1);
    const int kb_last = qlast / AT_KB;     // last key block of the workgroup
    const int kbw = q0w < T ? min(T - 1, q0w + 31) / AT_KB : -1;  // last key block of this wave

    // Q carries scale * log2(e): scores come out in log2 units and
    // p = 2^(s - m) / l = 2^(s - (m + log2 l))
    v4f qf[DH / 8];
    const float qsc = scale * AT_LOG2E;
    {
        const float *qrow = Q + (row0 + min(qi, T - 1)) * ld + hc + 4 * lg;
#pragma unroll
        for (int q = 0; q < DH / 8; q++) qf[q] = *reinterpret_cast<const v4f *>(qrow + 8 * q) * qsc;
    }
    // buffer u of the double-buffered K and V blocks
    auto Kb = [&](int u) { return lds + (u & 1) * (TL::KFL + TL::VFL); };
    auto Vb = [&](int u) { return lds + (u & 1) * (TL::KFL + TL::VFL) + TL::KFL; };
    v4f kr[TL::PT], vr[TL::PT];

    // ---- pass 1: row maximum and exp-sum over keys j <= i (this lane's half)
    float m = -INFINITY, l = 0.f;
    at_load<DH>(kr, K + hc, ld, row0, 0, T, tid);
    at_store<DH, TL::KS>(Kb(0), kr, tid);
    __syncthreads();
    for (int kb = 0; kb <= kb_last; kb++) {
        if (kb < kb_last) at_load<DH>(kr, K + hc, ld, row0, (kb + 1) * AT_KB, T, tid);
        if (kb <= kbw) {
            const v16f s = at_scores<DH>(Kb(kb), qf, r32, lg);
            float x[16];
            const float mn = fmaxf(m, at_mask(s, kb * AT_KB >= q0w || (kb + 1) * AT_KB > T, kb * AT_KB, qi, T,
                                              lg, x));
            if (mn != -INFINITY) {  // this lane half may not have seen a key yet
                float acc = 0.f;
#pragma unroll
                for (int v = 0; v < 16; v++) acc += __builtin_amdgcn_exp2f(x[v] - mn);
                l = l * __builtin_amdgcn_exp2f(m - mn) + acc;
                m = mn;
            }
        }
        if (kb < kb_last) at_store<DH, TL::KS>(Kb(kb + 1), kr, tid);
        __syncthreads();
    }
    // combine the two key halves of each query (lanes c and c + 32)
    {
        const float mo = __shfl_xor(m, 32), lo = __shfl_xor(l, 32);
        const float mx = fmaxf(m, mo);
        const float lt = (m == -INFINITY ? 0.f : l * __builtin_amdgcn_exp2f(m - mx)) +
                         (mo == -INFINITY ? 0.f : lo * __builtin_amdgcn_exp2f(mo - mx));
        m = mx + __log2f(lt);  // p = 2^(s - m) from here on
    }

    // ---- pass 2: normalised probabilities, stored if asked, and O^T += V^T P^T
    v16f oacc[DH / 32];
#pragma unroll
    for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
        for (int v = 0; v < 16; v++) oacc[nb][v] = 0.f;
    const bool store_p = P != nullptr && qi < T;
    float *prow = store_p ? P + ((long)bh * T + qi) * T : nullptr;
    const bool vec_p = (T & 3) == 0 && (reinterpret_cast<uintptr_t>(P) & 15) == 0;
    at_load<DH>(kr, K + hc, ld, row0, 0, T, tid);
    at_load<DH>(vr, V + hc, ld, row0, 0, T, tid);
    at_store<DH, TL::KS>(Kb(0), kr, tid);
    at_store<DH, TL::VS>(Vb(0), vr, tid);
    __syncthreads();
    for (int kb = 0; kb <= kb_last; kb++) {
        if (kb < kb_last) {
            at_load<DH>(kr, K + hc, ld, row0, (kb + 1) * AT_KB, T, tid);
            at_load<DH>(vr, V + hc, ld, row0, (kb + 1) * AT_KB, T, tid);
        }
        if (kb <= kbw) {
            const v16f s = at_scores<DH>(Kb(kb), qf, r32, lg);
            float p[16];
            at_mask(s, kb * AT_KB >= q0w || (kb + 1) * AT_KB > T, kb * AT_KB, qi, T, lg, p);
#pragma unroll
            for (int v = 0; v < 16; v++) p[v] = __builtin_amdgcn_exp2f(p[v] - m);  // 2^-inf = 0
            // elements 4g .. 4g+3 are keys 8g + 4lg + 0..3: one 16-byte store each
            if (store_p && vec_p && (kb + 1) * AT_KB <= T) {  // a whole block inside T
                float *pr = prow + kb * AT_KB + 4 * lg;
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++)
                    *reinterpret_cast<v4f *>(pr + 8 * g4) = v4f{p[4 * g4], p[4 * g4 + 1], p[4 * g4 + 2], p[4 * g4 + 3]};
            } else if (store_p) {
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const int j0 = kb * AT_KB + 8 * g4 + 4 * lg;
                    if (vec_p && j0 + 3 < T) {
                        *reinterpret_cast<v4f *>(prow + j0) =
                            v4f{p[4 * g4], p[4 * g4 + 1], p[4 * g4 + 2], p[4 * g4 + 3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (j0 + e < T) prow[j0 + e] = p[4 * g4 + e];
                    }
                }
            }
            at_accum<DH>(oacc, Vb(kb), p, r32, lg);
        }
        if (kb < kb_last) {
            at_store<DH, TL::KS>(Kb(kb + 1), kr, tid);
            at_store<DH, TL::VS>(Vb(kb + 1), vr, tid);
        }
        __syncthreads();
    }

    // att: O^T element v of block nb is (d = 32 nb + key-layout row v, query qi)
    if (qi < T) {
        float *orow = O + (row0 + qi) * ldo + hc;
#pragma unroll
        for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
            for (int v = 0; v < 16; v++) orow[nb * 32 + at_key(v, lg)] = oacc[nb][v];
    }
    // probabilities right of this wave's last key block are zero (the future)
    if (P != nullptr && q0w < T) {
        const int c0 = (kbw + 1) * AT_KB;
        for (int rr = 0; rr < 32 && q0w + rr < T; rr++) {
            float *zr = P + ((long)bh * T + q0w + rr) * T;
            for (int c = c0 + lane; c < T; c += 64) zr[c] = 0.f;
        }
    }
}

// One pass with a running maximum, for callers that need no probabilities:
// per key block the two lanes of a query agree on the block maximum (one
// exchange) and add 2^(s - m) . v (at_online: base 2, scale folded into Q,
// masking and rescaling only where a block needs them). Scores are computed
// once (2/3 of the two-pass matrix work); att = O / l, and the row's natural
// log-sum-exp ln2 (m + log2 l) is stored when lse is given
// (p_ij = exp(scale q_i.k_j - lse_i)).
template <int DH, int SB>
__global__ __launch_bounds__(256, 2) void attn_fwd_online_kernel(const float *__restrict__ Q,
                                                                 const float *__restrict__ K,
                                                                 const float *__restrict__ V, long ld,
                                                                 float *__restrict__ O, long ldo,
                                                                 float *__restrict__ lse, int T, int H,
                                                                 int BH, float scale) {
    using TL = AttnTile<DH>;
    __shared__ __attribute__((aligned(16))) float lds[2 * SB * (TL::KFL + TL::VFL)];
    const int tid = threadIdx.x, lane = tid & 63, r32 = lane & 31, lg = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nqb = (T + AT_QB - 1) / AT_QB, half = (nqb + 1) / 2;
    const int L = (int)(blockIdx.x / BH), bh = (int)(blockIdx.x % BH);
    const int qblk = L < half ? nqb - 1 - L : L - half;
    // the light half takes its 32-query slices in reverse wave order, so the
    // waves sharing a SIMD (one from each half) sum to the same work
    const int wslot = L < half ? wave : 3 - wave;
    const int b = bh / H, h = bh % H;
    const long row0 = (long)b * T;
    const int hc = h * DH;
    const int q0 = qblk * AT_QB, q0w = q0 + wslot * 32;
    const int qi = q0w + r32;
    const int qlast = min(T - 1, q0 + AT_QB - 1);
    const int kb_last = qlast / AT_KB;
    const int kbw = q0w < T ? min(T - 1, q0w + 31) / AT_KB : -1;

    v4f qf[DH / 8];
    const float qsc = scale * AT_LOG2E;  // scores in log2 units
    {
        const float *qrow = Q + (row0 + min(qi, T - 1)) * ld + hc + 4 * lg;
#pragma unroll
        for (int q = 0; q < DH / 8; q++) qf[q] = *reinterpret_cast<const v4f *>(qrow + 8 * q) * qsc;
    }
    // SB key blocks per stage of a double-buffered ring, one barrier per stage
    auto Kb = [&](int u, int sb) { return lds + ((u & 1) * SB + sb) * (TL::KFL + TL::VFL); };
    auto Vb = [&](int u, int sb) { return lds + ((u & 1) * SB + sb) * (TL::KFL + TL::VFL) + TL::KFL; };
    v4f kr[SB][TL::PT], vr[SB][TL::PT];
    const int nst = kb_last / SB + 1;

    v16f oacc[DH / 32];
#pragma unroll
    for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
        for (int v = 0; v < 16; v++) oacc[nb][v] = 0.f;
    float m = -INFINITY, l = 0.f;
#pragma unroll
    for (int sb = 0; sb < SB; sb++) {
        at_load<DH>(kr[sb], K + hc, ld, row0, sb * AT_KB, T, tid);
        at_load<DH>(vr[sb], V + hc, ld, row0, sb * AT_KB, T, tid);
    }
#pragma unroll
    for (int sb = 0; sb < SB; sb++) {
        at_store<DH, TL::KS>(Kb(0, sb), kr[sb], tid);
        at_store<DH, TL::VS>(Vb(0, sb), vr[sb], tid);
    }
    __syncthreads();
    for (int st = 0; st < nst; st++) {
        if (st + 1 < nst) {
#pragma unroll
            for (int sb = 0; sb < SB; sb++) {
                at_load<DH>(kr[sb], K + hc, ld, row0, ((st + 1) * SB + sb) * AT_KB, T, tid);
                at_load<DH>(vr[sb], V + hc, ld, row0, ((st + 1) * SB + sb) * AT_KB, T, tid);
            }
        }
#pragma unroll
        for (int sb = 0; sb < SB; sb++) {
            const int kb = st * SB + sb;
            if (kb <= kbw) {
                const v16f s = at_scores<DH>(Kb(st, sb), qf, r32, lg);
                float p[16];
                at_online<DH>(s, kb * AT_KB >= q0w || (kb + 1) * AT_KB > T, kb * AT_KB, qi, T, lg, m, l, oacc, p);
                at_accum<DH>(oacc, Vb(st, sb), p, r32, lg);
            }
        }
        if (st + 1 < nst) {
#pragma unroll
            for (int sb = 0; sb < SB; sb++) {
                at_store<DH, TL::KS>(Kb(st + 1, sb), kr[sb], tid);
                at_store<DH, TL::VS>(Vb(st + 1, sb), vr[sb], tid);
            }
        }
        __syncthreads();
    }
    l += __shfl_xor(l, 32);  // the two key halves share m
    if (qi < T) {
        const float inv = 1.f / l;
        float *orow = O + (row0 + qi) * ldo + hc;
#pragma unroll
        for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
            for (int v = 0; v < 16; v++) orow[nb * 32 + at_key(v, lg)] = oacc[nb][v] * inv;
        if (lse && lg == 0) lse[(long)bh * T + qi] = (m + __log2f(l)) * AT_LN2;
    }
}

// ---------------------------------------------------------------- backward
// train.c:374-407 attention_backward / gpu_kernels.cu:437-486 attn_bwd, from
// the forward's stored probabilities P:
//   dP_ij = dO_i . v_j,  D_i = sum_j P_ij dP_ij,  dS_ij = P_ij (dP_ij - D_i) scale
//   dQ_i = sum_j dS_ij k_j,  dK_j = sum_i dS_ij q_i,  dV_j = sum_i P_ij dO_i
// Kernel A (per 128 queries of one head, like the forward): dP^T = V_blk .
// dO^T in the score layout (lane = query, 16 keys), pass 1 sums D_i, pass 2
// forms dS (stored to the [B*H][T][T] scratch for kernel B, 16-byte pieces)
// and accumulates dQ^T = K^T dS^T with dS^T as the register B operand.
// Kernel B (per 128 keys): dV^T = dO^T P and dK^T = Q^T dS over the query
// blocks at or after the keys (causal), with dO and Q blocks in LDS (A
// operand, one float per lane) and P, dS rows read straight from HBM as the B
// operand (32 consecutive keys per lane half: one 128-byte row piece).

template <int DH>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_kernel(
    const float *__restrict__ dO, long ldo, const float *__restrict__ K,
    const float *__restrict__ V, long ld, const float *__restrict__ P, float *__restrict__ dS,
    float *__restrict__ dQ, long ldg, int T, int H, int BH, float scale, int accumulate,
    const float *__restrict__ Ofw, long ldfw) {
    using TL = AttnTile<DH>;
    __shared__ __attribute__((aligned(16))) float lds[2 * (TL::KFL + TL::VFL)];
    const int tid = threadIdx.x, lane = tid & 63, r32 = lane & 31, lg = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nqb = (T + AT_QB - 1) / AT_QB, half = (nqb + 1) / 2;
    const int L = (int)(blockIdx.x / BH), bh = (int)(blockIdx.x % BH);
    const int qblk = L < half ? nqb - 1 - L : L - half;
    const int b = bh / H, h = bh % H;
    const long row0 = (long)b * T;
    const int hc = h * DH;
    const int q0 = qblk * AT_QB, q0w = q0 + wave * 32;
    const int qi = q0w + r32;
    const int kb_last = min(T - 1, q0 + AT_QB - 1) / AT_KB;
    const int kbw = q0w < T ? min(T - 1, q0w + 31) / AT_KB : -1;
    const bool vec_p = (T & 3) == 0 && (reinterpret_cast<uintptr_t>(P) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(dS) & 15) == 0;

    v4f df[DH / 8];  // dO of this lane's query, score k order
    {
        const float *drow = dO + (row0 + min(qi, T - 1)) * ldo + hc + 4 * lg;
#pragma unroll
        for (int q = 0; q < DH / 8; q++) df[q] = *reinterpret_cast<const v4f *>(drow + 8 * q);
    }
    // V blocks take the score operand's slot (stride KS), K blocks the
    // value operand's (stride VS)
    auto Vs = [&](int u) { return lds + (u & 1) * (TL::KFL + TL::VFL); };
    auto Ks = [&](int u) { return lds + (u & 1) * (TL::KFL + TL::VFL) + TL::KFL; };
    v4f vr[TL::PT], kr[TL::PT];
    const long prow = ((long)bh * T + min(qi, T - 1)) * T;
    // P_ij for this lane's 16 keys of block kb (zero past T)
    auto load_p = [&](const float *X, int kb, float (&x)[16]) {
        // a whole block inside T (wave-uniform; 128-wide heads keep the
        // per-piece form, whose registers they can hold without a spill)
        if (DH <= 64 && vec_p && (kb + 1) * AT_KB <= T) {
            const float *xr = X + prow + kb * AT_KB + 4 * lg;
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const v4f t = *reinterpret_cast<const v4f *>(xr + 8 * g4);
#pragma unroll
                for (int e = 0; e < 4; e++) x[4 * g4 + e] = t[e];
            }
            return;
        }
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            const int j0 = kb * AT_KB + 8 * g4 + 4 * lg;
            if (vec_p && j0 + 3 < T) {
                const v4f t = *reinterpret_cast<const v4f *>(X + prow + j0);
#pragma unroll
                for (int e = 0; e < 4; e++) x[4 * g4 + e] = t[e];
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) x[4 * g4 + e] = j0 + e < T ? X[prow + j0 + e] : 0.f;
            }
        }
    };

    // ---- pass 1: D_i = sum_j P_ij dP_ij (this lane's half of the keys), or,
    // given the forward's output, D_i = dO_i . att_i (the same sum, since
    // att_i = sum_j P_ij v_j) from the lane's half of the row
    float Dsum = 0.f, pn[16];
    if (Ofw) {
        const float *orow = Ofw + (row0 + min(qi, T - 1)) * ldfw + hc + 4 * lg;
#pragma unroll
        for (int q = 0; q < DH / 8; q++) {
            const v4f o = *reinterpret_cast<const v4f *>(orow + 8 * q);
#pragma unroll
            for (int e = 0; e < 4; e++) Dsum += df[q][e] * o[e];
        }
    } else {
        // P rows are fetched one key block ahead of their use (HBM latency is
        // about one block of MFMA work)
        at_load<DH>(vr, V + hc, ld, row0, 0, T, tid);
        if (kbw >= 0) load_p(P, 0, pn);
        at_store<DH, TL::KS>(Vs(0), vr, tid);
        __syncthreads();
        for (int kb = 0; kb <= kb_last; kb++) {
            if (kb < kb_last) at_load<DH>(vr, V + hc, ld, row0, (kb + 1) * AT_KB, T, tid);
            if (kb <= kbw) {
                float pv[16];
#pragma unroll
                for (int v = 0; v < 16; v++) pv[v] = pn[v];
                if (kb < kbw) load_p(P, kb + 1, pn);
                const v16f dp = at_scores<DH>(Vs(kb), df, r32, lg);
#pragma unroll
                for (int v = 0; v < 16; v++) Dsum += pv[v] * dp[v];
            }
            if (kb < kb_last) at_store<DH, TL::KS>(Vs(kb + 1), vr, tid);
            __syncthreads();
        }
    }
    Dsum += __shfl_xor(Dsum, 32);

    // ---- pass 2: dS (stored) and dQ^T += K^T dS^T
    v16f qacc[DH / 32];
#pragma unroll
    for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
        for (int v = 0; v < 16; v++) qacc[nb][v] = 0.f;
    const bool live = qi < T;
    at_load<DH>(vr, V + hc, ld, row0, 0, T, tid);
    at_load<DH>(kr, K + hc, ld, row0, 0, T, tid);
    if (kbw >= 0) load_p(P, 0, pn);
    at_store<DH, TL::KS>(Vs(0), vr, tid);
    at_store<DH, TL::VS>(Ks(0), kr, tid);
    __syncthreads();
    for (int kb = 0; kb <= kb_last; kb++) {
        if (kb < kb_last) {
            at_load<DH>(vr, V + hc, ld, row0, (kb + 1) * AT_KB, T, tid);
            at_load<DH>(kr, K + hc, ld, row0, (kb + 1) * AT_KB, T, tid);
        }
        if (kb <= kbw) {
            float pv[16], ds[16];
#pragma unroll
            for (int v = 0; v < 16; v++) pv[v] = pn[v];
            if (kb < kbw) load_p(P, kb + 1, pn);
            const v16f dp = at_scores<DH>(Vs(kb), df, r32, lg);
            if constexpr (DH > 64) {  // the mask on every block (no spill at 256 registers)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int j = kb * AT_KB + at_key(v, lg);
                    ds[v] = (j <= qi && j < T) ? pv[v] * (dp[v] - Dsum) * scale : 0.f;
                }
            } else {
#pragma unroll
                for (int v = 0; v < 16; v++) ds[v] = pv[v] * (dp[v] - Dsum) * scale;
                if (kb * AT_KB >= q0w || (kb + 1) * AT_KB > T) {  // diagonal or tail block (wave-uniform)
                    const int lim = min(qi, T - 1) - kb * AT_KB;
#pragma unroll
                    for (int v = 0; v < 16; v++) ds[v] = at_key(v, lg) <= lim ? ds[v] : 0.f;
                }
            }
            if (DH <= 64 && live && vec_p && (kb + 1) * AT_KB <= T) {
                float *sr = dS + prow + kb * AT_KB + 4 * lg;
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++)
                    *reinterpret_cast<v4f *>(sr + 8 * g4) = v4f{ds[4 * g4], ds[4 * g4 + 1], ds[4 * g4 + 2], ds[4 * g4 + 3]};
            } else if (live) {
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const int j0 = kb * AT_KB + 8 * g4 + 4 * lg;
                    if (vec_p && j0 + 3 < T) {
                        *reinterpret_cast<v4f *>(dS + prow + j0) =
                            v4f{ds[4 * g4], ds[4 * g4 + 1], ds[4 * g4 + 2], ds[4 * g4 + 3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (j0 + e < T) dS[prow + j0 + e] = ds[4 * g4 + e];
                    }
                }
            }
            at_accum<DH>(qacc, Ks(kb), ds, r32, lg);
        }
        if (kb < kb_last) {
            at_store<DH, TL::KS>(Vs(kb + 1), vr, tid);
            at_store<DH, TL::VS>(Ks(kb + 1), kr, tid);
        }
        __syncthreads();
    }
    if (live) {
        float *grow = dQ + (row0 + qi) * ldg + hc;
#pragma unroll
        for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                float *o = grow + nb * 32 + at_key(v, lg);
                *o = accumulate ? *o + qacc[nb][v] : qacc[nb][v];
            }
    }
}

template <int DH>
__global__ __launch_bounds__(256, 2) void attn_bwd_dkv_kernel(
    const float *__restrict__ dO, long ldo, const float *__restrict__ Q, long ld,
    const float *__restrict__ P, const float *__restrict__ dS, float *__restrict__ dK,
    float *__restrict__ dV, long ldg, int T, int H, int BH, int accumulate) {
    using TL = AttnTile<DH>;
    __shared__ __attribute__((aligned(16))) float lds[2 * 2 * TL::VFL];
    const int tid = threadIdx.x, lane = tid & 63, r32 = lane & 31, lg = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // key block k needs the query blocks from k on: work falls with k, so the
    // first half of the grid takes the light-to-heavy mirror of the forward's
    const int nkb = (T + AT_QB - 1) / AT_QB, half = (nkb + 1) / 2;
    const int L = (int)(blockIdx.x / BH), bh = (int)(blockIdx.x % BH);
    const int kblk = L < half ? L : nkb - 1 - (L - half);
    const int b = bh / H, h = bh % H;
    const long row0 = (long)b * T;
    const int hc = h * DH;
    const int k0 = kblk * AT_QB, k0w = k0 + wave * 32;
    const int kj = k0w + r32;  // this lane's key (its output column)
    const int qb_first = k0 / AT_KB, qb_last = (T - 1) / AT_KB;
    const int qbw = k0w / AT_KB;  // this wave's first query block

    auto Os = [&](int u) { return lds + (u & 1) * 2 * TL::VFL; };
    auto Qs = [&](int u) { return lds + (u & 1) * 2 * TL::VFL + TL::VFL; };
    v4f orr[TL::PT], qr[TL::PT];
    v16f vacc[DH / 32], kacc[DH / 32];
#pragma unroll
    for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
        for (int v = 0; v < 16; v++) vacc[nb][v] = 0.f, kacc[nb][v] = 0.f;
    const float *Pbh = P + (long)bh * T * T, *Sbh = dS + (long)bh * T * T;
    const int kcol = min(kj, T - 1);

    // P and dS of queries qb*32 + key-layout row s4, key kj, fetched one
    // query block ahead of their use. Heads of 32 and 64: rows past T read
    // row T-1 and keys past T key T-1, finite values that meet zero dO / Q
    // rows in LDS or land in output columns that are not stored, so nothing
    // is zeroed, and a block inside T addresses row qb*32 + at_key(s4, lg) as
    // a uniform row base plus the lane's 32-bit offset. 128-wide heads keep
    // the per-element clamp and zero (the other form's addresses spill there).
    float pn[16], sn[16];
    const unsigned lane_off = (unsigned)(4 * lg * T + kcol);
    auto load_ps = [&](int qb) {
        if constexpr (DH > 64) {
#pragma unroll
            for (int s4 = 0; s4 < 16; s4++) {
                const int i = qb * AT_KB + at_key(s4, lg);
                const long o = (long)min(i, T - 1) * T + kcol;
                const bool ok = i < T && kj < T;
                pn[s4] = ok ? Pbh[o] : 0.f;
                sn[s4] = ok ? Sbh[o] : 0.f;
            }
        } else if ((qb + 1) * AT_KB <= T) {
            const float *pr = Pbh + (long)qb * AT_KB * T, *sr = Sbh + (long)qb * AT_KB * T;
#pragma unroll
            for (int s4 = 0; s4 < 16; s4++) {
                const long ro = (long)(8 * (s4 >> 2) + (s4 & 3)) * T;
                pn[s4] = (pr + ro)[lane_off];
                sn[s4] = (sr + ro)[lane_off];
            }
        } else {
#pragma unroll
            for (int s4 = 0; s4 < 16; s4++) {
                const long o = (long)min(qb * AT_KB + at_key(s4, lg), T - 1) * T + kcol;
                pn[s4] = Pbh[o];
                sn[s4] = Sbh[o];
            }
        }
    };
    at_load<DH>(orr, dO + hc, ldo, row0, qb_first * AT_KB, T, tid);
    at_load<DH>(qr, Q + hc, ld, row0, qb_first * AT_KB, T, tid);
    if (k0w < T) load_ps(max(qb_first, qbw));
    at_store<DH, TL::VS>(Os(0), orr, tid);
    at_store<DH, TL::VS>(Qs(0), qr, tid);
    __syncthreads();
    for (int qb = qb_first; qb <= qb_last; qb++) {
        const int u = qb - qb_first;
        if (qb < qb_last) {
            at_load<DH>(orr, dO + hc, ldo, row0, (qb + 1) * AT_KB, T, tid);
            at_load<DH>(qr, Q + hc, ld, row0, (qb + 1) * AT_KB, T, tid);
        }
        if (k0w < T && qb >= qbw) {
            float pv[16], sv[16];
#pragma unroll
            for (int s4 = 0; s4 < 16; s4++) pv[s4] = pn[s4], sv[s4] = sn[s4];
            if (qb < qb_last) load_ps(qb + 1);
            if (qb == qbw) {  // the diagonal block: queries before the key take nothing
#pragma unroll
                for (int s4 = 0; s4 < 16; s4++)
                    if (qb * AT_KB + at_key(s4, lg) < kj) pv[s4] = 0.f, sv[s4] = 0.f;
            }
            at_accum<DH>(vacc, Os(u), pv, r32, lg);
            at_accum<DH>(kacc, Qs(u), sv, r32, lg);
        }
        if (qb < qb_last) {
            at_store<DH, TL::VS>(Os(u + 1), orr, tid);
            at_store<DH, TL::VS>(Qs(u + 1), qr, tid);
        }
        __syncthreads();
    }
    if (kj < T) {
        float *vrow = dV + (row0 + kj) * ldg + hc, *krow = dK + (row0 + kj) * ldg + hc;
#pragma unroll
        for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int d = nb * 32 + at_key(v, lg);
                vrow[d] = accumulate ? vrow[d] + vacc[nb][v] : vacc[nb][v];
                krow[d] = accumulate ? krow[d] + kacc[nb][v] : kacc[nb][v];
            }
    }
}

hipError_t launch_attn_bwd(const float *dO, long ldo, const float *Q, const float *K,
                           const float *V, long ld, const float *P, float *dS, float *dQ,
                           float *dK, float *dV, long ldg, int B, int T, int H, int dh,
                           float scale, int accumulate, hipStream_t stream, const float *Ofw,
                           long ldfw) {
    const int BH = B * H, nb = (T + AT_QB - 1) / AT_QB;
    if (BH == 0 || T == 0) return hipSuccess;
    const dim3 grid((unsigned)((long)nb * BH)), block(256);
#define PCL_ATTN_BWD(D)                                                                            \
    hipLaunchKernelGGL(attn_bwd_dq_kernel<D>, grid, block, 0, stream, dO, ldo, K, V, ld, P, dS, dQ,  \
                       ldg, T, H, BH, scale, accumulate, Ofw, ldfw);                               \
    hipLaunchKernelGGL(attn_bwd_dkv_kernel<D>, grid, block, 0, stream, dO, ldo, Q, ld, P, dS, dK, dV, \
                       ldg, T, H, BH, accumulate)
    switch (dh) {
        case 32: PCL_ATTN_BWD(32); break;
        case 64: PCL_ATTN_BWD(64); break;
        case 128: PCL_ATTN_BWD(128); break;
        default: return hipErrorInvalidValue;
    }
#undef PCL_ATTN_BWD
    return hipGetLastError();
}

hipError_t launch_attn_fwd(const float *Q, const float *K, const float *V, long ld, float *O,
                           long ldo, float *P, int B, int T, int H, int dh, float scale,
                           hipStream_t stream, float *lse) {
    const int BH = B * H, nqb = (T + AT_QB - 1) / AT_QB;
    if (BH == 0 || T == 0) return hipSuccess;
    const dim3 grid((unsigned)((long)nqb * BH)), block(256);
    if (P == nullptr) {  // no probabilities: one pass
        switch (dh) {
            case 32:
                hipLaunchKernelGGL((attn_fwd_online_kernel<32, 2>), grid, block, 0, stream, Q, K, V, ld, O, ldo, lse, T, H, BH, scale);
                break;
            case 64:
                hipLaunchKernelGGL((attn_fwd_online_kernel<64, 2>), grid, block, 0, stream, Q, K, V, ld, O, ldo, lse, T, H, BH, scale);
                break;
            case 128:
                hipLaunchKernelGGL((attn_fwd_online_kernel<128, 1>), grid, block, 0, stream, Q, K, V, ld, O, ldo, lse, T, H, BH, scale);
                break;
            default:
                return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (lse) return hipErrorInvalidValue;
    switch (dh) {
        case 32:
            hipLaunchKernelGGL(attn_fwd_kernel<32>, grid, block, 0, stream, Q, K, V, ld, O, ldo, P, T, H, BH, scale);
            break;
        case 64:
            hipLaunchKernelGGL(attn_fwd_kernel<64>, grid, block, 0, stream, Q, K, V, ld, O, ldo, P, T, H, BH, scale);
            break;
        case 128:
            hipLaunchKernelGGL(attn_fwd_kernel<128>, grid, block, 0, stream, Q, K, V, ld, O, ldo, P, T, H, BH, scale);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace pcl
