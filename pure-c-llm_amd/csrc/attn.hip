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
// the normalised p (the reference's order: p = exp(s - max) / sum, then
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

// S^T block (keys x queries) of this wave: A = K rows from LDS (16-byte piece
// 8q + 4lg of row r32, element e at MFMA step 4q + e), B = the wave's Q in the
// same k order (registers).
template <int DH>
__device__ __forceinline__ v16f at_scores(const float *Ks, const v4f (&qf)[DH / 8], int r32, int lg) {
    v16f s;
#pragma unroll
    for (int v = 0; v < 16; v++) s[v] = 0.f;
    const float *krow = Ks + r32 * AttnTile<DH>::KS + 4 * lg;
#pragma unroll
    for (int q = 0; q < DH / 8; q++) {
        const v4f kf = *reinterpret_cast<const v4f *>(krow + 8 * q);
#pragma unroll
        for (int e = 0; e < 4; e++) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[e], qf[q][e], s, 0, 0, 0);
    }
    return s;
}

// key offset (within the block) of accumulator element v for lane half lg
__device__ __forceinline__ constexpr int at_key(int v, int lg) { return (v >> 2) * 8 + lg * 4 + (v & 3); }

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
    // heaviest query blocks first (causal work grows with the query index)
    const int nqb = (T + AT_QB - 1) / AT_QB;
    const int qblk = nqb - 1 - (int)(blockIdx.x / BH), bh = (int)(blockIdx.x % BH);
    const int b = bh / H, h = bh % H;
    const long row0 = (long)b * T;  // first token row of this sequence
    const int hc = h * DH;          // first column of this head
    const int q0 = qblk * AT_QB, q0w = q0 + wave * 32;
    const int qi = q0w + r32;              // this lane's query
    const int qlast = min(T - 1, q0 + AT_QB - 1);
    const int kb_last = qlast / AT_KB;     // last key block of the workgroup
    const int kbw = q0w < T ? min(T - 1, q0w + 31) / AT_KB : -1;  // last key block of this wave

    v4f qf[DH / 8];
    {
        const float *qrow = Q + (row0 + min(qi, T - 1)) * ld + hc + 4 * lg;
#pragma unroll
        for (int q = 0; q < DH / 8; q++) qf[q] = *reinterpret_cast<const v4f *>(qrow + 8 * q);
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
            float x[16], bm = -INFINITY;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int j = kb * AT_KB + at_key(v, lg);
                x[v] = (j <= qi && j < T) ? s[v] * scale : -INFINITY;
                bm = fmaxf(bm, x[v]);
            }
            const float mn = fmaxf(m, bm);
            if (mn != -INFINITY) {
                float acc = 0.f;
#pragma unroll
                for (int v = 0; v < 16; v++) acc += __expf(x[v] - mn);
                l = l * __expf(m - mn) + acc;
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
        const float lt = (m == -INFINITY ? 0.f : l * __expf(m - mx)) +
                         (mo == -INFINITY ? 0.f : lo * __expf(mo - mx));
        m = mx;
        l = lt;
    }
    const float inv = 1.f / l;

    // ---- pass 2: normalised probabilities, stored if asked, and O^T += V^T P^T
    v16f oacc[DH / 32];
#pragma unroll
    for (int nb = 0; nb < DH / 32; nb++)
#pragma unroll
        for (int v = 0; v < 16; v++) oacc[nb][v] = 0.f;
    const bool store_p = P != nullptr && qi < T;
    float *prow = store_p ? P + ((long)bh * T + qi) * T : nullptr;
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
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int j = kb * AT_KB + at_key(v, lg);
                p[v] = (j <= qi && j < T) ? __expf(s[v] * scale - m) * inv : 0.f;
                if (store_p && j < T) prow[j] = p[v];
            }
            const float *vcol = Vb(kb) + r32;
#pragma unroll
            for (int s4 = 0; s4 < 16; s4++) {
                const float *vrow = vcol + at_key(s4, lg) * TL::VS;
#pragma unroll
                for (int nb = 0; nb < DH / 32; nb++)
                    oacc[nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[nb * 32], p[s4], oacc[nb], 0, 0, 0);
            }
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

hipError_t launch_attn_fwd(const float *Q, const float *K, const float *V, long ld, float *O,
                           long ldo, float *P, int B, int T, int H, int dh, float scale,
                           hipStream_t stream) {
    const int BH = B * H, nqb = (T + AT_QB - 1) / AT_QB;
    if (BH == 0 || T == 0) return hipSuccess;
    const dim3 grid((unsigned)((long)nqb * BH)), block(256);
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
