// decode.hip -- the non-GEMV kernels of one KV-cached decode step
// (generate.c:118-183): token + position embedding, attention of the new
// token over the cache (appending its k, v), the INT8 step's LayerNorm /
// GELU + quantisation kernels for rows too long for the fused GEMV, and a
// greedy argmax that writes the next token and advances the position. (The
// fp32 step's LayerNorm and GELU run inside the GEMVs, gemv.hip.)
//
// The token and position live in device memory (tokpos[0], tokpos[1]), so a
// whole step -- these kernels and the GEMVs between them -- can be captured
// once as a graph and replayed token after token with no host round trip.
#include "internal.h"

#include <math.h>

namespace pcl {

// x = wte[tok] + wpe[pos]   (generate.c:172-175)
__global__ void dec_embed_kernel(const float *__restrict__ wte, const float *__restrict__ wpe,
                                 float *__restrict__ x, int D, const int *__restrict__ tokpos) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= D) return;
    const long tok = tokpos[0], pos = tokpos[1];
    x[i] = wte[tok * D + i] + wpe[pos * D + i];
}

// A wave's maximum (any values) or sum in its last lane, on the DPP network:
// row_shr 1, 2, 4, 8 within rows of 16 lanes, then row_bcast 15 and 31 across
// rows. For the maximum a lane with no source keeps its own value; for the
// sum it adds 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dec_dpp_keep(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWS, 0xF, false));
}
template <int CTRL, int ROWS>
__device__ __forceinline__ float dec_dpp_zero(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, true));
}
// v + the value of lane ^ 16 (v_permlane16_swap exchanges the odd rows of one
// copy with the even rows of the other) and v + lane ^ 32 (permlane32_swap):
// the sums of a shuffle butterfly, as VALU operations.
__device__ __forceinline__ float dec_swap16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float dec_swap32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float dec_wave_max_last(float v) {
    v = fmaxf(v, dec_dpp_keep<0x111, 0xF>(v));
    v = fmaxf(v, dec_dpp_keep<0x112, 0xF>(v));
    v = fmaxf(v, dec_dpp_keep<0x114, 0xF>(v));
    v = fmaxf(v, dec_dpp_keep<0x118, 0xF>(v));
    v = fmaxf(v, dec_dpp_keep<0x142, 0xA>(v));
    return fmaxf(v, dec_dpp_keep<0x143, 0xC>(v));
}
__device__ __forceinline__ float dec_wave_sum_last(float v) {
    v += dec_dpp_zero<0x111, 0xF>(v);
    v += dec_dpp_zero<0x112, 0xF>(v);
    v += dec_dpp_zero<0x114, 0xF>(v);
    v += dec_dpp_zero<0x118, 0xF>(v);
    v += dec_dpp_zero<0x142, 0xA>(v);
    return v + dec_dpp_zero<0x143, 0xC>(v);
}

// Block-wide sum of one value per thread (256 threads, 4 waves).
__device__ __forceinline__ float dec_block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}


// One head per workgroup (generate.c:130-152): append this position's k, v to
// the cache, scores s_j = (q . k_j) * scale for j <= pos (the new row from
// LDS, older rows from the cache), softmax, att = sum_j p_j v_j. qkv holds
// [q | k | v] (3*D floats) and bqkv, when given, is added to it here (the
// INT8 step's projections carry no bias); the cache rows are D floats. dh
// divides 256. DHT > 0: the head size at compile time, cache rows read as
// 16-byte vectors (D % 4 == 0, 16-byte aligned cache); DHT == 0: any head
// size, scalar reads. p . v: with DHT > 0 thread t owns 4 columns (t mod
// DHT/4) of every (256 / (DHT/4))-th key, and issues the 16-byte loads of 8
// of its keys together, the first 8 before the scores (they depend on the
// position only), so at the grown model's head size (32) and a block of 256
// every V row the sum needs arrives under the scores and the softmax; each
// thread sums its keys in order, the key groups of a wave are added by
// shuffles and the four waves in order. DHT == 0: thread (column, key group),
// 8 keys per load batch.
template <int DHT>
__global__ __launch_bounds__(256) void dec_attn_kernel(const float *__restrict__ qkv,
                                                       const float *__restrict__ bqkv,
                                                       float *__restrict__ kc,
                                                       float *__restrict__ vc,
                                                       float *__restrict__ att, int D, int dh_rt,
                                                       const int *__restrict__ tokpos,
                                                       float scale) {
    extern __shared__ __attribute__((aligned(16))) float dec_lds[];  // [blk] scores, then partial sums
    __shared__ float red[4], red2[4], qs[256], ks[256];
    __shared__ __attribute__((aligned(16))) float vs[256];
    const int dh = DHT > 0 ? DHT : dh_rt;
    const int h = blockIdx.x, tid = threadIdx.x, off = h * dh;
    const int pos = tokpos[1];
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    // The new token's q, k, v (+ bias) load first: the staging barrier waits
    // for them, and a load issued later does not hold up that wait. Then, for
    // DHT > 0, the cache rows this thread reads first, which depend on pos
    // only: the first batch of its V rows and key row tid (if tid < pos).
    // (the pointers are materialised first, so the row loads do not wait for
    // the scalar load of pos)
    const float *qkv_p = qkv, *bqkv_p = bqkv;
    asm volatile("" : "+s"(qkv_p), "+s"(bqkv_p));
    float nq = 0.f, nk = 0.f, nv = 0.f, bq = 0.f, bk = 0.f, bv = 0.f;
    if (tid < dh) {  // global (not flat) loads: a flat load would also count in the wait for pos
        const auto qg = gbl(qkv_p);
        nq = qg[off + tid], nk = qg[D + off + tid], nv = qg[2 * D + off + tid];
        if (bqkv_p) {
            const auto bg = gbl(bqkv_p);
            bq = bg[off + tid], bk = bg[D + off + tid], bv = bg[2 * D + off + tid];
        }
    }
    constexpr int PVL = DHT > 0 ? DHT / 4 : 1, PVG = 256 / PVL;  // lanes per V row, key groups
    v4f_t vpre[8], kpre[DHT > 0 ? DHT / 4 : 1];
    if constexpr (DHT > 0) {
        const float *vrow = vc + off + 4 * (tid % PVL);
#pragma unroll
        for (int u = 0; u < 8; u++) {  // rows past pos (and row pos) read row 0 and add nothing
            const int j = tid / PVL + u * PVG;
            vpre[u] = *reinterpret_cast<const v4f_t *>(vrow + (long)(j < pos ? j : 0) * D);
        }
        const v4f_t *kj = reinterpret_cast<const v4f_t *>(kc + (long)(tid < pos ? tid : 0) * D + off);
#pragma unroll
        for (int c = 0; c < DHT / 4; c++) kpre[c] = kj[c];
    }
    if (tid < dh) {
        nq += bq, nk += bk, nv += bv;
        qs[tid] = nq;
        ks[tid] = nk;
        vs[tid] = nv;
        kc[(long)pos * D + off + tid] = nk;
        vc[(long)pos * D + off + tid] = nv;
    }
    __syncthreads();
    const float *q = qs, *knew = ks, *vnew = vs;
    float *sc = dec_lds;
    float mloc = -INFINITY;
    for (int j = tid; j <= pos; j += 256) {
        float dot = 0.f;
        if (j == pos) {
            for (int d = 0; d < dh; d++) dot += q[d] * knew[d];
        } else if constexpr (DHT > 0) {
            const v4f_t *kj = reinterpret_cast<const v4f_t *>(kc + (long)j * D + off);
            v4f_t kv[DHT / 4];
#pragma unroll
            for (int c = 0; c < DHT / 4; c++) kv[c] = j == tid ? kpre[c] : kj[c];
#pragma unroll
            for (int c = 0; c < DHT / 4; c++) {
                dot += q[4 * c] * kv[c][0];
                dot += q[4 * c + 1] * kv[c][1];
                dot += q[4 * c + 2] * kv[c][2];
                dot += q[4 * c + 3] * kv[c][3];
            }
        } else {
            const float *kj = kc + (long)j * D + off;
            for (int d = 0; d < dh; d++) dot += q[d] * kj[d];
        }
        dot *= scale;
        sc[j] = dot;
        mloc = fmaxf(mloc, dot);
    }
    // block max: each wave's in its last lane (DPP), then the four waves
    mloc = dec_wave_max_last(mloc);
    if ((tid & 63) == 63) red[tid >> 6] = mloc;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sloc = 0.f;
    for (int j = tid; j <= pos; j += 256) {
        const float e = expf(sc[j] - m);
        sc[j] = e;
        sloc += e;
    }
    // block sum the same way (its barrier also orders the sc[] writes)
    sloc = dec_wave_sum_last(sloc);
    if ((tid & 63) == 63) red2[tid >> 6] = sloc;
    __syncthreads();
    const float inv = 1.0f / (((red2[0] + red2[1]) + red2[2]) + red2[3]);
    float *part = dec_lds + ((pos + 1 + 3) & ~3);
    if constexpr (DHT > 0) {
        constexpr int L = PVL, KG = PVG;
        const int d4 = tid % L, kg = tid / L;
        const float *vrow = vc + off + 4 * d4;
        v4f_t acc = {0.f, 0.f, 0.f, 0.f};
        for (int j0 = kg; j0 <= pos; j0 += 8 * KG) {
            v4f_t v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {  // rows past pos read row 0 and add nothing
                const int j = j0 + u * KG;
                v[u] = j0 == kg ? vpre[u] : *reinterpret_cast<const v4f_t *>(vrow + (long)(j < pos ? j : 0) * D);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int j = j0 + u * KG;
                if (j <= pos) {
                    const float p = sc[j] * inv;
                    const v4f_t vv = j == pos ? *reinterpret_cast<const v4f_t *>(vnew + 4 * d4) : v[u];
                    acc[0] += p * vv[0];
                    acc[1] += p * vv[1];
                    acc[2] += p * vv[2];
                    acc[3] += p * vv[3];
                }
            }
        }
        // the 64 / L key groups of a wave added by shuffles (lane bits above
        // the column's), then the four waves' sums in wave order
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float a = acc[c];
            if constexpr (L == 8) a += dec_dpp_zero<0x128, 0xF>(a);  // row_ror:8 = lane ^ 8
            if constexpr (L <= 16) a = dec_swap16_sum(a);
            if constexpr (L <= 32) a = dec_swap32_sum(a);
            acc[c] = a;
        }
        if ((tid & 63) < L) *reinterpret_cast<v4f_t *>(part + (tid >> 6) * DHT + 4 * d4) = acc;
        __syncthreads();
        if (tid < DHT) att[off + tid] = ((part[tid] + part[DHT + tid]) + part[2 * DHT + tid]) + part[3 * DHT + tid];
    } else {
        // output: thread t owns column d = t % dh of key group t / dh
        const int G = 256 / dh, d = tid % dh, gq = tid / dh;
        float acc = 0.f;
        if (gq < G) {
            const float *vcol = vc + off + d;
            int j = gq;
            for (; j + 7 * G < pos; j += 8 * G) {  // 8 cache rows, none of them row pos
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) v[u] = vcol[(long)(j + u * G) * D];
#pragma unroll
                for (int u = 0; u < 8; u++) acc += sc[j + u * G] * inv * v[u];
            }
            for (; j <= pos; j += G) acc += sc[j] * inv * (j == pos ? vnew[d] : vcol[(long)j * D]);
        }
        part[tid] = acc;
        __syncthreads();
        if (tid < dh) {
            float o = 0.f;
            for (int g2 = 0; g2 < G; g2++) o += part[g2 * dh + tid];
            att[off + tid] = o;
        }
    }
}

// One step of a (value, index) maximum across lanes on the DPP network: the
// larger value wins, equal values the smaller index (so the order of the
// steps does not matter); a lane with no source, or outside ROWS, keeps its
// own pair. NaN never wins.
template <int CTRL, int ROWS>
__device__ __forceinline__ void dec_amax_step(float &best, int &idx) {
    const float ov = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(best), __float_as_int(best), CTRL, ROWS, 0xF, false));
    const int oi = __builtin_amdgcn_update_dpp(idx, idx, CTRL, ROWS, 0xF, false);
    if (ov > best || (ov == best && oi < idx)) best = ov, idx = oi;
}
// the pair of a row of 16 lanes (rows of 16, then W = 64 lanes) in its last lane
template <int W>
__device__ __forceinline__ void dec_amax_last(float &best, int &idx) {
    dec_amax_step<0x111, 0xF>(best, idx);  // row_shr:1, 2, 4, 8
    dec_amax_step<0x112, 0xF>(best, idx);
    dec_amax_step<0x114, 0xF>(best, idx);
    dec_amax_step<0x118, 0xF>(best, idx);
    if constexpr (W >= 32) dec_amax_step<0x142, 0xA>(best, idx);  // row_bcast:15
    if constexpr (W >= 64) dec_amax_step<0x143, 0xC>(best, idx);  // row_bcast:31
}

// Greedy pick (generate.c:188-191: the first index of the maximum), written
// as the next token; the position advances and out[pos + 1] records it. 1024
// threads read the logits in batches of four loads each (one memory latency
// per 4096 logits), each wave's pair lands in its last lane, and wave 0 picks
// among the 16 waves' pairs.
__global__ __launch_bounds__(1024) void dec_argmax_kernel(const float *__restrict__ logits, int V,
                                                          int *__restrict__ tokpos,
                                                          int *__restrict__ out, int out_cap) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const int tid = threadIdx.x;
    const int pos = tokpos[1];
    float best = -INFINITY;
    int idx = V;
    for (int i0 = tid; i0 < V; i0 += 4096) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = i0 + 1024 * u < V ? logits[i0 + 1024 * u] : -INFINITY;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + 1024 * u;
            if (i < V && (v[u] > best || (v[u] == best && i < idx))) best = v[u], idx = i;
        }
    }
    dec_amax_last<64>(best, idx);
    if ((tid & 63) == 63) bv[tid >> 6] = best, bi[tid >> 6] = idx;
    __syncthreads();
    if (tid < 16) {
        best = bv[tid], idx = bi[tid];
        dec_amax_last<16>(best, idx);
        if (tid == 15) {
            if (idx >= V) idx = 0;  // all NaN: keep a valid token
            tokpos[0] = idx;
            if (pos + 1 < out_cap) out[pos + 1] = idx;
            tokpos[1] = pos + 1;
        }
    }
}

hipError_t launch_decode_embed(const float *wte, const float *wpe, float *x, int D,
                               const int *tokpos, hipStream_t s) {
    hipLaunchKernelGGL(dec_embed_kernel, dim3((D + 255) / 256), dim3(256), 0, s, wte, wpe, x, D,
                       tokpos);
    return hipGetLastError();
}
hipError_t launch_decode_attn(const float *qkv, const float *bqkv, float *kc, float *vc, float *att,
                              int D, int H, int blk, const int *tokpos, hipStream_t s) {
    const int dh = D / H;
    if (dh <= 0 || 256 % dh != 0) return hipErrorInvalidValue;
    const size_t lds = sizeof(float) * ((size_t)((blk + 3) & ~3) + 1024);  // scores, then 256 x 4 partials
    const float scale = 1.0f / sqrtf((float)dh);
    const bool vec = D % 4 == 0 && ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & 15) == 0;
    if (vec && dh == 32)
        hipLaunchKernelGGL(dec_attn_kernel<32>, dim3(H), dim3(256), lds, s, qkv, bqkv, kc, vc, att, D,
                           dh, tokpos, scale);
    else if (vec && dh == 64)
        hipLaunchKernelGGL(dec_attn_kernel<64>, dim3(H), dim3(256), lds, s, qkv, bqkv, kc, vc, att, D,
                           dh, tokpos, scale);
    else if (vec && dh == 128)
        hipLaunchKernelGGL(dec_attn_kernel<128>, dim3(H), dim3(256), lds, s, qkv, bqkv, kc, vc, att, D,
                           dh, tokpos, scale);
    else
        hipLaunchKernelGGL(dec_attn_kernel<0>, dim3(H), dim3(256), lds, s, qkv, bqkv, kc, vc, att, D,
                           dh, tokpos, scale);
    return hipGetLastError();
}

// ---- INT8 step: quantised activations (the per-row rule of quant.hip) ----
// Per-row quantisation of the n values in v (LDS) into q (Kpad bytes, 128 past
// n) with its scale, by one workgroup.
__device__ void dec_quant_row(const float *v, int n, uint8_t *__restrict__ q, int Kpad,
                              float *__restrict__ sa, float *red) {
    float mx = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, fabsf(v[i]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float amax = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), AMAX_INIT);
    const float scale = amax * RCP127, inv = 1.0f / scale;
    if (threadIdx.x == 0) *sa = scale;
    for (int k = threadIdx.x; k < Kpad; k += 256) q[k] = (uint8_t)((k < n ? quant_q(v[k], inv) : 0) + 128);
}

// x += t + b (the pending residual: t = the previous product without its bias
// b; skipped when t is NULL), then y = LayerNorm(x) quantised per row
// (generate.c:106-114 and :155/166's additions, then the INT8 operand).
__global__ __launch_bounds__(256) void dec_add_ln_quant_kernel(
    float *__restrict__ x, const float *__restrict__ t, const float *__restrict__ b,
    const float *__restrict__ g, const float *__restrict__ beta, uint8_t *__restrict__ q,
    float *__restrict__ sa, int D, int Kpad) {
    extern __shared__ float dec_lds[];  // [D]
    __shared__ float red[4];
    float s = 0.f;
    for (int i = threadIdx.x; i < D; i += 256) {
        float v = x[i];
        if (t) {
            v = v + (t[i] + b[i]);
            x[i] = v;
        }
        dec_lds[i] = v;
        s += v;
    }
    const float mu = dec_block_sum(s, red) / D;
    float qq = 0.f;
    for (int i = threadIdx.x; i < D; i += 256) {
        const float d = dec_lds[i] - mu;
        qq += d * d;
    }
    const float var = dec_block_sum(qq, red) / D;
    const float rs = 1.0f / sqrtf(var + 1e-5f);
    for (int i = threadIdx.x; i < D; i += 256) dec_lds[i] = (dec_lds[i] - mu) * rs * g[i] + beta[i];
    dec_quant_row(dec_lds, D, q, Kpad, sa, red);
}

// y = gelu(h + b) quantised per row (generate.c:159-164 after the W1 product).
__global__ __launch_bounds__(256) void dec_bias_gelu_quant_kernel(const float *__restrict__ h,
                                                                  const float *__restrict__ b,
                                                                  uint8_t *__restrict__ q,
                                                                  float *__restrict__ sa, int F,
                                                                  int Kpad) {
    extern __shared__ float dec_lds[];  // [F]
    __shared__ float red[4];
    for (int i = threadIdx.x; i < F; i += 256) {
        const float v = h[i] + b[i];
        dec_lds[i] = 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
    }
    dec_quant_row(dec_lds, F, q, Kpad, sa, red);
}

hipError_t launch_decode_add_ln_quant(float *x, const float *t, const float *b, const float *g,
                                      const float *beta, uint8_t *q, float *sa, int D, int Kpad,
                                      hipStream_t s) {
    hipLaunchKernelGGL(dec_add_ln_quant_kernel, dim3(1), dim3(256), sizeof(float) * (size_t)D, s, x,
                       t, b, g, beta, q, sa, D, Kpad);
    return hipGetLastError();
}
hipError_t launch_decode_bias_gelu_quant(const float *h, const float *b, uint8_t *q, float *sa,
                                         int F, int Kpad, hipStream_t s) {
    hipLaunchKernelGGL(dec_bias_gelu_quant_kernel, dim3(1), dim3(256), sizeof(float) * (size_t)F, s,
                       h, b, q, sa, F, Kpad);
    return hipGetLastError();
}
hipError_t launch_decode_argmax(const float *logits, int V, int *tokpos, int *out, int out_cap,
                                hipStream_t s) {
    hipLaunchKernelGGL(dec_argmax_kernel, dim3(1), dim3(1024), 0, s, logits, V, tokpos, out, out_cap);
    return hipGetLastError();
}

}  // namespace pcl
