// model.cpp -- a CKP1 checkpoint on the GPU and its KV-cached greedy decode.
//
// The checkpoint (train.c:633-670 writes it, generate.c:49-76 reads it): an
// int[8] header {magic 'CKP1', block, d_model, n_heads, d_ff, n_layers, vocab,
// step} followed by every tensor's floats in registration order: wte (V x D),
// wpe (block x D), per layer g1, b1, Wq, bq, Wk, bk, Wv, bv, Wo, bo, g2, b2,
// W1 (D x FF), bff1, W2 (FF x D), bff2, then gf, bf. It is read once into one
// device arena (weights, KV cache, per-token state); Wq, Wk, Wv are joined
// column-wise into one D x 3D matrix so the three projections are one GEMV.
//
// One decode step is generate.c's forward(tok, pos) (:118-183): embedding,
// per layer LayerNorm -> QKV GEMV -> attention over the cache -> O GEMV added
// into x -> LayerNorm -> FF1 GEMV -> GELU -> FF2 GEMV added into x, then the
// final LayerNorm, the tied-head GEMV and a greedy argmax. The token and
// position live in device memory and the argmax advances them, so a step is
// captured once as a graph and replayed per generated token.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <algorithm>
#include <new>
#include <vector>

#include "../../include/pcl_hip.h"
#include "internal.h"

namespace {

constexpr int CKP1_MAGIC = 0x434B5031;

struct Layer {
    float *g1, *b1, *wqkv, *bqkv, *wo, *bo, *g2, *b2, *w1, *bf1, *w2, *bf2, *kc, *vc;
};
// INT8 projections: packed s8 (rows of Kp bytes per output column) + scales
struct QLayer {
    int8_t *wqkv, *wo, *w1, *w2;
    float *sqkv, *so, *s1, *s2;
};
int kpad256(int k) { return (k + 255) / 256 * 256; }

int fail(int status, const char *msg) { return pcl::shim_error(status, msg); }

}  // namespace

struct pcl_model {
    int hdr[8];
    int blk, d, h, df, nl, v;
    float *arena = nullptr;
    int *ints = nullptr;  // tokpos[2], then out[blk + 1]
    int *host_tp = nullptr;  // pinned: {token, position} per position, copied to tokpos
    float *wte, *wpe, *gf, *bf;
    std::vector<Layer> lay;
    float *x, *qkv, *att, *hh, *logits;
    void *stream = nullptr;
    void *graph = nullptr;
    // INT8 weights (PCL_W_INT8): projections and the tied head quantised once
    int wmode = PCL_W_FP32;
    int kpd = 0, kpf = 0;
    int8_t *i8 = nullptr;
    float *qscale = nullptr;  // weight scales, a D-float product, the activation scale
    std::vector<QLayer> ql;
    int8_t *whead = nullptr;
    float *shead = nullptr, *sa = nullptr, *tmp = nullptr;
    uint8_t *xq = nullptr;
    // verification tap (pcl_model_capture): one slot per INT8 product,
    // written by the eager steps of pcl_model_forward while tap_on
    unsigned char *tap = nullptr;
    bool tap_on = false;
    long tap_km = 0, tap_nm = 0, tap_kpm = 0;
};

namespace {

#define M_HIP(call)                                                        \
    do {                                                                   \
        hipError_t e_ = (call);                                            \
        if (e_ != hipSuccess) {                                            \
            char b_[256];                                                  \
            snprintf(b_, sizeof b_, "%s: %s", #call, hipGetErrorString(e_)); \
            return fail(PCL_ERR_HIP, b_);                                  \
        }                                                                  \
    } while (0)
#define M_OK(expr)                  \
    do {                            \
        int s_ = (expr);            \
        if (s_ != PCL_OK) return s_; \
    } while (0)

// A tap slot: the product's input row before its transform (K floats), its
// dequantised output before bias and residual (N floats), the row's scale,
// and the quantised row (Kp bytes). Products 0-3 of layer l are QKV, O, FF1,
// FF2; layer n_layers holds the head.
struct TapSlot {
    float *xin, *y, *sa;
    uint8_t *xq;
};
long tap_slot_bytes(const pcl_model *m) {
    return 4 * (m->tap_km + m->tap_nm + 4) + (m->tap_kpm + 15) / 16 * 16;
}
TapSlot tap_slot(const pcl_model *m, int l, int p) {
    unsigned char *b = m->tap + (size_t)(l * 4 + p) * (size_t)tap_slot_bytes(m);
    float *f = reinterpret_cast<float *>(b);
    return TapSlot{f, f + m->tap_km, f + m->tap_km + m->tap_nm,
                   reinterpret_cast<uint8_t *>(f + m->tap_km + m->tap_nm + 4)};
}
// Fused products: record the input row, and aim the kernel's own tap at the
// slot (it writes the quantised row, its scale and the product).
int tap_fused(pcl_model *m, int l, int p, const float *x, int K, pcl::GemvTap *t) {
    if (!m->tap_on) return PCL_OK;
    const TapSlot sl = tap_slot(m, l, p);
    M_HIP(hipMemcpyAsync(sl.xin, x, sizeof(float) * (size_t)K, hipMemcpyDeviceToDevice,
                         (hipStream_t)m->stream));
    *t = pcl::GemvTap{sl.xq, sl.sa, sl.y};
    return PCL_OK;
}
// Unfused products: the input row, the quantised row and scale the GEMV reads
// (m->xq, m->sa), then its output.
int tap_row(pcl_model *m, int l, int p, const float *x, int K, int Kp) {
    if (!m->tap_on) return PCL_OK;
    const TapSlot sl = tap_slot(m, l, p);
    hipStream_t s = (hipStream_t)m->stream;
    M_HIP(hipMemcpyAsync(sl.xin, x, sizeof(float) * (size_t)K, hipMemcpyDeviceToDevice, s));
    M_HIP(hipMemcpyAsync(sl.xq, m->xq, (size_t)Kp, hipMemcpyDeviceToDevice, s));
    M_HIP(hipMemcpyAsync(sl.sa, m->sa, sizeof(float), hipMemcpyDeviceToDevice, s));
    return PCL_OK;
}
int tap_out(pcl_model *m, int l, int p, const float *y, int N) {
    if (!m->tap_on) return PCL_OK;
    M_HIP(hipMemcpyAsync(tap_slot(m, l, p).y, y, sizeof(float) * (size_t)N, hipMemcpyDeviceToDevice,
                         (hipStream_t)m->stream));
    return PCL_OK;
}

// The fp32 step over the N x K projections. Each product is one sgemv_q
// launch that makes its input row (LayerNorm, or bias + GELU) and, for Wo and
// W2, adds product + bias into x: five launches per layer. Dims the kernel
// does not take (K % 4 != 0 or beyond its LDS row) use the transposed-weight
// GEMV with the same transforms instead.
int step(pcl_model *m) {
    hipStream_t s = (hipStream_t)m->stream;
    const int D = m->d, F = m->df, V = m->v;
    int *tokpos = m->ints, *out = m->ints + 2;
    M_HIP(pcl::launch_decode_embed(m->wte, m->wpe, m->x, D, tokpos, s));
    const bool fused = D % 4 == 0 && F % 4 == 0 && D <= pcl::SGEMV_Q_MAX_K && F <= pcl::SGEMV_Q_MAX_K;
    for (const Layer &y : m->lay) {
        if (fused) {
            M_HIP(pcl::launch_sgemv_q(1, 0, m->x, y.g1, y.b1, D, y.wqkv, y.bqkv, m->qkv, 3 * D, s));
            M_HIP(pcl::launch_decode_attn(m->qkv, nullptr, y.kc, y.vc, m->att, D, m->h, m->blk, tokpos, s));
            M_HIP(pcl::launch_sgemv_q(0, 1, m->att, nullptr, nullptr, D, y.wo, y.bo, m->x, D, s));
            M_HIP(pcl::launch_sgemv_q(1, 0, m->x, y.g2, y.b2, D, y.w1, nullptr, m->hh, F, s));
            M_HIP(pcl::launch_sgemv_q(2, 1, m->hh, nullptr, y.bf1, F, y.w2, y.bf2, m->x, D, s));
        } else {
            M_OK(pcl::sgemv_xf(1, 3 * D, D, m->x, y.wqkv, D, y.g1, y.b1, y.bqkv, 0, m->qkv, s));
            M_HIP(pcl::launch_decode_attn(m->qkv, nullptr, y.kc, y.vc, m->att, D, m->h, m->blk, tokpos, s));
            M_OK(pcl::sgemv_xf(0, D, D, m->att, y.wo, D, nullptr, nullptr, y.bo, 1, m->x, s));
            M_OK(pcl::sgemv_xf(1, F, D, m->x, y.w1, D, y.g2, y.b2, y.bf1, 0, m->hh, s));
            M_OK(pcl::sgemv_xf(2, D, F, m->hh, y.w2, F, nullptr, nullptr, y.bf2, 1, m->x, s));
        }
    }
    if (fused)
        M_HIP(pcl::launch_sgemv_q(1, 0, m->x, m->gf, m->bf, D, m->wte, nullptr, m->logits, V, s));
    else
        M_OK(pcl::sgemv_xf(1, V, D, m->x, m->wte, D, m->gf, m->bf, nullptr, 0, m->logits, s));
    M_HIP(pcl::launch_decode_argmax(m->logits, V, tokpos, out, m->blk + 1, s));
    return PCL_OK;
}

// The same step with INT8 products: each product's input row is quantised per
// row (u8 + scale, 0x80 past its length up to Kp) by the kernel that makes it,
// the GEMV dequantises (sa * sb), and the bias -- plus the residual add -- is
// applied by the next kernel (the QKV bias inside the attention kernel).
int step_int8(pcl_model *m) {
    hipStream_t s = (hipStream_t)m->stream;
    const int D = m->d, F = m->df, V = m->v, KD = m->kpd, KF = m->kpf;
    int *tokpos = m->ints, *out = m->ints + 2;
    M_HIP(pcl::launch_decode_embed(m->wte, m->wpe, m->x, D, tokpos, s));
    const float *t = nullptr, *tb = nullptr;  // pending product and its bias, added into x
    const int L = (int)m->lay.size();
    for (int l = 0; l < L; l++) {
        const Layer &y = m->lay[(size_t)l];
        const QLayer &q = m->ql[(size_t)l];
        M_HIP(pcl::launch_decode_add_ln_quant(m->x, t, tb, y.g1, y.b1, m->xq, m->sa, D, KD, s));
        M_OK(tap_row(m, l, 0, m->x, D, KD));
        M_OK(pcl_gemv_u8s8_dq(m->xq, KD, q.wqkv, nullptr, m->sa, q.sqkv, m->qkv, 3 * D, 1, 3 * D, KD, s));
        M_OK(tap_out(m, l, 0, m->qkv, 3 * D));
        M_HIP(pcl::launch_decode_attn(m->qkv, y.bqkv, y.kc, y.vc, m->att, D, m->h, m->blk, tokpos, s));
        M_HIP(pcl::launch_quantize_a_rows(m->att, 1, D, m->xq, KD, m->sa, s));
        M_OK(tap_row(m, l, 1, m->att, D, KD));
        M_OK(pcl_gemv_u8s8_dq(m->xq, KD, q.wo, nullptr, m->sa, q.so, m->tmp, D, 1, D, KD, s));
        M_OK(tap_out(m, l, 1, m->tmp, D));
        M_HIP(pcl::launch_decode_add_ln_quant(m->x, m->tmp, y.bo, y.g2, y.b2, m->xq, m->sa, D, KD, s));
        M_OK(tap_row(m, l, 2, m->x, D, KD));
        M_OK(pcl_gemv_u8s8_dq(m->xq, KD, q.w1, nullptr, m->sa, q.s1, m->hh, F, 1, F, KD, s));
        M_OK(tap_out(m, l, 2, m->hh, F));
        M_HIP(pcl::launch_decode_bias_gelu_quant(m->hh, y.bf1, m->xq, m->sa, F, KF, s));
        M_OK(tap_row(m, l, 3, m->hh, F, KF));
        M_OK(pcl_gemv_u8s8_dq(m->xq, KF, q.w2, nullptr, m->sa, q.s2, m->tmp, D, 1, D, KF, s));
        M_OK(tap_out(m, l, 3, m->tmp, D));
        t = m->tmp, tb = y.bf2;
    }
    M_HIP(pcl::launch_decode_add_ln_quant(m->x, t, tb, m->gf, m->bf, m->xq, m->sa, D, KD, s));
    M_OK(tap_row(m, L, 0, m->x, D, KD));
    M_OK(pcl_gemv_u8s8_dq(m->xq, KD, m->whead, nullptr, m->sa, m->shead, m->logits, V, 1, V, KD, s));
    M_OK(tap_out(m, L, 0, m->logits, V));
    M_HIP(pcl::launch_decode_argmax(m->logits, V, tokpos, out, m->blk + 1, s));
    return PCL_OK;
}

// The INT8 step with the transform and the quantisation of each product's
// input done by the GEMV itself (launch_igemv_q), and the Wo / W2 products
// added with their biases straight into x: five launches per layer.
int step_int8_fused(pcl_model *m) {
    hipStream_t s = (hipStream_t)m->stream;
    const int D = m->d, F = m->df, V = m->v, KD = m->kpd, KF = m->kpf;
    int *tokpos = m->ints, *out = m->ints + 2;
    M_HIP(pcl::launch_decode_embed(m->wte, m->wpe, m->x, D, tokpos, s));
    const int L = (int)m->lay.size();
    pcl::GemvTap tp[4], th;  // stay null unless the tap is on
    for (int l = 0; l < L; l++) {
        const Layer &y = m->lay[(size_t)l];
        const QLayer &q = m->ql[(size_t)l];
        M_OK(tap_fused(m, l, 0, m->x, D, &tp[0]));
        M_HIP(pcl::launch_igemv_q(1, 0, m->x, y.g1, y.b1, D, q.wqkv, KD, q.sqkv, nullptr, m->qkv, 3 * D, s, tp[0]));
        M_HIP(pcl::launch_decode_attn(m->qkv, y.bqkv, y.kc, y.vc, m->att, D, m->h, m->blk, tokpos, s));
        M_OK(tap_fused(m, l, 1, m->att, D, &tp[1]));
        M_HIP(pcl::launch_igemv_q(0, 1, m->att, nullptr, nullptr, D, q.wo, KD, q.so, y.bo, m->x, D, s, tp[1]));
        M_OK(tap_fused(m, l, 2, m->x, D, &tp[2]));
        M_HIP(pcl::launch_igemv_q(1, 0, m->x, y.g2, y.b2, D, q.w1, KD, q.s1, nullptr, m->hh, F, s, tp[2]));
        M_OK(tap_fused(m, l, 3, m->hh, F, &tp[3]));
        M_HIP(pcl::launch_igemv_q(2, 1, m->hh, nullptr, y.bf1, F, q.w2, KF, q.s2, y.bf2, m->x, D, s, tp[3]));
    }
    M_OK(tap_fused(m, L, 0, m->x, D, &th));
    M_HIP(pcl::launch_igemv_q(1, 0, m->x, m->gf, m->bf, D, m->whead, KD, m->shead, nullptr, m->logits, V, s, th));
    M_HIP(pcl::launch_decode_argmax(m->logits, V, tokpos, out, m->blk + 1, s));
    return PCL_OK;
}

int run_eager(pcl_model *m) {
    if (m->wmode != PCL_W_INT8) return step(m);
    return m->kpd <= pcl::IGEMV_Q_MAX_K && m->kpf <= pcl::IGEMV_Q_MAX_K ? step_int8_fused(m)
                                                                          : step_int8(m);
}

// Quantise every projection (per output column) and the tied head once.
int quantize_weights(pcl_model *m) {
    const long D = m->d, F = m->df, V = m->v;
    if (F > 32768)  // bias + GELU + quantisation keeps a d_ff row in LDS
        return fail(PCL_ERR_INVALID_ARG, "pcl_model_load: INT8 weights need d_ff <= 32768");
    const int KD = kpad256((int)D), KF = kpad256((int)F);
    m->kpd = KD, m->kpf = KF;
    const long per = 3 * D * KD + D * KD + F * KD + D * KF;
    const long bytes = m->nl * per + V * KD;
    const long scales = m->nl * (3 * D + D + F + D) + V + 1 + D;
    M_HIP(hipMalloc((void **)&m->i8, (size_t)bytes));
    M_HIP(hipMalloc((void **)&m->qscale, sizeof(float) * (size_t)scales));
    M_HIP(hipMalloc((void **)&m->xq, (size_t)(KD > KF ? KD : KF)));
    hipStream_t s = (hipStream_t)m->stream;
    int8_t *b = m->i8;
    float *sc = m->qscale;
    m->ql.resize(m->lay.size());
    for (size_t l = 0; l < m->lay.size(); l++) {
        const Layer &y = m->lay[l];
        QLayer &q = m->ql[l];
        q.wqkv = b, b += 3 * D * KD;
        q.wo = b, b += D * KD;
        q.w1 = b, b += F * KD;
        q.w2 = b, b += D * KF;
        q.sqkv = sc, sc += 3 * D;
        q.so = sc, sc += D;
        q.s1 = sc, sc += F;
        q.s2 = sc, sc += D;
        M_HIP(pcl::launch_quantize_b_cols(y.wqkv, (int)D, (int)(3 * D), 0, q.wqkv, KD, KD, q.sqkv, nullptr, s));
        M_HIP(pcl::launch_quantize_b_cols(y.wo, (int)D, (int)D, 0, q.wo, KD, KD, q.so, nullptr, s));
        M_HIP(pcl::launch_quantize_b_cols(y.w1, (int)D, (int)F, 0, q.w1, KD, KD, q.s1, nullptr, s));
        M_HIP(pcl::launch_quantize_b_cols(y.w2, (int)F, (int)D, 0, q.w2, KF, KF, q.s2, nullptr, s));
    }
    m->whead = b;
    m->shead = sc, sc += V;
    m->tmp = sc, sc += D;
    m->sa = sc;
    // the head quantises wte per vocabulary row: its transpose (D x V) is the
    // K x N operand of the per-column rule
    float *wt = nullptr;
    M_HIP(hipMalloc((void **)&wt, sizeof(float) * (size_t)(V * D)));
    std::vector<float> h((size_t)(V * D)), ht((size_t)(V * D));
    M_HIP(hipMemcpy(h.data(), m->wte, sizeof(float) * (size_t)(V * D), hipMemcpyDeviceToHost));
    for (long v = 0; v < V; v++)
        for (long d = 0; d < D; d++) ht[(size_t)(d * V + v)] = h[(size_t)(v * D + d)];
    int st = PCL_OK;
    if (hipMemcpy(wt, ht.data(), sizeof(float) * (size_t)(V * D), hipMemcpyHostToDevice) != hipSuccess ||
        pcl::launch_quantize_b_cols(wt, (int)D, (int)V, 0, m->whead, KD, KD, m->shead, nullptr, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        st = fail(PCL_ERR_HIP, "pcl_model_load: INT8 weight quantisation failed");
    (void)hipFree(wt);
    if (st == PCL_OK) m->wmode = PCL_W_INT8;
    return st;
}

// Each position has its own pinned slot, so a copy still queued on the stream
// never reads a slot rewritten for a later position (callers synchronise the
// stream before positions repeat).
int set_tokpos(pcl_model *m, int tok, int pos) {
    int *tp = m->host_tp + 2 * pos;
    tp[0] = tok;
    tp[1] = pos;
    M_HIP(hipMemcpyAsync(m->ints, tp, 2 * sizeof(int), hipMemcpyHostToDevice, (hipStream_t)m->stream));
    return PCL_OK;
}

// nk: store the projections N x K (a row of K floats per output), the layout
// the fp32 decode GEMVs read; otherwise K x N as in the file (the INT8
// quantiser's input).
int load(pcl_model *m, const char *path, bool nk) {
    FILE *f = fopen(path, "rb");
    if (!f) return fail(PCL_ERR_INVALID_ARG, "pcl_model_load: cannot open the checkpoint");
    std::vector<float> w;
    int st = PCL_OK;
    do {
        if (fread(m->hdr, sizeof(int), 8, f) != 8 || m->hdr[0] != CKP1_MAGIC) {
            st = fail(PCL_ERR_INVALID_ARG, "pcl_model_load: not a CKP1 checkpoint");
            break;
        }
        m->blk = m->hdr[1], m->d = m->hdr[2], m->h = m->hdr[3], m->df = m->hdr[4];
        m->nl = m->hdr[5], m->v = m->hdr[6];
        const int dh = m->h > 0 ? m->d / m->h : 0;
        if (m->blk <= 0 || m->d <= 0 || m->h <= 0 || m->df <= 0 || m->nl <= 0 || m->v <= 0 ||
            m->d % m->h != 0 || 256 % dh != 0 || (long)m->d * m->df > (1L << 30) ||
            (long)m->v * m->d > (1L << 30) || m->blk > 32768 || m->d > 32768) {
            // the cache attention keeps a block of scores, and the INT8 LayerNorm
            // a row, in LDS (160 KB per workgroup)
            st = fail(PCL_ERR_INVALID_ARG,
                      "pcl_model_load: unsupported dims (head size must divide 256; block and "
                      "d_model at most 32768)");
            break;
        }
        const long D = m->d, F = m->df;
        const long per_layer = 2 * D + 3 * (D * D + D) + (D * D + D) + 2 * D + (D * F + F) + (F * D + D);
        // the header's float count must match what the file holds, checked
        // before anything is sized from it (a corrupt n_layers would
        // otherwise ask for an arbitrary allocation)
        long file_floats = -1;
        const long here = ftell(f);
        if (here >= 0 && fseek(f, 0, SEEK_END) == 0) {
            const long end = ftell(f);
            if (end >= here) file_floats = (end - here) / (long)sizeof(float);
            if (fseek(f, here, SEEK_SET) != 0) file_floats = -1;
        }
        if (m->nl > (1 << 20) || file_floats < 0) {
            st = fail(PCL_ERR_INVALID_ARG, "pcl_model_load: unreadable checkpoint size");
            break;
        }
        const long n = (long)m->v * D + (long)m->blk * D + m->nl * per_layer + 2 * D;
        if (n > file_floats) {
            st = fail(PCL_ERR_INVALID_ARG, "pcl_model_load: short read in the checkpoint");
            break;
        }
        try {
            w.resize((size_t)n);
        } catch (const std::bad_alloc &) {
            st = fail(PCL_ERR_OOM, "pcl_model_load: out of host memory");
            break;
        }
        if (fread(w.data(), sizeof(float), (size_t)n, f) != (size_t)n) {
            st = fail(PCL_ERR_INVALID_ARG, "pcl_model_load: short read in the checkpoint");
            break;
        }
    } while (0);
    fclose(f);
    if (st != PCL_OK) return st;

    const long D = m->d, F = m->df, V = m->v, BLK = m->blk;
    // device layout: weights (QKV joined), KV caches, per-token state
    const long per_layer_dev = 2 * D + (3 * D * D + 3 * D) + (D * D + D) + 2 * D + (D * F + F) +
                               (F * D + D) + 2 * BLK * D;
    const long state = D + 3 * D + D + F + V;  // x, qkv, att, hh, logits
    const long total = V * D + BLK * D + m->nl * per_layer_dev + 2 * D + state;
    std::vector<float> h((size_t)total);
    const float *src = w.data();
    float *dst = h.data();
    long at = 0;
    auto take = [&](long cnt) {  // copy cnt floats from the file stream, return the device offset
        const long o = at;
        memcpy(dst + at, src, sizeof(float) * cnt);
        src += cnt;
        at += cnt;
        return o;
    };
    const long o_wte = take(V * D), o_wpe = take(BLK * D);
    struct LOff { long g1, b1, wqkv, bqkv, wo, bo, g2, b2, w1, bf1, w2, bf2, kc, vc; };
    std::vector<LOff> lo((size_t)m->nl);
    for (int l = 0; l < m->nl; l++) {
        LOff &y = lo[(size_t)l];
        y.g1 = take(D), y.b1 = take(D);
        // Wq, bq, Wk, bk, Wv, bv -> [Wq | Wk | Wv] (D x 3D) and [bq | bk | bv]
        y.wqkv = at;
        at += 3 * D * D;
        y.bqkv = at;
        at += 3 * D;
        for (int part = 0; part < 3; part++) {
            if (nk) {  // rows part*D + c of the joined matrix's transpose
                for (long k = 0; k < D; k++)
                    for (long c = 0; c < D; c++) dst[y.wqkv + (part * D + c) * D + k] = src[k * D + c];
            } else {
                for (long k = 0; k < D; k++)
                    memcpy(dst + y.wqkv + k * 3 * D + part * D, src + k * D, sizeof(float) * D);
            }
            src += D * D;
            memcpy(dst + y.bqkv + part * D, src, sizeof(float) * D);
            src += D;
        }
        auto take_w = [&](long K, long N) {  // a K x N matrix, transposed when nk
            if (!nk) return take(K * N);
            const long o = at;
            for (long k = 0; k < K; k++)
                for (long n = 0; n < N; n++) dst[o + n * K + k] = src[k * N + n];
            src += K * N;
            at += K * N;
            return o;
        };
        y.wo = take_w(D, D), y.bo = take(D);
        y.g2 = take(D), y.b2 = take(D);
        y.w1 = take_w(D, F), y.bf1 = take(F);
        y.w2 = take_w(F, D), y.bf2 = take(D);
        y.kc = at;
        at += BLK * D;
        y.vc = at;
        at += BLK * D;
    }
    const long o_gf = take(D), o_bf = take(D);
    const long o_state = at;
    at += state;
    if (at != total || src != w.data() + w.size())
        return fail(PCL_ERR_INVALID_ARG, "pcl_model_load: internal layout mismatch");
    memset(dst + o_state, 0, sizeof(float) * state);
    for (int l = 0; l < m->nl; l++)
        memset(dst + lo[(size_t)l].kc, 0, sizeof(float) * 2 * BLK * D);

    M_HIP(hipMalloc((void **)&m->arena, sizeof(float) * (size_t)total));
    M_HIP(hipMalloc((void **)&m->ints, sizeof(int) * (size_t)(BLK + 3)));
    M_HIP(hipMemcpy(m->arena, h.data(), sizeof(float) * (size_t)total, hipMemcpyHostToDevice));
    M_HIP(hipMemset(m->ints, 0, sizeof(int) * (size_t)(BLK + 3)));
    M_HIP(hipHostMalloc((void **)&m->host_tp, sizeof(int) * 2 * (size_t)BLK, hipHostMallocDefault));
    float *a = m->arena;
    m->wte = a + o_wte, m->wpe = a + o_wpe, m->gf = a + o_gf, m->bf = a + o_bf;
    m->lay.resize((size_t)m->nl);
    for (int l = 0; l < m->nl; l++) {
        const LOff &y = lo[(size_t)l];
        m->lay[(size_t)l] = Layer{a + y.g1, a + y.b1, a + y.wqkv, a + y.bqkv, a + y.wo,
                                  a + y.bo, a + y.g2, a + y.b2, a + y.w1, a + y.bf1,
                                  a + y.w2, a + y.bf2, a + y.kc, a + y.vc};
    }
    float *sp = a + o_state;
    m->x = sp, sp += D;
    m->qkv = sp, sp += 3 * D;
    m->att = sp, sp += D;
    m->hh = sp, sp += F;
    m->logits = sp;
    m->stream = pcl_stream_create();
    if (!m->stream) return pcl_last_status();
    return PCL_OK;
}

void release(pcl_model *m) {
    if (m->graph) pcl_graph_destroy(m->graph);
    if (m->stream) pcl_stream_destroy(m->stream);
    if (m->arena) (void)hipFree(m->arena);
    if (m->i8) (void)hipFree(m->i8);
    if (m->qscale) (void)hipFree(m->qscale);
    if (m->xq) (void)hipFree(m->xq);
    if (m->tap) (void)hipFree(m->tap);
    if (m->ints) (void)hipFree(m->ints);
    if (m->host_tp) (void)hipHostFree(m->host_tp);
    delete m;
}

// run one step on the model's stream, as a replay of the captured step when
// use_graph (capturing it the first time)
int run_step(pcl_model *m, int use_graph) {
    if (!use_graph) return run_eager(m);
    void *prev = pcl_get_stream();
    int st = PCL_OK;
    pcl_set_stream(m->stream);
    if (!m->graph) {
        st = pcl_graph_begin();
        if (st == PCL_OK) {
            const int s1 = run_eager(m);
            void *g = nullptr;
            const int s2 = pcl_graph_end(&g);
            st = s1 != PCL_OK ? s1 : s2;
            if (st == PCL_OK) m->graph = g;
            else if (g) pcl_graph_destroy(g);
        }
    }
    if (st == PCL_OK) st = pcl_graph_launch(m->graph);
    pcl_set_stream(prev);
    return st;
}

}  // namespace

extern "C" {

pcl_model *pcl_model_load_ex(const char *path, int weights) {
    if (!path) {
        fail(PCL_ERR_INVALID_ARG, "pcl_model_load: path is NULL");
        return nullptr;
    }
    if (weights != PCL_W_FP32 && weights != PCL_W_INT8) {
        fail(PCL_ERR_INVALID_ARG, "pcl_model_load: weights must be PCL_W_FP32 or PCL_W_INT8");
        return nullptr;
    }
    if (pcl::shim_init() != PCL_OK) return nullptr;
    pcl_model *m = new (std::nothrow) pcl_model();
    if (!m) {
        fail(PCL_ERR_OOM, "pcl_model_load: out of host memory");
        return nullptr;
    }
    int lst;
    try {  // host staging vectors: no exception crosses the C ABI
        lst = load(m, path, weights == PCL_W_FP32);
        if (lst == PCL_OK && weights == PCL_W_INT8) lst = quantize_weights(m);
    } catch (const std::bad_alloc &) {
        lst = fail(PCL_ERR_OOM, "pcl_model_load: out of host memory");
    }
    if (lst != PCL_OK) {
        const int st = pcl_last_status();
        char msg[512];
        snprintf(msg, sizeof msg, "%s", pcl_last_error());
        release(m);
        fail(st, msg);
        return nullptr;
    }
    return m;
}

pcl_model *pcl_model_load(const char *path) { return pcl_model_load_ex(path, PCL_W_FP32); }

int pcl_model_header(const pcl_model *m, int hdr[8]) {
    if (!m || !hdr) return fail(PCL_ERR_INVALID_ARG, "pcl_model_header: NULL argument");
    memcpy(hdr, m->hdr, sizeof m->hdr);
    return PCL_OK;
}

int pcl_model_forward(pcl_model *m, int tok, int pos, float *logits) {
    if (!m) return fail(PCL_ERR_INVALID_ARG, "pcl_model_forward: model is NULL");
    if (tok < 0 || tok >= m->v || pos < 0 || pos >= m->blk)
        return fail(PCL_ERR_INVALID_ARG, "pcl_model_forward: token or position out of range");
    M_OK(set_tokpos(m, tok, pos));
    m->tap_on = m->tap != nullptr;
    const int st = run_eager(m);
    m->tap_on = false;
    M_OK(st);
    if (logits)
        M_HIP(hipMemcpyAsync(logits, m->logits, sizeof(float) * (size_t)m->v, hipMemcpyDeviceToHost,
                             (hipStream_t)m->stream));
    M_HIP(hipStreamSynchronize((hipStream_t)m->stream));
    return PCL_OK;
}

int pcl_model_generate(pcl_model *m, const int *prompt, int n_prompt, int n_new, int *out,
                       int use_graph) {
    if (!m || !prompt || (n_new > 0 && !out))
        return fail(PCL_ERR_INVALID_ARG, "pcl_model_generate: NULL argument");
    // Positions fed: 0 .. n_prompt-1 for the prompt, then n_prompt .. n_prompt+n_new-2;
    // each must be below block (cache rows, wpe rows, pinned token slots).
    if (n_prompt < 1 || n_new < 0 || n_prompt > m->blk || (long)n_prompt + n_new - 1 > m->blk)
        return fail(PCL_ERR_INVALID_ARG,
                    "pcl_model_generate: need 1 <= n_prompt <= block and n_prompt + n_new - 1 <= block");
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= m->v)
            return fail(PCL_ERR_INVALID_ARG, "pcl_model_generate: prompt token out of range");
    for (int i = 0; i < n_prompt; i++) {
        M_OK(set_tokpos(m, prompt[i], i));
        M_OK(run_eager(m));
    }
    // the last prompt step left the first new token and position n_prompt in
    // device memory; each further step feeds the previous pick
    for (int t = 1; t < n_new; t++) M_OK(run_step(m, use_graph));
    if (n_new > 0)
        M_HIP(hipMemcpyAsync(out, m->ints + 2 + n_prompt, sizeof(int) * (size_t)n_new,
                             hipMemcpyDeviceToHost, (hipStream_t)m->stream));
    M_HIP(hipStreamSynchronize((hipStream_t)m->stream));
    return PCL_OK;
}

void pcl_model_free(pcl_model *m) {
    if (m) release(m);
}

int pcl_model_capture(pcl_model *m, int on) {
    if (!m) return fail(PCL_ERR_INVALID_ARG, "pcl_model_capture: model is NULL");
    if (m->wmode != PCL_W_INT8)
        return fail(PCL_ERR_INVALID_ARG, "pcl_model_capture: the model has no INT8 products");
    if (!on) {
        if (m->tap) {
            M_HIP(hipStreamSynchronize((hipStream_t)m->stream));
            M_HIP(hipFree(m->tap));
        }
        m->tap = nullptr;
        return PCL_OK;
    }
    if (m->tap) return PCL_OK;
    const long D = m->d, F = m->df, V = m->v;
    m->tap_km = D > F ? D : F;
    m->tap_nm = std::max(std::max(3 * D, F), V);
    m->tap_kpm = m->kpd > m->kpf ? m->kpd : m->kpf;
    const size_t bytes = (size_t)(4 * m->nl + 1) * (size_t)tap_slot_bytes(m);
    M_HIP(hipMalloc((void **)&m->tap, bytes));
    M_HIP(hipMemset(m->tap, 0, bytes));
    return PCL_OK;
}

int pcl_model_capture_read(const pcl_model *m, int layer, int product, float *xin, uint8_t *xq,
                           float *sa, float *y) {
    if (!m || !m->tap)
        return fail(PCL_ERR_INVALID_ARG, "pcl_model_capture_read: no capture on this model");
    if (layer < 0 || layer > m->nl || product < 0 || product > 3 || (layer == m->nl && product != 0))
        return fail(PCL_ERR_INVALID_ARG, "pcl_model_capture_read: no such product");
    const long D = m->d, F = m->df;
    long K = D, N = D;
    if (layer == m->nl) N = m->v;
    else if (product == 0) N = 3 * D;
    else if (product == 2) N = F;
    else if (product == 3) K = F;
    const long Kp = K == D ? m->kpd : m->kpf;
    const TapSlot sl = tap_slot(m, layer, product);
    M_HIP(hipStreamSynchronize((hipStream_t)m->stream));
    if (xin) M_HIP(hipMemcpy(xin, sl.xin, sizeof(float) * (size_t)K, hipMemcpyDeviceToHost));
    if (xq) M_HIP(hipMemcpy(xq, sl.xq, (size_t)Kp, hipMemcpyDeviceToHost));
    if (sa) M_HIP(hipMemcpy(sa, sl.sa, sizeof(float), hipMemcpyDeviceToHost));
    if (y) M_HIP(hipMemcpy(y, sl.y, sizeof(float) * (size_t)N, hipMemcpyDeviceToHost));
    return PCL_OK;
}

}  // extern "C"
