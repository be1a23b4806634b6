/*
 * pcl_oracle.c -- CPU restatement of pure-c-llm's matrix-multiply hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): see pcl_oracle.h.
 * Reference citations are file:line into the pure-c-llm repository.
 *
 * Pinning (how each function is checked independently of this file):
 *   orc_matmul_ikj / naive ...... tensor.c:204-241 closed-form KAT (C[0,0]=0.07
 *                                 and the full closed-form matrix), identity and
 *                                 ones-matrix invariants, the reference's own
 *                                 tensor.c matmul built from source (oracle/_ref)
 *   orc_gemm_f64 / nn / nt / tn . brute-force identities ((AB)^T = B^T A^T links
 *                                 the three layouts), A=I, K=0, accumulate=twice
 *   orc_matmul_backward, tied_* . train.c built from source (oracle/_ref) at small
 *                                 dims, plus f64 transposition identities
 *   orc_quantize_*, VNNI pack ... gemm_bench.c built from source (oracle/_ref):
 *                                 byte-exact comparison of Au, Bp, scales, colsum
 *   orc_gemm_u8s8_i32 ........... exact int64 brute force; the VNNI identity
 *                                 sum Au*Bq - 128*colsum = sum (Au-128)*Bq checked
 *                                 against the reference gemm_int8_kernel output
 *   orc_dequant ................. bit-exact against gemm_bench.c's float output
 *   orc_gelu_forward / _backward  train.c built from source (oracle/_ref); the
 *                                 exact erf GELU within the tanh approximation's
 *                                 error; the derivative against central
 *                                 differences of the forward
 *   orc_cross_entropy ........... train.c built from source (oracle/_ref): loss and
 *                                 d_logits; closed forms (uniform logits give
 *                                 log V and (1/V - onehot)/M; rows of d_logits sum
 *                                 to zero; a constant added to a row changes
 *                                 nothing); the loss against an f64 log-sum-exp
 *   orc_head_ce ................. the pinned tied head and cross-entropy in the
 *                                 trainer's order; d_lnf and dwte against central
 *                                 differences of the f64 loss
 *   orc_model_forward_int8 ..... no counterpart in the reference: composed of the
 *                                 pinned quantisers, exact int GEMM and dequant
 *                                 below; against generate.c built from source
 *                                 within the quantisation error (< 5% normwise)
 *   orc_model_load / _forward .. generate.c (with tokenizer.c) built from source
 *                                 (oracle/_ref) on written checkpoints: logits
 *                                 token by token; T = 1 and equal-key closed forms
 *                                 through the attention above
 *   orc_attention_forward / _backward
 *                                 train.c built from source (oracle/_ref) at two
 *                                 head sizes (16 and 64); closed forms (T = 1 gives
 *                                 att = v; equal keys give uniform p and running
 *                                 means of v); probability rows sum to one; the
 *                                 backward against central differences of the
 *                                 f64 forward
 */
#include "pcl_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif

/* ---------------------------------------------------------------- PRNG ---- */
static uint32_t seed_or_default(uint32_t seed) { return seed ? seed : 0x9E3779B9u; }

uint32_t orc_xorshift32(uint32_t *s) {
    /* train.c:75 / model.c:120-122 */
    uint32_t x = *s;
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    *s = x;
    return x;
}

static float unit24(uint32_t x) { return (float)(x & 0x00FFFFFFu) / (float)0x01000000; }

void orc_fill_frand(float *p, size_t n, uint32_t seed, float scale) {
    uint32_t s = seed_or_default(seed);
    for (size_t i = 0; i < n; i++) {
        float u = unit24(orc_xorshift32(&s));
        p[i] = (u * 2.0f - 1.0f) * scale; /* train.c:76-77 */
    }
}

void orc_fill_uniform(float *p, size_t n, uint32_t seed, float lo, float hi) {
    uint32_t s = seed_or_default(seed);
    for (size_t i = 0; i < n; i++) p[i] = lo + (hi - lo) * unit24(orc_xorshift32(&s));
}

void orc_fill_normal(float *p, size_t n, uint32_t seed, float mean, float std) {
    uint32_t s = seed_or_default(seed);
    for (size_t i = 0; i < n; i++) {
        double u1 = ((double)(orc_xorshift32(&s) & 0x00FFFFFFu) + 0.5) / 16777216.0;
        double u2 = (double)(orc_xorshift32(&s) & 0x00FFFFFFu) / 16777216.0;
        double z = sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2);
        p[i] = (float)(mean + std * z);
    }
}

void orc_fill_u8(uint8_t *p, size_t n, uint32_t seed) {
    uint32_t s = seed_or_default(seed);
    for (size_t i = 0; i < n; i++) p[i] = (uint8_t)((orc_xorshift32(&s) >> 16) & 0xFFu);
}

void orc_fill_s8(int8_t *p, size_t n, uint32_t seed) {
    uint32_t s = seed_or_default(seed);
    for (size_t i = 0; i < n; i++) p[i] = (int8_t)(uint8_t)((orc_xorshift32(&s) >> 16) & 0xFFu);
}

void orc_fill_kat_tensor(float *A, size_t na, float *B, size_t nb) {
    /* tensor.c:204-205 (int index i, so the pattern restarts per element index) */
    for (size_t i = 0; i < na; i++) A[i] = (float)((int)(i % 13) - 6) * 0.1f;
    for (size_t i = 0; i < nb; i++) B[i] = (float)((int)(i % 7) - 3) * 0.1f;
}

/* ---------------------------------------------------- FP32 GEMM family ---- */
void orc_matmul_ikj(const float *A, const float *B, float *C, int M, int K, int N) {
    /* tensor.c:34-53 */
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++) {
        float *crow = C + (size_t)i * N;
        for (int j = 0; j < N; j++) crow[j] = 0.0f;
        for (int k = 0; k < K; k++) {
            const float a = A[(size_t)i * K + k];
            const float *brow = B + (size_t)k * N;
            for (int j = 0; j < N; j++) crow[j] += a * brow[j];
        }
    }
}

void orc_matmul_naive(const float *A, const float *B, float *C, int M, int K, int N) {
    /* gemm_bench.c:60-67 */
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc += A[(size_t)i * K + k] * B[(size_t)k * N + j];
            C[(size_t)i * N + j] = acc;
        }
}

void orc_gemm_f64(const float *A, long sam, long sak, const float *B, long sbk, long sbn,
                  const float *bias, float *C, long ldc, int M, int N, int K, int accum) {
    double *row = NULL;
#pragma omp parallel private(row)
    {
        row = (double *)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
#pragma omp for schedule(static)
        for (int m = 0; m < M; m++) {
            for (int n = 0; n < N; n++) row[n] = 0.0;
            for (int k = 0; k < K; k++) {
                double a = (double)A[(long)m * sam + (long)k * sak];
                const float *bk = B + (long)k * sbk;
                if (sbn == 1) {
                    for (int n = 0; n < N; n++) row[n] += a * (double)bk[n];
                } else {
                    for (int n = 0; n < N; n++) row[n] += a * (double)bk[(long)n * sbn];
                }
            }
            float *c = C + (long)m * ldc;
            for (int n = 0; n < N; n++) {
                double v = row[n];
                if (bias) v += (double)bias[n];
                if (accum) v += (double)c[n];
                c[n] = (float)v;
            }
        }
        free(row);
    }
}

void orc_gemm_nn(const float *A, const float *B, const float *bias, float *C, int M, int K, int N) {
    /* gpu_kernels.h:44, gpu_kernels.cu:112-120 */
    orc_gemm_f64(A, K, 1, B, N, 1, bias, C, N, M, N, K, 0);
}

void orc_gemm_nt(const float *A, const float *B, float *C, int M, int K, int N, int accum) {
    /* gpu_kernels.h:45, gpu_kernels.cu:122-129: B is (N,K) row-major */
    orc_gemm_f64(A, K, 1, B, 1, K, NULL, C, N, M, N, K, accum);
}

void orc_gemm_tn(const float *A, const float *B, float *C, int M, int K, int N) {
    /* gpu_kernels.h:46, gpu_kernels.cu:131-138: C(K,N) += A(M,K)^T B(M,N) */
    orc_gemm_f64(A, 1, K, B, N, 1, NULL, C, N, K, N, M, 1);
}

void orc_bias_bwd(float *db, const float *dY, int M, int N) {
    /* gpu_kernels.cu:102-108 */
    for (int n = 0; n < N; n++) {
        float s = 0.0f;
        for (int m = 0; m < M; m++) s += dY[(size_t)m * N + n];
        db[n] += s;
    }
}

void orc_matmul_forward(float *out, const float *in, const float *W, const float *bias,
                        int M, int K, int N) {
    /* train.c:181-211, the i-k-j branch (:192-203) and the bias pass (:204-210) */
    orc_matmul_ikj(in, W, out, M, K, N);
    if (bias)
        for (int m = 0; m < M; m++) {
            float *o = out + (size_t)m * N;
            for (int n = 0; n < N; n++) o[n] += bias[n];
        }
}

void orc_matmul_backward(const float *dY, const float *X, const float *W, float *dX,
                         float *dW, float *db, int M, int K, int N) {
    /* train.c:219-252 */
    if (dX) {
#pragma omp parallel for schedule(static)
        for (int m = 0; m < M; m++) {
            const float *dy = dY + (size_t)m * N;
            float *dx = dX + (size_t)m * K;
            for (int k = 0; k < K; k++) {
                const float *wr = W + (size_t)k * N;
                float s = 0.0f;
                for (int n = 0; n < N; n++) s += dy[n] * wr[n];
                dx[k] += s;
            }
        }
    }
    if (dW) {
#pragma omp parallel for schedule(static)
        for (int k = 0; k < K; k++) {
            float *dwr = dW + (size_t)k * N;
            for (int m = 0; m < M; m++) {
                float a = X[(size_t)m * K + k];
                const float *dy = dY + (size_t)m * N;
                for (int n = 0; n < N; n++) dwr[n] += a * dy[n];
            }
        }
    }
    if (db) {
        for (int n = 0; n < N; n++) {
            float s = 0.0f;
            for (int m = 0; m < M; m++) s += dY[(size_t)m * N + n];
            db[n] += s;
        }
    }
}

void orc_tied_head_forward(float *logits, const float *lnf, const float *wte, int M, int D, int V) {
    /* train.c:412-423 */
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++) {
        const float *x = lnf + (size_t)m * D;
        float *lo = logits + (size_t)m * V;
        for (int vv = 0; vv < V; vv++) {
            const float *wr = wte + (size_t)vv * D;
            float s = 0.0f;
            for (int d = 0; d < D; d++) s += x[d] * wr[d];
            lo[vv] = s;
        }
    }
}

void orc_tied_head_backward(float *d_lnf, float *dwte, const float *dlogits, const float *lnf,
                            const float *wte, int M, int D, int V) {
    /* train.c:424-447 */
    if (d_lnf) {
#pragma omp parallel for schedule(static)
        for (int m = 0; m < M; m++) {
            const float *dl = dlogits + (size_t)m * V;
            float *dx = d_lnf + (size_t)m * D;
            for (int d = 0; d < D; d++) dx[d] = 0.0f;
            for (int vv = 0; vv < V; vv++) {
                float g = dl[vv];
                const float *wr = wte + (size_t)vv * D;
                for (int d = 0; d < D; d++) dx[d] += g * wr[d];
            }
        }
    }
    if (dwte) {
#pragma omp parallel for schedule(static)
        for (int vv = 0; vv < V; vv++) {
            float *dw = dwte + (size_t)vv * D;
            for (int m = 0; m < M; m++) {
                float g = dlogits[(size_t)m * V + vv];
                const float *lr = lnf + (size_t)m * D;
                for (int d = 0; d < D; d++) dw[d] += g * lr[d];
            }
        }
    }
}

void orc_lm_head(float *logits, const float *x, const float *wte, int T, int D, int V) {
    /* model.c:64-77 */
#pragma omp parallel for schedule(static)
    for (int v = 0; v < V; v++) {
        const float *wv = wte + (size_t)v * D;
        for (int t = 0; t < T; t++) {
            const float *xt = x + (size_t)t * D;
            float dot = 0.0f;
            for (int d = 0; d < D; d++) dot += xt[d] * wv[d];
            logits[(size_t)t * V + v] = dot;
        }
    }
}

void orc_matvec(float *out, const float *x, const float *W, const float *b, int M, int K, int N) {
    /* transformer.c:174-195, generate.c:95-107: bias initialises out, then
     * k-sequential accumulation; one independent row per m. */
    for (int m = 0; m < M; m++) {
        float *o = out + (size_t)m * N;
        const float *xm = x + (size_t)m * K;
        for (int n = 0; n < N; n++) o[n] = b ? b[n] : 0.0f;
        for (int k = 0; k < K; k++) {
            const float a = xm[k];
            const float *wr = W + (size_t)k * N;
            for (int n = 0; n < N; n++) o[n] += a * wr[n];
        }
    }
}

/* ------------------------------------------------------------- GELU ------ */
static const float ORC_GELU_K = 0.7978845608028654f; /* sqrt(2/pi), train.c:315 */

void orc_gelu_forward(float *out, const float *in, long n) {
    /* train.c:316-322 */
    for (long i = 0; i < n; i++) {
        const float x = in[i];
        const float t = tanhf(ORC_GELU_K * (x + 0.044715f * x * x * x));
        out[i] = 0.5f * x * (1.0f + t);
    }
}

void orc_gelu_backward(float *din, const float *dout, const float *in, long n) {
    /* train.c:324-333 */
    for (long i = 0; i < n; i++) {
        const float x = in[i];
        const float u = ORC_GELU_K * (x + 0.044715f * x * x * x);
        const float t = tanhf(u);
        const float dudx = ORC_GELU_K * (1.0f + 3.0f * 0.044715f * x * x);
        const float dgelu = 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * dudx;
        din[i] = dout[i] * dgelu;
    }
}

/* ------------------------------------------------------ CKP1 decode ------ */
struct orc_model {
    int hdr[8];
    int BLK, D, H, DF, L, V, DH;
    float *wte, *wpe, *gf, *bf, *buf;
    float **lw; /* per layer: g1 b1 Wq bq Wk bk Wv bv Wo bo g2 b2 W1 bff1 W2 bff2 */
    float *kc, *vc;
    float *x, *ln, *q, *att, *proj, *h, *sc;
    /* INT8 mode: matrices 2 4 6 8 12 14 of each layer and the tied head
     * quantised per output column (made on the first INT8 call) */
    int8_t *q8, **lq, *hq;
    float *q8s, **ls, *hs;
    uint8_t *xq;
    int32_t *acc;
};

orc_model *orc_model_load(const char *path) {
    /* generate.c:49-76 */
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    if (fread(m->hdr, sizeof(int), 8, f) != 8 || m->hdr[0] != 0x434B5031) {
        fclose(f);
        free(m);
        return NULL;
    }
    m->BLK = m->hdr[1], m->D = m->hdr[2], m->H = m->hdr[3], m->DF = m->hdr[4];
    m->L = m->hdr[5], m->V = m->hdr[6], m->DH = m->D / m->H;
    const long D = m->D, F = m->DF;
    const long sizes[16] = {D, D, D * D, D, D * D, D, D * D, D, D * D, D, D, D, D * F, F, F * D, D};
    long per = 0;
    for (int i = 0; i < 16; i++) per += sizes[i];
    const long n = (long)m->V * D + (long)m->BLK * D + m->L * per + 2 * D;
    m->buf = (float *)malloc(sizeof(float) * (size_t)n);
    if (fread(m->buf, sizeof(float), (size_t)n, f) != (size_t)n) {
        fclose(f);
        free(m->buf);
        free(m);
        return NULL;
    }
    fclose(f);
    float *p = m->buf;
    m->wte = p, p += (long)m->V * D;
    m->wpe = p, p += (long)m->BLK * D;
    m->lw = (float **)malloc(sizeof(float *) * 16 * (size_t)m->L);
    for (int l = 0; l < m->L; l++)
        for (int i = 0; i < 16; i++) m->lw[l * 16 + i] = p, p += sizes[i];
    m->gf = p, p += D;
    m->bf = p;
    m->kc = (float *)calloc((size_t)m->L * m->BLK * D, sizeof(float));
    m->vc = (float *)calloc((size_t)m->L * m->BLK * D, sizeof(float));
    m->x = (float *)malloc(sizeof(float) * D);
    m->ln = (float *)malloc(sizeof(float) * D);
    m->q = (float *)malloc(sizeof(float) * D);
    m->att = (float *)malloc(sizeof(float) * D);
    m->proj = (float *)malloc(sizeof(float) * D);
    m->h = (float *)malloc(sizeof(float) * F);
    m->sc = (float *)malloc(sizeof(float) * (size_t)m->BLK);
    return m;
}

void orc_model_header(const orc_model *m, int hdr[8]) { memcpy(hdr, m->hdr, sizeof m->hdr); }

void orc_layernorm_row(const float *x, const float *g, const float *b, float *y, int n) {
    /* generate.c:109-117 */
    float mu = 0, var = 0;
    for (int i = 0; i < n; i++) mu += x[i];
    mu /= n;
    for (int i = 0; i < n; i++) {
        const float d = x[i] - mu;
        var += d * d;
    }
    var /= n;
    const float rs = 1.0f / sqrtf(var + 1e-5f);
    for (int i = 0; i < n; i++) y[i] = (x[i] - mu) * rs * g[i] + b[i];
}

static const int ORC_QMAT[6] = {2, 4, 6, 8, 12, 14};

static void orc_model_quantize(orc_model *m) {
    const long D = m->D, F = m->DF, V = m->V;
    const long K[6] = {D, D, D, D, D, F}, N[6] = {D, D, D, D, F, D};
    long nb = V * D, ns = V;
    for (int i = 0; i < 6; i++) nb += m->L * K[i] * N[i], ns += m->L * N[i];
    m->q8 = (int8_t *)malloc((size_t)nb);
    m->q8s = (float *)malloc(sizeof(float) * (size_t)ns);
    m->lq = (int8_t **)malloc(sizeof(int8_t *) * 6 * (size_t)m->L);
    m->ls = (float **)malloc(sizeof(float *) * 6 * (size_t)m->L);
    int8_t *b = m->q8;
    float *sc = m->q8s;
    for (int l = 0; l < m->L; l++)
        for (int i = 0; i < 6; i++) {
            m->lq[l * 6 + i] = b, m->ls[l * 6 + i] = sc;
            orc_quantize_B_cols(m->lw[l * 16 + ORC_QMAT[i]], b, sc, (int)K[i], (int)N[i]);
            b += K[i] * N[i], sc += N[i];
        }
    /* the head's K x N operand is wte transposed: one column per vocabulary row */
    float *wt = (float *)malloc(sizeof(float) * (size_t)(V * D));
    for (long v = 0; v < V; v++)
        for (long d = 0; d < D; d++) wt[d * V + v] = m->wte[v * D + d];
    m->hq = b, m->hs = sc;
    orc_quantize_B_cols(wt, m->hq, m->hs, (int)D, (int)V);
    free(wt);
    const long kmax = D > F ? D : F, nmax = V > F ? (V > D ? V : D) : (F > D ? F : D);
    m->xq = (uint8_t *)malloc((size_t)kmax);
    m->acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)nmax);
}

/* out = dequant(quant_row(x) . Wq) (+ b): the per-token activation rule, int32
 * sums, sa * sb[n] applied to the sum, then the bias added to the result. */
static void orc_qmatvec(orc_model *m, float *out, const float *x, const int8_t *Wq,
                        const float *ws, const float *b, int K, int N) {
    float sa;
    orc_quantize_A_rows(x, m->xq, &sa, 1, K, K);
    orc_gemm_u8s8_i32(m->xq, K, Wq, N, m->acc, N, 1, N, K);
    orc_dequant(m->acc, N, &sa, ws, out, N, 1, N);
    if (b)
        for (int n = 0; n < N; n++) out[n] = out[n] + b[n];
}

void orc_decode_attention(const float *q, const float *kc, const float *vc, int ld, int pos,
                          int H, int DH, float *att, float *sc) {
    /* generate.c:130-152: per head, scores of q against cache rows 0..pos
     * (row stride ld), scaled by 1/sqrt(DH), max-subtracted softmax, and the
     * weighted sum of the value rows; sc holds pos + 1 floats of scratch */
    const float scale = 1.0f / sqrtf((float)DH);
    for (int h = 0; h < H; h++) {
        const int off = h * DH;
        float maxv = -1e30f;
        for (int j = 0; j <= pos; j++) {
            const float *kj = kc + (size_t)j * ld + off;
            float dot = 0;
            for (int d = 0; d < DH; d++) dot += q[off + d] * kj[d];
            dot *= scale;
            sc[j] = dot;
            if (dot > maxv) maxv = dot;
        }
        float sum = 0;
        for (int j = 0; j <= pos; j++) {
            const float e = expf(sc[j] - maxv);
            sc[j] = e;
            sum += e;
        }
        const float inv = 1.0f / sum;
        float *oh = att + off;
        for (int d = 0; d < DH; d++) oh[d] = 0;
        for (int j = 0; j <= pos; j++) {
            const float pj = sc[j] * inv;
            const float *vj = vc + (size_t)j * ld + off;
            for (int d = 0; d < DH; d++) oh[d] += pj * vj[d];
        }
    }
}

int orc_model_int8_weights(orc_model *m, int layer, int which, int8_t *Bq, float *sb) {
    /* the INT8 step's quantised operand (K x N, row-major) and its per-column
     * scales: which 0..5 = Wq Wk Wv Wo W1 W2 of a layer, or the head (layer ==
     * n_layers, which 0). Returns K * N, or 0 for no such matrix. */
    if (layer < 0 || layer > m->L || which < 0 || which > 5 || (layer == m->L && which != 0)) return 0;
    if (!m->q8) orc_model_quantize(m);
    const long D = m->D, F = m->DF;
    long K = D, N = D;
    const int8_t *src;
    const float *ss;
    if (layer == m->L) {
        N = m->V, src = m->hq, ss = m->hs;
    } else {
        if (which == 4) N = F;
        if (which == 5) K = F;
        src = m->lq[layer * 6 + which], ss = m->ls[layer * 6 + which];
    }
    if (Bq) memcpy(Bq, src, (size_t)(K * N));
    if (sb) memcpy(sb, ss, sizeof(float) * (size_t)N);
    return (int)(K * N);
}

static void orc_model_step(orc_model *m, int tok, int pos, float *logits, int int8) {
    /* generate.c:170-183 forward and :118-167 block */
    const int D = m->D, DH = m->DH, F = m->DF;
    if (int8 && !m->q8) orc_model_quantize(m);
#define ORC_MV(out, x, wi, K, N)                                                      \
    (int8 ? orc_qmatvec(m, out, x, m->lq[l * 6 + (wi)], m->ls[l * 6 + (wi)],           \
                        w[ORC_QMAT[wi] + 1], K, N)                                     \
          : orc_matvec(out, x, w[ORC_QMAT[wi]], w[ORC_QMAT[wi] + 1], 1, K, N))
    const float *te = m->wte + (size_t)tok * D, *pe = m->wpe + (size_t)pos * D;
    for (int i = 0; i < D; i++) m->x[i] = te[i] + pe[i];
    for (int l = 0; l < m->L; l++) {
        float **w = m->lw + l * 16;
        float *kc = m->kc + (size_t)l * m->BLK * D, *vc = m->vc + (size_t)l * m->BLK * D;
        float *krow = kc + (size_t)pos * D, *vrow = vc + (size_t)pos * D;
        orc_layernorm_row(m->x, w[0], w[1], m->ln, D);
        ORC_MV(m->q, m->ln, 0, D, D);
        ORC_MV(krow, m->ln, 1, D, D);
        ORC_MV(vrow, m->ln, 2, D, D);
        orc_decode_attention(m->q, kc, vc, D, pos, m->H, DH, m->att, m->sc);
        ORC_MV(m->proj, m->att, 3, D, D);
        for (int i = 0; i < D; i++) m->x[i] += m->proj[i];
        orc_layernorm_row(m->x, w[10], w[11], m->ln, D);
        ORC_MV(m->h, m->ln, 4, D, F);
        orc_gelu_forward(m->h, m->h, F);
        ORC_MV(m->proj, m->h, 5, F, D);
        for (int i = 0; i < D; i++) m->x[i] += m->proj[i];
    }
#undef ORC_MV
    orc_layernorm_row(m->x, m->gf, m->bf, m->ln, D);
    if (int8) {
        orc_qmatvec(m, logits, m->ln, m->hq, m->hs, NULL, D, m->V);
        return;
    }
    for (int v = 0; v < m->V; v++) {
        const float *wv = m->wte + (size_t)v * D;
        float dot = 0;
        for (int d = 0; d < D; d++) dot += m->ln[d] * wv[d];
        logits[v] = dot;
    }
}

void orc_model_forward(orc_model *m, int tok, int pos, float *logits) {
    orc_model_step(m, tok, pos, logits, 0);
}

void orc_model_forward_int8(orc_model *m, int tok, int pos, float *logits) {
    orc_model_step(m, tok, pos, logits, 1);
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    free(m->q8), free(m->q8s), free(m->lq), free(m->ls), free(m->xq), free(m->acc);
    free(m->buf), free(m->lw), free(m->kc), free(m->vc);
    free(m->x), free(m->ln), free(m->q), free(m->att), free(m->proj), free(m->h), free(m->sc);
    free(m);
}

/* ---------------------------------------------------- cross-entropy ------ */
float orc_cross_entropy(const float *logits, int ld, const int *targets, float *dlogits, int ldd,
                        int M, int V) {
    /* train.c:449-465 with explicit V and leading dimensions: per row the
     * max, e = expf(l - max) summed in v order, p = e * (1/sum), the loss term
     * -log((double)p[t] + 1e-30), dl = (p - onehot) / (float)M; the mean as
     * (float)(double sum / M). dlogits may be logits itself (same ld). */
    double loss = 0.0;
    for (int m = 0; m < M; m++) {
        const float *lo = logits + (size_t)m * ld;
        float *dl = dlogits + (size_t)m * ldd;
        const int t = targets[m];
        float maxl = lo[0];
        for (int v = 1; v < V; v++)
            if (lo[v] > maxl) maxl = lo[v];
        float sum = 0.0f;
        for (int v = 0; v < V; v++) {
            const float e = expf(lo[v] - maxl);
            dl[v] = e;
            sum += e;
        }
        const float inv = 1.0f / sum;
        for (int v = 0; v < V; v++) dl[v] *= inv;
        loss += -log((double)dl[t] + 1e-30);
        for (int v = 0; v < V; v++) dl[v] = (dl[v] - (v == t ? 1.0f : 0.0f)) / (float)M;
    }
    return (float)(loss / M);
}

float orc_head_ce(const float *lnf, const float *wte, const int *targets, int M, int D, int V,
                  float *d_lnf, float *dwte) {
    /* train.c:531 (tied_head_forward), :718 (cross_entropy), :542
     * (tied_head_backward: d_lnf set, dwte accumulated) in sequence */
    float *lg = (float *)malloc(sizeof(float) * (size_t)M * V);
    orc_tied_head_forward(lg, lnf, wte, M, D, V);
    const float loss = orc_cross_entropy(lg, V, targets, lg, V, M, V);
    orc_tied_head_backward(d_lnf, dwte, lg, lnf, wte, M, D, V);
    free(lg);
    return loss;
}

/* -------------------------------------------------------- attention ------ */
void orc_attention_forward(const float *q, const float *k, const float *v, int ld, float *att,
                           int ld_att, float *probs, int B, int T, int H, int dh) {
    /* train.c:339-370, per (b, h) and query i: scores over j <= i with the
     * running max, expf and the sum in j order, p *= 1/sum, then the
     * j-sequential weighted sum of v rows. */
    const float scale = 1.0f / sqrtf((float)dh);
    float *row = (float *)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
    for (int bh = 0; bh < B * H; bh++) {
        const int b = bh / H, off = (bh % H) * dh;
        for (int i = 0; i < T; i++) {
            const float *qi = q + (size_t)(b * T + i) * ld + off;
            float *p = probs ? probs + ((size_t)bh * T + i) * T : row;
            float maxv = -1e30f;
            for (int j = 0; j <= i; j++) {
                const float *kj = k + (size_t)(b * T + j) * ld + off;
                float dot = 0.0f;
                for (int d = 0; d < dh; d++) dot += qi[d] * kj[d];
                dot *= scale;
                p[j] = dot;
                if (dot > maxv) maxv = dot;
            }
            float sum = 0.0f;
            for (int j = 0; j <= i; j++) {
                const float e = expf(p[j] - maxv);
                p[j] = e;
                sum += e;
            }
            const float inv = 1.0f / sum;
            for (int j = 0; j <= i; j++) p[j] *= inv;
            for (int j = i + 1; j < T; j++) p[j] = 0.0f;
            float *oi = att + (size_t)(b * T + i) * ld_att + off;
            for (int d = 0; d < dh; d++) oi[d] = 0.0f;
            for (int j = 0; j <= i; j++) {
                const float pj = p[j];
                const float *vj = v + (size_t)(b * T + j) * ld + off;
                for (int d = 0; d < dh; d++) oi[d] += pj * vj[d];
            }
        }
    }
    free(row);
}

void orc_attention_backward(float *dq, float *dk, float *dv, const float *d_att, int ld_att,
                            const float *q, const float *k, const float *v, int ld,
                            const float *probs, int B, int T, int H, int dh) {
    /* train.c:374-407: d_probs_j = dao . v_j and dv_j += p_j dao; then
     * dot = sum_j p_j d_probs_j, ds_j = p_j (d_probs_j - dot) scale,
     * dq_i += ds_j k_j, dk_j += ds_j q_i -- all in j order per query i. */
    const float scale = 1.0f / sqrtf((float)dh);
    float *dprobs = (float *)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
    for (int bh = 0; bh < B * H; bh++) {
        const int b = bh / H, off = (bh % H) * dh;
        for (int i = 0; i < T; i++) {
            const float *dao = d_att + (size_t)(b * T + i) * ld_att + off;
            const float *p = probs + ((size_t)bh * T + i) * T;
            for (int j = 0; j <= i; j++) {
                const float *vj = v + (size_t)(b * T + j) * ld + off;
                float *dvj = dv + (size_t)(b * T + j) * ld + off;
                float dp = 0.0f;
                for (int d = 0; d < dh; d++) {
                    dp += dao[d] * vj[d];
                    dvj[d] += p[j] * dao[d];
                }
                dprobs[j] = dp;
            }
            float dot = 0.0f;
            for (int j = 0; j <= i; j++) dot += p[j] * dprobs[j];
            float *dqi = dq + (size_t)(b * T + i) * ld + off;
            const float *qi = q + (size_t)(b * T + i) * ld + off;
            for (int j = 0; j <= i; j++) {
                const float ds = p[j] * (dprobs[j] - dot) * scale;
                const float *kj = k + (size_t)(b * T + j) * ld + off;
                float *dkj = dk + (size_t)(b * T + j) * ld + off;
                for (int d = 0; d < dh; d++) {
                    dqi[d] += ds * kj[d];
                    dkj[d] += ds * qi[d];
                }
            }
        }
    }
    free(dprobs);
}

void orc_attention_forward_f64(const float *q, const float *k, const float *v, int ld, float *att,
                               int ld_att, float *probs, int B, int T, int H, int dh) {
    const double scale = 1.0 / sqrt((double)dh);
    double *row = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
    for (int bh = 0; bh < B * H; bh++) {
        const int b = bh / H, off = (bh % H) * dh;
        for (int i = 0; i < T; i++) {
            const float *qi = q + (size_t)(b * T + i) * ld + off;
            double maxv = -1e300, sum = 0.0;
            for (int j = 0; j <= i; j++) {
                const float *kj = k + (size_t)(b * T + j) * ld + off;
                double dot = 0.0;
                for (int d = 0; d < dh; d++) dot += (double)qi[d] * kj[d];
                row[j] = dot * scale;
                if (row[j] > maxv) maxv = row[j];
            }
            for (int j = 0; j <= i; j++) {
                row[j] = exp(row[j] - maxv);
                sum += row[j];
            }
            for (int j = 0; j <= i; j++) row[j] /= sum;
            if (probs) {
                float *p = probs + ((size_t)bh * T + i) * T;
                for (int j = 0; j < T; j++) p[j] = j <= i ? (float)row[j] : 0.0f;
            }
            float *oi = att + (size_t)(b * T + i) * ld_att + off;
            for (int d = 0; d < dh; d++) {
                double o = 0.0;
                for (int j = 0; j <= i; j++) o += row[j] * v[(size_t)(b * T + j) * ld + off + d];
                oi[d] = (float)o;
            }
        }
    }
    free(row);
}

/* ------------------------------------------------------------- INT8 ------ */
/* gemm_bench.c:228 and :243 write `amax/127.0f`. The reference is built with
 * -ffast-math (README.md:104, gemm_bench.c:8), under which gcc emits
 * amax * fl(1/127): the scales (and hence the bytes) of the reference as it
 * actually runs come from that multiplication, which differs from a correctly
 * rounded division by one ulp for ~4% of inputs. The restatement follows the
 * built reference; tests/test_oracle.py pins this against oracle/_ref. */
#define RCP127 (1.0f / 127.0f)

static int clamp127(int q) { return q > 127 ? 127 : (q < -127 ? -127 : q); }

float orc_quantize_A(const float *A, uint8_t *Au, int M, int K, int Kpad) {
    /* gemm_bench.c:225-236 */
    float amax = 1e-8f;
    for (size_t i = 0; i < (size_t)M * K; i++) {
        float v = fabsf(A[i]);
        if (v > amax) amax = v;
    }
    float scale = amax * RCP127, inv = 1.0f / scale;
    for (int m = 0; m < M; m++)
        for (int k = 0; k < Kpad; k++) {
            int q = 0;
            if (k < K) q = clamp127((int)lroundf(A[(size_t)m * K + k] * inv));
            Au[(size_t)m * Kpad + k] = (uint8_t)(q + 128);
        }
    return scale;
}

void orc_quantize_A_rows(const float *A, uint8_t *Au, float *sa, int M, int K, int Kpad) {
    /* gemm_bench.c:225-236 rule applied per row (per-token activation scale) */
    for (int m = 0; m < M; m++) {
        const float *a = A + (size_t)m * K;
        float amax = 1e-8f;
        for (int k = 0; k < K; k++) {
            float v = fabsf(a[k]);
            if (v > amax) amax = v;
        }
        float scale = amax * RCP127, inv = 1.0f / scale;
        sa[m] = scale;
        for (int k = 0; k < Kpad; k++) {
            int q = 0;
            if (k < K) q = clamp127((int)lroundf(a[k] * inv));
            Au[(size_t)m * Kpad + k] = (uint8_t)(q + 128);
        }
    }
}

void orc_quantize_B_cols(const float *B, int8_t *Bq, float *bscale, int K, int N) {
    /* gemm_bench.c:240-244 scale rule and :249-253 rounding, unpacked output */
    for (int n = 0; n < N; n++) {
        float bmax = 1e-8f;
        for (int k = 0; k < K; k++) {
            float v = fabsf(B[(size_t)k * N + n]);
            if (v > bmax) bmax = v;
        }
        bscale[n] = bmax * RCP127;
        float inv = 1.0f / bscale[n];
        for (int k = 0; k < K; k++)
            Bq[(size_t)k * N + n] = (int8_t)clamp127((int)lroundf(B[(size_t)k * N + n] * inv));
    }
}

void orc_quantize_B_pack(const float *B, int8_t *Bp, float *bscale, int32_t *colsum,
                         int K, int N, int Kpad) {
    /* gemm_bench.c:238-259 */
    for (int n = 0; n < N; n++) {
        float bmax = 1e-8f;
        for (int k = 0; k < K; k++) {
            float v = fabsf(B[(size_t)k * N + n]);
            if (v > bmax) bmax = v;
        }
        bscale[n] = bmax * RCP127;
    }
    int kgc = Kpad / 4, panels = N / 16;
    for (int p = 0; p < panels; p++) {
        int n0 = p * 16;
        int8_t *base = Bp + (size_t)p * kgc * 64;
        for (int i = 0; i < 16; i++) {
            float inv = 1.0f / bscale[n0 + i];
            int s = 0;
            for (int kg = 0; kg < kgc; kg++)
                for (int j = 0; j < 4; j++) {
                    int kk = kg * 4 + j, q = 0;
                    if (kk < K) q = clamp127((int)lroundf(B[(size_t)kk * N + n0 + i] * inv));
                    base[(size_t)kg * 64 + i * 4 + j] = (int8_t)q;
                    s += q;
                }
            colsum[n0 + i] = s;
        }
    }
}

void orc_unpack_vnni(const int8_t *Bp, int8_t *Bq, int K, int N, int Kpad) {
    /* inverse of the layout written at gemm_bench.c:254 */
    int kgc = Kpad / 4;
    for (int k = 0; k < K; k++)
        for (int n = 0; n < N; n++) {
            int p = n / 16, i = n % 16, kg = k / 4, j = k % 4;
            Bq[(size_t)k * N + n] = Bp[(size_t)p * kgc * 64 + (size_t)kg * 64 + i * 4 + j];
        }
}

long orc_gemm_u8s8_i32(const uint8_t *Au, int lda, const int8_t *Bq, int ldb, int32_t *C, int ldc,
                       int M, int N, int K) {
    long bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad)
    for (int m = 0; m < M; m++) {
        const uint8_t *a = Au + (size_t)m * lda;
        for (int n = 0; n < N; n++) {
            int64_t acc = 0;
            for (int k = 0; k < K; k++)
                acc += (int64_t)((int)a[k] - 128) * (int64_t)Bq[(size_t)k * ldb + n];
            if (acc > INT32_MAX || acc < INT32_MIN) bad++;
            C[(size_t)m * ldc + n] = (int32_t)acc;
        }
    }
    return bad;
}

long orc_gemm_u8s8_raw_i32(const uint8_t *Au, int lda, const int8_t *Bq, int ldb, int32_t *C,
                           int ldc, int M, int N, int K) {
    long bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad)
    for (int m = 0; m < M; m++) {
        const uint8_t *a = Au + (size_t)m * lda;
        for (int n = 0; n < N; n++) {
            int64_t acc = 0;
            for (int k = 0; k < K; k++) acc += (int64_t)a[k] * (int64_t)Bq[(size_t)k * ldb + n];
            if (acc > INT32_MAX || acc < INT32_MIN) bad++;
            C[(size_t)m * ldc + n] = (int32_t)acc;
        }
    }
    return bad;
}

void orc_gemm_int8_kernel(const uint8_t *Au, int Kpad, const int8_t *Bp, const int32_t *corr,
                          const float *dq, float *C, int M, int N) {
    /* gemm_bench.c:260-285: vpdpbusd accumulates in int32 with wrap-around;
     * v = acc - corr (:274) and C = cvt(v) * dq (:275). */
    int kgc = Kpad / 4, panels = N / 16;
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int p = 0; p < panels; p++) {
            const int8_t *bp = Bp + (size_t)p * kgc * 64;
            for (int i = 0; i < 16; i++) {
                uint32_t acc = 0;
                for (int kg = 0; kg < kgc; kg++)
                    for (int j = 0; j < 4; j++)
                        acc += (uint32_t)((int32_t)Au[(size_t)m * Kpad + kg * 4 + j] *
                                          (int32_t)bp[(size_t)kg * 64 + i * 4 + j]);
                int n = p * 16 + i;
                int32_t v = (int32_t)(acc - (uint32_t)corr[n]);
                C[(size_t)m * N + n] = (float)v * dq[n];
            }
        }
}

void orc_dequant(const int32_t *V, int ldv, const float *sa, const float *sb, float *C, int ldc,
                 int M, int N) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float dq = sa ? sa[m] * sb[n] : sb[n];
            C[(size_t)m * ldc + n] = (float)V[(size_t)m * ldv + n] * dq;
        }
}

double orc_rms_rel(const float *X, const float *R, long n) {
    /* gemm_bench.c:302-306 */
    double se = 0.0, sr = 0.0;
    for (long i = 0; i < n; i++) {
        double d = (double)X[i] - R[i];
        se += d * d;
        sr += (double)R[i] * R[i];
    }
    return sqrt(se / (sr + 1e-30));
}

double orc_max_abs_diff(const float *X, const float *Y, long n) {
    /* gemm_bench.c:53-57 */
    double d = 0.0;
    for (long i = 0; i < n; i++) {
        double e = fabs((double)X[i] - Y[i]);
        if (e > d) d = e;
    }
    return d;
}
