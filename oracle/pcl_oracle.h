/*
 * pcl_oracle.h -- CPU restatement of pure-c-llm's matrix-multiply hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels in
 * libpcl_hip: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. The product path never links or calls it.
 *
 * Every function states the reference file:line whose semantics it follows
 * (paths are relative to the reference repository root). Arithmetic choices:
 *   - float functions that restate a reference loop keep the reference's
 *     accumulation order (k-sequential per output element) in fp32;
 *   - *_f64 functions accumulate in double and round once: the "truth" used to
 *     judge both the reference-order restatements and the GPU kernels;
 *   - integer functions accumulate in int64 and report overflow of int32.
 * The library is compiled with -ffp-contract=off so that a*b+c is never fused:
 * the restatements are reproducible bit-for-bit on any x86-64 host.
 */
#ifndef PCL_ORACLE_H
#define PCL_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- PRNG ---- */
/* xorshift32 step, the recurrence of train.c:73-78 and model.c:117-125. */
uint32_t orc_xorshift32(uint32_t *state);
/* p[i] = (u*2-1)*scale with u = (s & 0xFFFFFF)/2^24  (train.c:73-78 frand). */
void orc_fill_frand(float *p, size_t n, uint32_t seed, float scale);
/* p[i] = lo + (hi-lo)*u, same u as above (scales in U[1e-3,1e-2]). */
void orc_fill_uniform(float *p, size_t n, uint32_t seed, float lo, float hi);
/* Box-Muller N(mean, std) from two xorshift uniforms (u1 shifted off 0). */
void orc_fill_normal(float *p, size_t n, uint32_t seed, float mean, float std);
/* u8 uniform {0..255} and s8 uniform {-128..127}: bits 16..23 of each step. */
void orc_fill_u8(uint8_t *p, size_t n, uint32_t seed);
void orc_fill_s8(int8_t *p, size_t n, uint32_t seed);
/* tensor.c:204-205 self-test pattern: A[i]=((i%13)-6)*0.1, B[i]=((i%7)-3)*0.1 */
void orc_fill_kat_tensor(float *A, size_t na, float *B, size_t nb);

/* ---------------------------------------------------- FP32 GEMM family ---- */
/* tensor.c:34-53 matmul: C zeroed, then i-k-j accumulation in fp32. */
void orc_matmul_ikj(const float *A, const float *B, float *C, int M, int K, int N);
/* gemm_bench.c:60-67 v0 naive i-j-k, fp32 dot per element. */
void orc_matmul_naive(const float *A, const float *B, float *C, int M, int K, int N);

/*
 * Generic double-accumulated GEMM over strided operands -- the truth.
 *   C[m*ldc+n] = (accum ? C : 0) + sum_k A(m,k)*B(k,n) + (bias ? bias[n] : 0)
 *   A(m,k) = A[m*sam + k*sak], B(k,n) = B[k*sbk + n*sbn]
 * rounded once to fp32.
 */
void orc_gemm_f64(const float *A, long sam, long sak, const float *B, long sbk, long sbn,
                  const float *bias, float *C, long ldc, int M, int N, int K, int accum);

/* gpu_kernels.h:44-51 semantics (gpu_kernels.cu:112-142), computed in double:
 *   nn: C(M,N)  = A(M,K)·B(K,N) + bias
 *   nt: C(M,N) ?= A(M,K)·B(N,K)^T      (accum selects C += ...)
 *   tn: C(K,N) += A(M,K)^T·B(M,N)
 *   bias_bwd: db[n] += sum_m dY[m,n] (fp32, m-sequential; gpu_kernels.cu:102-108) */
void orc_gemm_nn(const float *A, const float *B, const float *bias, float *C, int M, int K, int N);
void orc_gemm_nt(const float *A, const float *B, float *C, int M, int K, int N, int accum);
void orc_gemm_tn(const float *A, const float *B, float *C, int M, int K, int N);
void orc_bias_bwd(float *db, const float *dY, int M, int N);

/* train.c:181-211 matmul_forward: out = in·W (+ bias added in a second pass),
 * fp32 i-k-j order of the non-AVX path. */
void orc_matmul_forward(float *out, const float *in, const float *W, const float *bias,
                        int M, int K, int N);
/* train.c:219-252 matmul_backward: dX += dY·W^T, dW += X^T·dY, db += colsum(dY),
 * each in the reference's fp32 loop order. dX/dW/db may be NULL to skip. */
void orc_matmul_backward(const float *dY, const float *X, const float *W, float *dX,
                         float *dW, float *db, int M, int K, int N);
/* train.c:412-423 tied_head_forward with D,V explicit: logits = lnf·wte^T. */
void orc_tied_head_forward(float *logits, const float *lnf, const float *wte, int M, int D, int V);
/* train.c:424-447 tied_head_backward: d_lnf = dlogits·wte (SET), dwte += dlogits^T·lnf. */
void orc_tied_head_backward(float *d_lnf, float *dwte, const float *dlogits, const float *lnf,
                            const float *wte, int M, int D, int V);
/* model.c:64-77 lm_head: logits[t,v] = x[t]·wte[v]. */
void orc_lm_head(float *logits, const float *x, const float *wte, int T, int D, int V);
/* transformer.c:174-195 proj_token / generate.c:95-107 matvec:
 * out(N) = bias (or 0), then += x[k]*W[k,n] k-sequential. Batched over M rows. */
void orc_matvec(float *out, const float *x, const float *W, const float *b, int M, int K, int N);

/* ------------------------------------------------------------- INT8 ------ */
/* gemm_bench.c:225-236 quantize_A: per-tensor scale amax*fl(1/127) (the -ffast-math
 * build of amax/127.0f), q=clamp(lroundf(x*(1/s))),
 * Au=q+128, K padded to Kpad with Au=128. Returns the scale. */
float orc_quantize_A(const float *A, uint8_t *Au, int M, int K, int Kpad);
/* Per-row (per-token) variant of the same rule: sa[m] = amax_row*fl(1/127). */
void orc_quantize_A_rows(const float *A, uint8_t *Au, float *sa, int M, int K, int Kpad);
/* gemm_bench.c:238-259 quantize_B_pack: per-column scale bmax*fl(1/127), VNNI panel
 * layout Bp[p*(Kpad/4)*64 + kg*64 + i*4 + j] = Bq[kg*4+j][p*16+i], colsum[n]=sum q. */
void orc_quantize_B_pack(const float *B, int8_t *Bp, float *bscale, int32_t *colsum,
                         int K, int N, int Kpad);
/* Same per-column rule, unpacked: Bq is K x N row-major s8. */
void orc_quantize_B_cols(const float *B, int8_t *Bq, float *bscale, int K, int N);
/* Unpack the VNNI panel layout back to Bq (K x N row-major; rows >= K unused). */
void orc_unpack_vnni(const int8_t *Bp, int8_t *Bq, int K, int N, int Kpad);

/* train.c:314-333 tanh-GELU: out = 0.5 x (1 + tanhf(K (x + 0.044715 x^3))),
 * K = 0.7978845608028654f; backward din = dout * dgelu(x) (SET). */
void orc_gelu_forward(float *out, const float *in, long n);
void orc_gelu_backward(float *din, const float *dout, const float *in, long n);

/* train.c:449-465: mean loss over M rows of V logits; dlogits = (p - onehot)/M
 * (may alias logits with ldd == ld). */
float orc_cross_entropy(const float *logits, int ld, const int *targets, float *dlogits, int ldd,
                        int M, int V);
/* train.c:531 + :718 + :542: logits = lnf.wte^T, cross-entropy, d_lnf SET and
 * dwte ACCUMULATED (either may be NULL); returns the mean loss. */
float orc_head_ce(const float *lnf, const float *wte, const int *targets, int M, int D, int V,
                  float *d_lnf, float *dwte);

/* generate.c:49-183 restated: a CKP1 checkpoint (train.c:633-648 layout) in
 * host memory with its KV cache, and forward(tok, pos) -> logits (V floats):
 * embedding, per layer ln -> Wq/Wk/Wv matvecs -> attention over the cache ->
 * Wo matvec added into x -> ln -> W1 matvec -> tanh-GELU -> W2 added into x,
 * final ln, tied head. NULL when the file is not a CKP1 checkpoint. */
typedef struct orc_model orc_model;
orc_model *orc_model_load(const char *path);
void orc_model_header(const orc_model *m, int hdr[8]);
void orc_model_forward(orc_model *m, int tok, int pos, float *logits);
/* The same step with INT8 products (one model object is used in one mode: the
 * KV cache is shared): every matrix and the tied head quantised per output
 * column (gemm_bench.c:238-259's rule), each product's input quantised per
 * token (gemm_bench.c:225-236's rule over one row), exact int32 sums,
 * dequantised by sa * sb[n], then the bias added. */
void orc_model_forward_int8(orc_model *m, int tok, int pos, float *logits);
void orc_model_free(orc_model *m);
/* The pieces of that step, for checking a decoder op by op: the LayerNorm row
 * (generate.c:109-117), the cached attention of one query (generate.c:130-152;
 * cache rows of ld floats, sc = pos + 1 floats of scratch), and the INT8
 * step's quantised operands (which 0..5 = Wq Wk Wv Wo W1 W2 of a layer, K x N
 * bytes row-major plus N scales; layer n_layers, which 0 = the head; returns
 * K * N, 0 when there is no such matrix). */
void orc_layernorm_row(const float *x, const float *g, const float *b, float *y, int n);
void orc_decode_attention(const float *q, const float *kc, const float *vc, int ld, int pos,
                          int H, int DH, float *att, float *sc);
int orc_model_int8_weights(orc_model *m, int layer, int which, int8_t *Bq, float *sb);

/* Causal multi-head attention, train.c:339-370 attention_forward generalised
 * to B sequences of T tokens, H heads of dh: q/k/v rows of ld floats (row
 * b*T + t, head h at columns [h*dh, (h+1)*dh)), att rows of ld_att.
 *   p_ij = exp(s_ij - max_j s) / sum_j exp(...),  s_ij = (q_i . k_j) * (1/sqrtf(dh)), j <= i
 *   att_i = sum_{j<=i} p_ij v_j
 * probs: NULL or [B*H][T][T]; entries j > i are set to 0 (gpu_kernels.cu:279). */
void orc_attention_forward(const float *q, const float *k, const float *v, int ld, float *att,
                           int ld_att, float *probs, int B, int T, int H, int dh);
/* train.c:374-407 attention_backward: dq, dk, dv (rows of ld) ACCUMULATE the
 * gradients given d_att (rows of ld_att) and the forward's probs. */
void orc_attention_backward(float *dq, float *dk, float *dv, const float *d_att, int ld_att,
                            const float *q, const float *k, const float *v, int ld,
                            const float *probs, int B, int T, int H, int dh);
/* Same mathematics in double precision (score, softmax and sums), rounded once
 * to float: the tolerance anchor for dh the reference is not built at. */
void orc_attention_forward_f64(const float *q, const float *k, const float *v, int ld, float *att,
                               int ld_att, float *probs, int B, int T, int H, int dh);

/* Exact u8 x s8 GEMM, the identity of gemm_bench.c:216-217:
 *   C[m,n] = sum_k (Au[m,k]-128) * Bq[k,n]   (Bq K x N row-major, ldb)
 * int64 accumulation; returns the number of outputs outside int32 (0 = ok). */
long orc_gemm_u8s8_i32(const uint8_t *Au, int lda, const int8_t *Bq, int ldb, int32_t *C, int ldc,
                       int M, int N, int K);
/* Raw VNNI sum without the offset fixup: sum_k Au*Bq (gemm_bench.c:264-270). */
long orc_gemm_u8s8_raw_i32(const uint8_t *Au, int lda, const int8_t *Bq, int ldb, int32_t *C,
                           int ldc, int M, int N, int K);
/* gemm_bench.c:260-285 gemm_int8_kernel restated in scalar C over the VNNI
 * layout: v = sum Au*Bq - corr[n]; C = (float)v * dq[n]. M%8==0, N%16==0. */
void orc_gemm_int8_kernel(const uint8_t *Au, int Kpad, const int8_t *Bp, const int32_t *corr,
                          const float *dq, float *C, int M, int N);
/* Dequant with the reference op order (gemm_bench.c:272-275, dq precomputed at :378):
 *   rowcol: C = (float)v * (sa[m]*sb[n]);   col (sa==NULL): C = (float)v * sb[n] */
void orc_dequant(const int32_t *V, int ldv, const float *sa, const float *sb, float *C, int ldc,
                 int M, int N);
/* gemm_bench.c:302-306 rms_rel and :53-57 max_abs_diff. */
double orc_rms_rel(const float *X, const float *R, long n);
double orc_max_abs_diff(const float *X, const float *Y, long n);

#ifdef __cplusplus
}
#endif
#endif /* PCL_ORACLE_H */
