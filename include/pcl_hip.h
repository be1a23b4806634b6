/*
 * pcl_hip.h -- C ABI of libpcl_hip, the MI355X (gfx950) matrix-multiply engine
 * for pure-c-llm.
 *
 * Three families of entry points:
 *
 *  1. Host-pointer drop-ins with the reference's exact C signatures. A C
 *     program that declares these functions (tensor.h, model.h, or the
 *     `static` ones of train.c / transformer.c / generate.c / gemm_bench.c
 *     turned into `extern` declarations) links against libpcl_hip instead of
 *     the CPU code. Each call copies its operands to the GPU, runs the HIP
 *     kernels and copies the result back before returning, exactly as
 *     synchronous as the CPU original. They return void like the reference;
 *     a failure is recorded in pcl_last_status()/pcl_last_error() (and aborts
 *     the process when pcl_set_abort_on_error(1) was called, like the
 *     reference's CUDA_CHECK / xmalloc).
 *
 *  2. Device-pointer drop-ins of the reference GPU API (gpu_kernels.h:38-51):
 *     gpu_init, gemm_nn, gemm_nt, gemm_tn, bias_bwd. Asynchronous on the
 *     calling thread's stream (pcl_set_stream; default: the null stream).
 *
 *  3. Native pcl_* entry points: device pointers, explicit leading
 *     dimensions and stream, an int status return (PCL_OK == 0). These are the
 *     timed path: inputs resident in HBM, no host traffic.
 *
 * Conventions (all families): row-major storage, the caller owns every buffer
 * (the library never frees caller memory; tensor.h:17-20), outputs never
 * alias inputs (tensor.h:37). M, N, K count elements; leading dimensions
 * count elements of the operand's type. Dimensions of 0 are valid and do
 * nothing except the defined output writes (e.g. C = bias when K == 0).
 */
#ifndef PCL_HIP_H
#define PCL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status ---- */
enum {
    PCL_OK = 0,
    PCL_ERR_INVALID_ARG = 1, /* negative dims, NULL operand, bad leading dim  */
    PCL_ERR_HIP = 2,         /* a HIP runtime call or kernel launch failed    */
    PCL_ERR_NO_DEVICE = 3,   /* no usable gfx950 device                       */
    PCL_ERR_OOM = 4,         /* device or host allocation failed              */
    PCL_ERR_UNSET_DIMS = 5,  /* a drop-in that needs pcl_set_model_dims       */
    PCL_ERR_RANGE = 6        /* an INT8 shape whose int32 sum could overflow  */
};

/* Library set-up. Every entry point initialises lazily; calling this first
 * only moves the cost (device query, workspace) out of the first GEMM. */
int pcl_init(void);
/* Status and message on this thread: the outcome of the most recent void
 * drop-in call (PCL_OK after a success), or of a later native call that
 * failed (native calls report success only through their return value). */
int pcl_last_status(void);
const char *pcl_last_error(void);
void pcl_clear_error(void);
/* 1: a failing void drop-in prints its message and calls exit(1), matching
 * the reference's CUDA_CHECK (gpu_kernels.h:34-36). Default 0. */
void pcl_set_abort_on_error(int on);
/* Stream used by this thread's calls (a hipStream_t; NULL = null stream). */
int pcl_set_stream(void *hip_stream);
void *pcl_get_stream(void);
int pcl_stream_synchronize(void);
/* Streams and graphs (no counterpart in the reference, which runs on the
 * CPU). A decode loop issues a short sequence of small products per token;
 * capturing the sequence once into a HIP graph and replaying it costs one
 * launch per token instead of one or two per product.
 *   pcl_stream_create: a new non-blocking stream (default priority).
 *   pcl_stream_destroy: waits for the stream, frees its scratch; destroy the
 *     graphs captured on it first.
 *   pcl_graph_begin/end: capture this thread's native device-pointer calls on
 *     its stream (which must come from pcl_stream_create) into *graph; the
 *     calls are recorded, not run. Host-pointer drop-ins cannot be captured:
 *     while the thread's stream captures (through pcl_graph_begin or the
 *     caller's own hipStreamBeginCapture) they fail with
 *     PCL_ERR_INVALID_ARG before touching the stream.
 *   pcl_graph_launch: replay on this thread's stream. Every replay uses the
 *     pointers and sizes recorded at capture time; scratch used by a graph
 *     stays allocated until its stream is destroyed. */
void *pcl_stream_create(void);
int pcl_stream_destroy(void *stream);
/* Scratch memory. Calls keep per-stream device buffers that grow to the
 * largest request and are reused: split-K partial sums, the padded INT8
 * activations, the INT8 GEMM's tile counters (64 bytes: the persistent kernel
 * of outputs past 256 MiB hands its tiles out from them, so calls on one
 * stream must not overlap -- stream order guarantees it), pcl_head_ce's
 * logits chunk, and the realigned copies of
 * misaligned FP32 operands that pcl_sgemm makes for products of >= 2^30
 * multiply-adds (for the trainer's head backward over 4096 x 50257 logits
 * about 0.8 GB). pcl_release_scratch waits for the stream (hip_stream, NULL =
 * null stream) and frees these buffers; the next call allocates again. It
 * fails with PCL_ERR_INVALID_ARG on a stream a graph was captured on (the
 * graph may use them; pcl_stream_destroy frees them). Calls on the stream
 * from other threads must not overlap it. No counterpart in the reference. */
int pcl_release_scratch(void *hip_stream);
int pcl_graph_begin(void);
int pcl_graph_end(void **graph);
int pcl_graph_launch(void *graph);
int pcl_graph_destroy(void *graph);
/* Device name and compute-unit count of the current device, for reports. */
int pcl_device_info(char *name, int name_len, int *num_cus, int *clock_khz);

/* Device memory plumbing for C hosts and bindings (hipMalloc & co.). */
void *pcl_malloc(size_t bytes);
int pcl_free(void *p);
int pcl_memcpy_h2d(void *dst, const void *src, size_t bytes);
int pcl_memcpy_d2h(void *dst, const void *src, size_t bytes);
int pcl_memcpy_d2d(void *dst, const void *src, size_t bytes);
int pcl_memset(void *dst, int value, size_t bytes);

/* Event timing on this thread's stream (hipEvent_t behind an opaque handle). */
void *pcl_event_create(void);
int pcl_event_record(void *ev);
int pcl_event_elapsed_ms(void *start, void *stop, float *ms); /* synchronises on stop */
int pcl_event_destroy(void *ev);

/* The reference's tied-head functions read compile-time D_MODEL/VOCAB_SIZE
 * (train.c:34-51, transformer.h:35-39, model.h:24). The drop-ins below read
 * them from here instead; they fail with PCL_ERR_UNSET_DIMS until set. */
int pcl_set_model_dims(int d_model, int vocab_size);
/* The attention drop-ins read compile-time N_HEADS (train.c:41) and, for the
 * GPU API, B_SIZE/T_SIZE/DIM (gpu_kernels.h:17-31); here they come from
 * pcl_set_attn_dims and pcl_set_model_dims (d_model = DIM), PCL_ERR_UNSET_DIMS
 * until set. Head size d_model / n_heads must be 32, 64 or 128. */
int pcl_set_attn_dims(int batch, int seq_len, int n_heads);

/* ============================== 1. host-pointer drop-ins ================= */

/* tensor.h:40 / tensor.c:34-53: C(M,N) = A(M,K)·B(K,N), C fully overwritten.
 * Also the signature of gemm_bench's gemm_fn rungs (gemm_bench.c:328). */
void matmul(const float *A, const float *B, float *C, int M, int K, int N);

/* train.c:181-211: out(M,N) = in(M,K)·W(K,N) + bias(N) (bias may be NULL). */
void matmul_forward(float *out, const float *in, const float *Wt, const float *bias,
                    int M, int K, int N);

/* train.c:219-252: dX += dY·W^T, dW += X^T·dY, db += colsum(dY) (db may be NULL). */
void matmul_backward(const float *dY, const float *X, const float *Wt, float *dX, float *dW,
                     float *db, int M, int K, int N);

/* train.c:412-423: logits(M,V) = lnf(M,D)·wte(V,D)^T. D,V from pcl_set_model_dims. */
void tied_head_forward(float *logits, const float *lnf, const float *wte, int M);

/* train.c:424-447: d_lnf = d_logits·wte (SET), dwte += d_logits^T·lnf. */
void tied_head_backward(float *d_lnf, float *dwte, const float *d_logits, const float *lnf,
                        const float *wte, int M);

/* model.h:56 / model.c:64-77: logits[t,v] = x[t]·wte[v], t < num_tokens. */
void lm_head(float *logits, const float *x, const float *wte, int num_tokens);

/* transformer.c:174-195: out(N) = in(K)·W(K,N) + bias (bias may be NULL). */
void proj_token(float *out, const float *in, const float *W, const float *bias, int K, int N);

/* generate.c:95-107: same contract as proj_token. */
void matvec(float *out, const float *x, const float *W, const float *b, int K, int N);

/* train.c:339-370: causal multi-head attention over B sequences of T tokens;
 * q/k/v/att are (B*T) x D_MODEL (head h at columns [h*D/H, (h+1)*D/H)),
 * probs [B*H][T][T] normalised for j <= i. Entries j > i are written 0 (the
 * CPU original leaves them untouched; gpu_kernels.cu:279 zeroes them).
 * D_MODEL from pcl_set_model_dims, N_HEADS from pcl_set_attn_dims. */
void attention_forward(const float *q, const float *k, const float *v, float *att, float *probs,
                       int B, int T);

/* train.c:374-407: given d_att and the forward's probs, dq, dk, dv ACCUMULATE
 * the attention gradients (same layouts and dims as attention_forward). */
void attention_backward(float *dq, float *dk, float *dv, const float *d_att, const float *q,
                        const float *k, const float *v, const float *probs, int B, int T);

/* train.c:449-465: softmax cross-entropy over M rows of VOCAB_SIZE logits
 * (pcl_set_model_dims); fills d_logits = (softmax - onehot)/M, returns the mean
 * of -log(p[target] + 1e-30). */
float cross_entropy(const float *logits, const int *targets, float *d_logits, int M);

/* gemm_bench.c:225-236: per-tensor symmetric quantisation to u8 (+128 offset),
 * K padded to Kpad with 128. Returns the scale amax*fl(1/127). */
float quantize_A(const float *A, uint8_t *Au, int M, int K, int Kpad);

/* gemm_bench.c:238-259: per-column s8 quantisation into the VNNI panel layout
 * Bp[p*(Kpad/4)*64 + kg*64 + i*4 + j] = Bq[kg*4+j][p*16+i]; colsum[n] = sum_k Bq.
 * N must be a multiple of 16 (gemm_bench.c:245). */
void quantize_B_pack(const float *B, int8_t *Bp, float *bscale, int32_t *colsum, int K, int N,
                     int Kpad);

/* gemm_bench.c:278-285: C(M,N) = float(sum_k Au·Bq - corr[n]) * dq[n] over the
 * VNNI layout above; int32 result bit-exact, dequant in the reference op order. */
void gemm_int8_kernel(const uint8_t *Au, int Kpad, const int8_t *Bp, const int32_t *corr,
                      const float *dq, float *C, int M, int N);

/* ============================== 2. device-pointer drop-ins =============== */

/* gpu_kernels.h:39 -- one-time set-up; here an alias of pcl_init. */
void gpu_init(void);
/* gpu_kernels.h:48: C(M,N) = A(M,K)·B(K,N) + bias (bias may be NULL). */
void gemm_nn(const float *A, const float *B, const float *bias, float *C, int M, int K, int N);
/* gpu_kernels.h:49: C(M,N) ?= A(M,K)·B(N,K)^T; accum != 0 adds into C. */
void gemm_nt(const float *A, const float *B, float *C, int M, int K, int N, int accum);
/* gpu_kernels.h:50: C(K,N) += A(M,K)^T·B(M,N). */
void gemm_tn(const float *A, const float *B, float *C, int M, int K, int N);
/* gpu_kernels.h:51: db(N) += colsum(dY(M,N)). */
void bias_bwd(float *db, const float *dY, int M, int N);
/* gpu_kernels.h:56-58 (gpu_kernels.cu:228-251): Y = tanh-GELU(X); dX = dY * GELU'(X)
 * (SET); C = A + B -- n elements each. */
void gelu_fwd(float *Y, const float *X, long n);
void gelu_bwd(float *dX, const float *dY, const float *X, long n);
void vec_add(float *C, const float *A, const float *B, long n);
/* gpu_kernels.h:63-64: causal attention of B_SIZE x T_SIZE tokens, DIM wide,
 * N_HEADS heads (pcl_set_attn_dims / pcl_set_model_dims); probs [B*H][T][T]
 * normalised, zero above the diagonal (gpu_kernels.cu:264-281, 403-432). */
void attn_fwd(const float *Q, const float *K, const float *V, float *att, float *probs);
/* gpu_kernels.h:65-68: dQ, dK, dV SET (gpu_kernels.cu:437-486, beta = 0) from
 * dAtt and the forward's probs; scratch holds B*H*T*T floats (dS). */
void attn_bwd(float *dQ, float *dK, float *dV, float *scratch, const float *dAtt, const float *Q,
              const float *K, const float *V, const float *probs);
/* gpu_kernels.h:78-81 (gpu_kernels.cu:518-547): M_ROWS = B_SIZE*T_SIZE rows
 * (pcl_set_attn_dims) of VOCAB_SIZE logits (pcl_set_model_dims); the mean loss
 * is ADDED into *loss_dev (zero it first); dlogits = (softmax - onehot)/M_ROWS
 * and may be the logits buffer itself. */
void ce_fwd_bwd(const float *logits, const int *targets, float *dlogits, float *loss_dev);

/* ============================== 3. native entry points =================== */

#define PCL_OP_N 0 /* operand stored as written: A is M x K, B is K x N */
#define PCL_OP_T 1 /* operand stored transposed: A is K x M, B is N x K */

/* FP32 GEMM on the f32 MFMA: C(M,N) = (accumulate ? C : 0) + op(A)·op(B) + bias.
 * Decode shapes (M <= 8, opA == N) run the HBM-bound GEMV kernels instead.
 * Replaces tensor.c:34-53, train.c:181-252/412-447, gpu_kernels.cu:112-138. */
int pcl_sgemm(int opA, int opB, int M, int N, int K, const float *A, int lda, const float *B,
              int ldb, const float *bias, int accumulate, float *C, int ldc, void *stream);

/* FP32 GEMM with a fused epilogue on v = op(A)·op(B) + bias (the elementwise pass
 * that follows the product in train.c:522-527/550-552 and gpu_kernels.cu:228-251):
 *   PCL_EPI_GELU      C = 0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))) (train.c:314-322);
 *                     aux_out (if not NULL) also receives v, the pre-activation the
 *                     backward needs (train.c keeps it as A_h)
 *   PCL_EPI_RESID     C = aux_in + v         (the residual adds, train.c:522, 527)
 *   PCL_EPI_GELU_BWD  C = v * GELU'(aux_in)  (dX of FF2 times gelu_backward, train.c:324-333)
 * aux arrays are M x N with leading dimension ld_aux; C is set (no accumulate).
 * Fused into the GEMM kernel for NN (GELU, RESID) and NT (GELU_BWD) products on
 * aligned operands with K % 32 == 0 and a full grid; otherwise the same result
 * comes from the GEMM plus one elementwise pass. PCL_EPI_NONE is pcl_sgemm. */
#define PCL_EPI_NONE 0
#define PCL_EPI_GELU 1
#define PCL_EPI_RESID 2
#define PCL_EPI_GELU_BWD 3
int pcl_sgemm_ex(int opA, int opB, int M, int N, int K, const float *A, int lda, const float *B,
                 int ldb, const float *bias, int epilogue, const float *aux_in, float *aux_out,
                 int ld_aux, float *C, int ldc, void *stream);

/* Elementwise passes of the reference GPU API with an explicit stream. */
int pcl_gelu_fwd(float *Y, const float *X, long n, void *stream);
int pcl_gelu_bwd(float *dX, const float *dY, const float *X, long n, void *stream);
int pcl_vec_add(float *C, const float *A, const float *B, long n, void *stream);

/* FP32 GEMV (M <= 8 rows): Y(M,N) = (accumulate ? Y : 0) + X(M,K)·op(W) + bias.
 * opW == PCL_OP_N: W is K x N (generate.c:95-107, transformer.c:174-195);
 * opW == PCL_OP_T: W is N x K (the tied head, model.c:64-77, generate.c:176-182). */
int pcl_sgemv(int opW, int M, int N, int K, const float *X, int ldx, const float *W, int ldw,
              const float *bias, int accumulate, float *Y, int ldy, void *stream);

/* pcl_sgemv without any allocation. No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments, kernels and results
 * as pcl_sgemv; the split-K partial sums go to a static 4 MiB device array held
 * by each GPU until the process ends, instead of a per-stream workspace.
 * Shapes needing more scratch than that fail with PCL_ERR_RANGE before any
 * launch. Every call on one GPU shares that array: calls that overlap on one
 * GPU (e.g. on two streams) race and must be ordered by the caller. */
int pcl_sgemv_noalloc(int opW, int M, int N, int K, const float *X, int ldx, const float *W,
                      int ldw, const float *bias, int accumulate, float *Y, int ldy, void *stream);

/* db(N) += colsum(dY) (gpu_kernels.cu:102-108), fixed m order per column. */
int pcl_bias_bwd(float *db, const float *dY, int M, int N, int ld, void *stream);

/* Softmax cross-entropy (train.c:449-465, gpu_kernels.cu:518-547) over M rows
 * of V logits (leading dimension ld): dlogits (ldd) = (p - onehot)/M with
 * p = expf(l - max)·(1/sum expf(l - max)); *loss += mean of -log(p[t] + 1e-30)
 * (row terms in double, summed in a fixed order). dlogits may be logits itself
 * (same ld) and must not otherwise overlap it. A target outside [0, V) makes
 * the loss NaN. Two passes over the logits, one write. */
int pcl_cross_entropy(const float *logits, int ld, const int *targets, float *dlogits, int ldd,
                      int M, int V, float *loss, void *stream);

/* The tied head and its cross-entropy, forward and backward in one call
 * (train.c:412-465 as the trainer runs them, :531 then :718 then :542;
 * train_kaggle.cu:165-174 + :409 on the GPU): over rows of at most chunk_bytes
 * of logits at a time (<= 0: 1 GiB; the 350M shape 4096 x 50257 fits whole),
 *   logits = lnf(M,D)·wte(V,D)^T, the cross-entropy above in place,
 *   d_lnf(M,D)  = dlogits·wte          (SET; skipped when NULL),
 *   dwte(V,D)  += dlogits^T·lnf        (ACCUMULATE; skipped when NULL),
 *   *loss      += mean loss.
 * The full M x V logits never exist at once beyond one chunk, which lives in the
 * library's per-stream workspace. All pointers are device memory, rows dense. */
int pcl_head_ce(const float *lnf, const float *wte, const int *targets, int M, int D, int V,
                float *loss, float *d_lnf, float *dwte, long chunk_bytes, void *stream);

/* Causal multi-head attention forward on the f32 MFMA (train.c:339-370,
 * gpu_kernels.cu:264-281/403-432), one fused launch: Q, K, V are (B*T) x ld
 * row-major with head h at columns [h*dh, (h+1)*dh); att (B*T) x ld_att gets
 * att_i = sum_{j<=i} p_ij v_j, p_ij = softmax_j(q_i.k_j / sqrtf(dh)). probs is
 * NULL or [B*H][T][T] (row (b*H+h)*T + i; p for j <= i, 0 above). dh must be
 * 32, 64 or 128; ld and ld_att multiples of 4; Q, K, V, att 16-byte aligned.
 * Q/K/V may be column slices of one fused (B*T) x 3D QKV buffer (ld = 3D). */
int pcl_attn_fwd(const float *Q, const float *K, const float *V, int ld, float *att, int ld_att,
                 float *probs, int B, int T, int H, int dh, void *stream);

/* The forward without probabilities, in one pass (a running row maximum;
 * pcl_attn_fwd takes the same path when probs is NULL): no counterpart in the
 * reference's interface, whose forward always stores probabilities. att as
 * pcl_attn_fwd (within fp32 rounding of it); lse NULL or (B*H) x T floats,
 * lse[(b*H + h)*T + i] = log sum_{j<=i} exp(q_i.k_j / sqrtf(dh)), so that
 * p_ij = exp(q_i.k_j / sqrtf(dh) - lse_i). Limits as pcl_attn_fwd. */
int pcl_attn_fwd_lse(const float *Q, const float *K, const float *V, int ld, float *att, int ld_att,
                     float *lse, int B, int T, int H, int dh, void *stream);

/* Its backward from the stored probs (train.c:374-407, gpu_kernels.cu:437-486):
 *   dP_ij = dAtt_i.v_j, D_i = sum_j p_ij dP_ij, dS_ij = p_ij (dP_ij - D_i)/sqrtf(dh),
 *   dQ_i = sum_j dS_ij k_j, dK_j = sum_i dS_ij q_i, dV_j = sum_i p_ij dAtt_i.
 * dQ, dK, dV ((B*T) x ld_grad) are set, or added to with accumulate != 0
 * (train.c's convention). scratch: NULL (library workspace) or B*H*T*T floats,
 * left holding dS for j <= i. Two launches on the stream; layouts and limits as
 * pcl_attn_fwd, dAtt (B*T) x ld_att 16-byte aligned. */
int pcl_attn_bwd(float *dQ, float *dK, float *dV, int ld_grad, float *scratch, const float *dAtt,
                 int ld_att, const float *Q, const float *K, const float *V, int ld,
                 const float *probs, int B, int T, int H, int dh, int accumulate, void *stream);

/* pcl_attn_bwd given also the forward's output att ((B*T) x ld_o, ld_o a
 * multiple of 4, 16-byte aligned): D_i = dAtt_i . att_i replaces the pass over
 * P and dP that forms D_i = sum_j p_ij dP_ij (the same sum, since att_i =
 * sum_j p_ij v_j), so the query-block kernel reads P once and issues dP once.
 * Results within fp32 rounding of pcl_attn_bwd. No counterpart in the
 * reference's interface, whose backward is not handed the forward's output. */
int pcl_attn_bwd_ex(float *dQ, float *dK, float *dV, int ld_grad, float *scratch,
                    const float *dAtt, int ld_att, const float *Q, const float *K, const float *V,
                    int ld, const float *probs, const float *att, int ld_o, int B, int T, int H,
                    int dh, int accumulate, void *stream);

/* ---- INT8: u8 activations x s8 weights -> int32 (gemm_bench.c:212-285) ----
 * Weights live in the GPU-native packed layout: N rows of Kp = pcl_s8_kpad(K)
 * bytes (K-contiguous per output column, zero-padded), i.e. B^T. */
int pcl_s8_kpad(int K);
size_t pcl_s8_packed_bytes(int K, int N);
/* Pack row-major s8 B(K,N) (ldb) into the native layout; colsum (may be NULL)
 * receives sum_k B[k,n]. */
int pcl_pack_b_s8(const int8_t *B, int ldb, int K, int N, int8_t *Bpk, int32_t *colsum,
                  void *stream);
/* Repack the reference VNNI layout (gemm_bench.c:245-257; N % 16 == 0) into
 * the native layout; colsum (may be NULL) as above. */
int pcl_pack_b_vnni(const int8_t *Bp, int K, int Kpad, int N, int8_t *Bpk, int32_t *colsum,
                    void *stream);

/* C32(M,N) = sum_k (A[m,k]-128)·B[k,n] exactly (the reference's fixed-up `v`,
 * gemm_bench.c:216-217, 274). A is M x K u8 with leading dim lda. */
int pcl_gemm_u8s8_i32(const uint8_t *A, int lda, const int8_t *Bpk, int32_t *C, int ldc, int M,
                      int N, int K, void *stream);

/* C(M,N) = float(v + col_off[n]) * dq with v as above and
 *   dq = sa[m]*sb[n]  (per-token x per-channel) when sa != NULL,
 *   dq = sb[n]        (gemm_bench.c:272-275, sb = a_scale*bscale) otherwise.
 * col_off may be NULL; the reference's `corr` maps to col_off = 128*colsum-corr. */
int pcl_gemm_u8s8_dq(const uint8_t *A, int lda, const int8_t *Bpk, const int32_t *col_off,
                     const float *sa, const float *sb, float *C, int ldc, int M, int N, int K,
                     void *stream);

/* Decode GEMV forms of the two calls above for M <= 8 (HBM-bound kernel). */
int pcl_gemv_u8s8_i32(const uint8_t *X, int ldx, const int8_t *Bpk, int32_t *Y, int ldy, int M,
                      int N, int K, void *stream);
int pcl_gemv_u8s8_dq(const uint8_t *X, int ldx, const int8_t *Bpk, const int32_t *col_off,
                     const float *sa, const float *sb, float *Y, int ldy, int M, int N, int K,
                     void *stream);

/* ---- measured roofs: gemm_bench's measure_peak_int8_gops (gemm_bench.c:287-301),
 * measure_peak_gflops (:309-325) and measure_bandwidth_gbs (:195-210) on the GPU.
 * Sustained matrix-core rate with the operands held in registers (eight waves
 * per CU; four independent 32x32x32 accumulators each for i8, eight 16x16x4
 * for f32): data 0 = i8 MFMA on uniformly random bytes (the gemm_bench INT8
 * data; the clock drops with the operands' switching), 1 = i8 on zeros, 2 = f32
 * MFMA on uniform random floats. *rate in TOP/s (i8) or TFLOP/s (f32); best of 5
 * launches after 30 warm-up launches. */
int pcl_measure_peak_mfma(int data, double *rate);
/* HBM over arrays of bytes_per_array (at least 64 MiB; use > 256 MB to leave
 * the Infinity Cache), 16-byte non-temporal accesses, best of 5, in GB/s:
 * gbs[0] STREAM triad a = b + s*c (3 arrays of traffic), gbs[1] copy (2),
 * gbs[2] read only (1), gbs[3] write only (1). Allocates the arrays. */
int pcl_measure_bandwidth(long bytes_per_array, double gbs[4]);
/* The operand feed of the INT8 GEMM's 128x128 tiles: one workgroup per output
 * tile of an M x N x K product streams the tile's A and B panels (rows of K
 * bytes) into LDS the way the kernels' producer waves do, in their tile order,
 * with no products; *gbs = GB/s into LDS, best of 5 batches of 50
 * back-to-back launches after one warm-up batch. M, N, K positive multiples of 128 (PCL_ERR_INVALID_ARG
 * otherwise). The K loop of a grid of one such tile per CU cannot run faster
 * than this feed. No counterpart in the reference (its roofs are gemm_bench's
 * CPU ones). Allocates its operands. */
int pcl_measure_lds_feed(int M, int N, int K, double *gbs);
/* The same operand stream (addresses, tile order, one workgroup per tile) read
 * into registers instead of LDS: eight waves per tile, each with the loads of
 * two K tiles in flight. *gbs = GB/s read, measured as pcl_measure_lds_feed;
 * the same arguments and errors. When the two agree, the feed's ceiling is the
 * path from L2 to the CU rather than the LDS DMA. No counterpart in the
 * reference. Allocates its operands. */
int pcl_measure_tile_read(int M, int N, int K, double *gbs);

/* ---- grouped decode GEMV: many independent products in one launch ----
 * Not a reference function: the reference runs its decode products one call
 * at a time (generate.c:95-107 matvec, three of them on one input for the
 * separate Wq, Wk, Wv; transformer.c:174-195 proj_token). A group streams
 * the weights of many independent products together (the projections of one
 * input, one layer for several sequences, a whole sweep), so short products
 * do not each pay for a launch. Each product is the single call's product:
 *   PCL_GEMV_F32_N  Y(M,N) = (accumulate ? Y : 0) + X(M,K)·W + bias, W K x N
 *                   (pcl_sgemv with PCL_OP_N);
 *   PCL_GEMV_F32_T  the same with W N x K (pcl_sgemv with PCL_OP_T);
 *   PCL_GEMV_U8S8   X u8 (+128 offset), W packed s8 (pcl_pack_b_s8; ldw = its
 *                   row length pcl_s8_kpad(K)): int32 Y when sb is NULL
 *                   (pcl_gemv_u8s8_i32), else Y = float(v + col_off[n]) *
 *                   (sa ? sa[m]*sb[n] : sb[n]) (pcl_gemv_u8s8_dq).
 * FP32 within the 1e-4 bar, INT8 bit-exact, as the single calls. Products must
 * be independent: no product's Y may share memory with another's X, W or Y. */
#define PCL_GEMV_F32_N 0
#define PCL_GEMV_F32_T 1
#define PCL_GEMV_U8S8 2
typedef struct pcl_gemv_desc {
    int kind, M, N, K;
    const void *X;
    int ldx;
    const void *W;
    int ldw;
    const float *bias; /* fp32 kinds; may be NULL */
    int accumulate;    /* fp32 kinds */
    const int32_t *col_off; /* PCL_GEMV_U8S8; may be NULL */
    const float *sa, *sb;   /* PCL_GEMV_U8S8 */
    void *Y;
    int ldy;
} pcl_gemv_desc;
typedef struct pcl_gemv_group pcl_gemv_group;
/* Validates the n products, plans one launch (each block owns a strip of one
 * product over its whole K, largest first) and copies the plan to the device:
 * the group's only allocation. Beyond the single calls it needs 1 <= M <= 8,
 * K >= 1, 16-byte aligned W with ldw % 4 == 0 and N % 4 == 0 (F32_N) or
 * K % 4 == 0 (F32_T), packed rows of ldw >= pcl_s8_kpad(K) (U8S8), and staged
 * operands within 112 KB of LDS per block: M' * K' * 4 bytes for fp32 (K'
 * = K rounded up to 64 for F32_T, to 128 for F32_N), M' * (pcl_s8_kpad(K) +
 * 16) + 16384 bytes for U8S8, with M' the group's largest M rounded up to 1,
 * 2, 4 or 8 (PCL_ERR_RANGE otherwise, at creation). The descriptors' pointers
 * are kept: the buffers must outlive the group. */
int pcl_gemv_group_create(const pcl_gemv_desc *descs, int n, pcl_gemv_group **group);
/* One launch computing every product of the group (asynchronous on stream). */
int pcl_gemv_group_run(const pcl_gemv_group *group, void *stream);
void pcl_gemv_group_free(pcl_gemv_group *group);

/* ---- quantisers (gemm_bench.c:225-259 rules: scale = amax * fl(1/127), the
 * reference's -ffast-math build of amax/127.0f (README.md:104), with amax
 * starting at 1e-8; q = clamp(lroundf(x * (1/scale)), -127, 127)) ---- */
/* Per-tensor: Au = q + 128, Kpad columns (padding 128); *scale_dev = scale. */
int pcl_quantize_a_tensor(const float *A, int M, int K, uint8_t *Au, int Kpad, float *scale_dev,
                          void *stream);
/* Per-row (per-token): sa[m] = amax(row m) * fl(1/127). */
int pcl_quantize_a_rows(const float *A, int M, int K, uint8_t *Au, int Kpad, float *sa,
                        void *stream);
/* Per-column weights from row-major fp32 B(K,N): writes the native packed
 * layout, bscale[n], and colsum[n] (may be NULL). */
int pcl_quantize_b_cols(const float *B, int K, int N, int8_t *Bpk, float *bscale, int32_t *colsum,
                        void *stream);
/* Same quantisation written in the reference VNNI layout (N % 16 == 0). */
int pcl_quantize_b_vnni(const float *B, int K, int N, int Kpad, int8_t *Bp, float *bscale,
                        int32_t *colsum, void *stream);

/* ============================== 4. a checkpoint on the GPU ================ */

/* A CKP1 checkpoint (train.c:633-670 writes it; generate.c:49-76 reads it:
 * int[8] {0x434B5031, block, d_model, n_heads, d_ff, n_layers, vocab, step}
 * then the tensors in registration order) loaded once into device memory with
 * its KV cache, decoded one token at a time as generate.c:118-183 does. The
 * head size d_model / n_heads must divide 256; block and d_model at most 32768
 * (d_ff too with INT8 weights). NULL on failure (the reason in pcl_last_error). */
typedef struct pcl_model pcl_model;
pcl_model *pcl_model_load(const char *path);
/* weights: PCL_W_FP32 (as pcl_model_load) or PCL_W_INT8: every projection and
 * the tied head quantised once at load, per output column (the rule of
 * gemm_bench.c:238-259), and each product's input quantised per token as it is
 * made (per-row u8, gemm_bench.c:225-236's rule per row): INT8 GEMVs with
 * int32 sums and per-row x per-column dequant; embeddings, LayerNorm, biases,
 * attention and the residual stream stay fp32. */
#define PCL_W_FP32 0
#define PCL_W_INT8 1
pcl_model *pcl_model_load_ex(const char *path, int weights);
/* The checkpoint's int[8] header. */
int pcl_model_header(const pcl_model *m, int hdr[8]);
/* generate.c forward(tok, pos): one KV-cached step (the cache rows 0..pos-1 must
 * hold this sequence's earlier positions); logits (host, vocab floats) may be
 * NULL. Synchronous. */
int pcl_model_forward(pcl_model *m, int tok, int pos, float *logits);
/* Greedy decoding (generate.c:188-191 argmax, temperature 0): feeds prompt[0..
 * n_prompt) at positions 0.., then produces n_new tokens into out, each fed back
 * on the GPU (the token and position stay in device memory). use_graph != 0
 * replays one captured step per token. Needs n_prompt + n_new - 1 <= block. */
int pcl_model_generate(pcl_model *m, const int *prompt, int n_prompt, int n_new, int *out,
                       int use_graph);
void pcl_model_free(pcl_model *m);
/* Verification tap of a PCL_W_INT8 model; no counterpart in the reference, for
 * callers that check each INT8 product on its own. With on != 0, every later
 * pcl_model_forward records per INT8 product what that product used: its
 * input row before the transform (K floats: the residual stream before a
 * LayerNorm, the attention row, or the d_ff row before bias + GELU), the
 * quantised row it read (u8 = q + 128, Kp = K rounded up to 256 bytes), the
 * row's scale, and its dequantised output v * sa * sb[n] before bias and
 * residual (N floats). pcl_model_generate records nothing; on = 0 releases the
 * slots. pcl_model_capture_read copies one product of the last forward to the
 * host: layer 0..n_layers-1 with product PCL_CAP_QKV (K d_model, N 3 d_model),
 * PCL_CAP_O (d_model, d_model), PCL_CAP_FF1 (d_model, d_ff), PCL_CAP_FF2
 * (d_ff, d_model); layer n_layers with product 0 is the head (d_model, vocab).
 * Any of xin, xq, sa, y may be NULL. */
#define PCL_CAP_QKV 0
#define PCL_CAP_O 1
#define PCL_CAP_FF1 2
#define PCL_CAP_FF2 3
int pcl_model_capture(pcl_model *m, int on);
int pcl_model_capture_read(const pcl_model *m, int layer, int product, float *xin, uint8_t *xq,
                           float *sa, float *y);

#ifdef __cplusplus
}
#endif
#endif /* PCL_HIP_H */
