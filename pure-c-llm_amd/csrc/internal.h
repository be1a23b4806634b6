// internal.h -- shared declarations between the HIP kernel files and the C-ABI
// shim of libpcl_hip. Not part of the public ABI (that is include/pcl_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pcl {

// Scratch memory that a launcher may use: the partial sums of a split-K GEMV
// ([splits][M][strips * rows per strip]), written by the GEMV kernel and
// summed by its reduce kernel on the same stream.
struct Workspace {
    void *buf = nullptr;  // bytes_cap bytes
    size_t bytes_cap = 0;
};

// Split-K GEMV geometry chosen by the launchers; the shim sizes the workspace.
struct GemvPlan {
    int strips;      // blocks along N
    int splits;      // blocks along K
    int kchunk;      // K rows per split (multiple of the kernel's K step)
    size_t part_bytes;  // workspace bytes for partials (0 when splits == 1)
    int cw = 64;     // columns per strip (sgemv over K x N weights: 64 or 16)
};

// ---- FP32 GEMM (sgemm.hip) ----
// Tile configuration and K split chosen for a shape; with splits > 1 the
// partial products ([splits][M][N] fp32, part_bytes) go to the workspace and a
// second kernel adds them in split order.
struct SgemmPlan {
    int cfg;
    int splits;
    int kchunk;         // K per split (a multiple of 64 when split)
    size_t part_bytes;  // workspace bytes (0 when splits == 1)
};
// a_kcontig: op(A) is K-contiguous (row-major A, no transpose), which the
// 32x64 small-grid configuration needs
SgemmPlan plan_sgemm(int M, int N, int K, bool a_kcontig = false);
// Epilogues on v = op(A).op(B) + bias (accumulate must be 0 with any but NONE):
//   EPI_GELU: aux_out[m,n] <- v (when aux_out != NULL), C <- gelu(v)
//   EPI_RESID: C <- aux_in[m,n] + v;  EPI_GELU_BWD: C <- v * gelu'(aux_in[m,n])
// aux arrays are M x N with leading dimension ld_aux.
enum SgemmEpi { EPI_NONE = 0, EPI_GELU = 1, EPI_RESID = 2, EPI_GELU_BWD = 3 };
// C(M,N) = (accumulate ? C : 0) + op(A)(M,K) . op(B)(K,N) + bias, then the epilogue
// a_kcontig: element (m,k) of A at A[m*lda + k] (else A[k*lda + m]);
// b_kcontig: element (k,n) of B at B[n*ldb + k] (else B[k*ldb + n]).
hipError_t launch_sgemm(const SgemmPlan &p, bool a_kcontig, bool b_kcontig, int M, int N, int K,
                        const float *A, long lda, const float *B, long ldb, const float *bias,
                        int accumulate, float *C, long ldc, const Workspace &ws,
                        hipStream_t stream, int epi = EPI_NONE, const float *aux_in = nullptr,
                        float *aux_out = nullptr, long ld_aux = 0);
// dst (rows x cols, ldd % 4 == 0, 16-byte aligned) <- src (lds, any alignment)
hipError_t launch_copy_rows(float *dst, long ldd, const float *src, long lds, int rows, int cols,
                            hipStream_t stream);
// op 0: out = gelu(a); 1: out = a * gelu'(b) (a = upstream gradient, b =
// pre-activation); 2: out = a + b -- n elements (gpu_kernels.cu:228-251)
hipError_t launch_elementwise(int op, long n, float *out, const float *a, const float *b,
                              hipStream_t stream);

// ---- INT8 GEMM (igemm.hip) ----
// out_mode 0: C is int32 v; 1: C = float(v+off)*sb[n]; 2: C = float(v+off)*(sa[m]*sb[n])
// Requires K % 256 == 0, lda % 16 == 0, A and Bpk 16-byte aligned, and packed
// weight rows of ldb >= K bytes (the packers use roundup(K_true, 256), zero
// past the true K; A columns past the true K must be 0x80).
// tile_ctr: IGEMM_TILE_CTRS ints, zero between launches (launch_igemm_tiles_init
// once; the kernels that use them leave them zero), private to the stream; or
// NULL (persistent kernels then give each workgroup fixed tiles).
constexpr int IGEMM_TILE_CTRS = 16;  // a fetch counter and a done counter per XCD
hipError_t launch_igemm(int out_mode, int M, int N, int K, const uint8_t *A, long lda,
                        const int8_t *Bpk, long ldb, const int32_t *col_off, const float *sa,
                        const float *sb, void *C, long ldc, int *tile_ctr, hipStream_t stream);
hipError_t launch_igemm_tiles_init(int *ctr, hipStream_t s);
// Copy A (M x K, lda) into dst (M x Kd, Kd >= K), padding with 0x80.
hipError_t launch_pad_a_u8(const uint8_t *A, long lda, int M, int K, uint8_t *dst, int Kd,
                           hipStream_t stream);

// ---- causal attention (attn.hip) ----
// Q, K, V: (B*T) x ld row-major, head h at columns [h*dh, (h+1)*dh); O: (B*T) x
// ldo; P: NULL or [B*H][T][T] probabilities (zero above the diagonal).
// dh in {32, 64, 128}; ld, ldo multiples of 4 and 16-byte aligned bases.
// Without P the one-pass kernel runs, and lse (NULL or (B*H) x T floats)
// receives each row's log-sum-exp of the scaled scores.
hipError_t launch_attn_fwd(const float *Q, const float *K, const float *V, long ld, float *O,
                           long ldo, float *P, int B, int T, int H, int dh, float scale,
                           hipStream_t stream, float *lse = nullptr);

// Backward from the stored probabilities P: dQ, dK, dV ((B*T) x ldg) set or,
// with accumulate, added to; dS ([B*H][T][T]) is written as scratch (entries
// j <= i of each causal row). dO is (B*T) x ldo. Ofw (NULL, or the forward's
// output, (B*T) x ldfw) gives D_i = dO_i . att_i directly instead of the
// query-block kernel's first pass over P and dP.
hipError_t launch_attn_bwd(const float *dO, long ldo, const float *Q, const float *K,
                           const float *V, long ld, const float *P, float *dS, float *dQ,
                           float *dK, float *dV, long ldg, int B, int T, int H, int dh,
                           float scale, int accumulate, hipStream_t stream,
                           const float *Ofw = nullptr, long ldfw = 0);

// ---- decode step (decode.hip); tokpos = {token, position} in device memory ----
hipError_t launch_decode_embed(const float *wte, const float *wpe, float *x, int D,
                               const int *tokpos, hipStream_t s);
// dh = D / H must divide 256; the cache holds blk rows of D floats; bqkv
// (3*D, may be NULL) is added to qkv inside the kernel
hipError_t launch_decode_attn(const float *qkv, const float *bqkv, float *kc, float *vc, float *att,
                              int D, int H, int blk, const int *tokpos, hipStream_t s);
// x += t + b (when t), q/sa = per-row quantised LayerNorm(x; g, beta), Kpad bytes
hipError_t launch_decode_add_ln_quant(float *x, const float *t, const float *b, const float *g,
                                      const float *beta, uint8_t *q, float *sa, int D, int Kpad,
                                      hipStream_t s);
// q/sa = per-row quantised gelu(h + b), Kpad bytes
hipError_t launch_decode_bias_gelu_quant(const float *h, const float *b, uint8_t *q, float *sa,
                                         int F, int Kpad, hipStream_t s);
hipError_t launch_decode_argmax(const float *logits, int V, int *tokpos, int *out, int out_cap,
                                hipStream_t s);

// ---- softmax cross-entropy (ce.hip) ----
// Rows [0, M) of logits (ld) -> dl (ldd, may alias logits): (p - onehot) / rows,
// columns [V, pad) of dl set to 0 (pad >= V); row_loss[m] = -log(p[t] + 1e-30)
// (NaN for a target outside [0, V)).
hipError_t launch_cross_entropy(const float *logits, long ld, const int *targets, float *dl,
                                long ldd, int M, int V, int pad, int rows, double *row_loss,
                                hipStream_t s);
// *loss += (float)(sum of row_loss[0..M) / rows)
hipError_t launch_ce_loss(const double *row_loss, int M, int rows, float *loss, hipStream_t s);

// Error reporting and device set-up of the C-ABI shim, for other translation
// units of the library (model.cpp).
int shim_error(int status, const char *msg);
int shim_init();
// launch_sgemv_xf on the stream's workspace (status as the C-ABI calls)
int sgemv_xf(int xf, int N, int K, const float *X, const float *W, int ldw,
             const float *g, const float *b, const float *bias, int accumulate, float *Y,
             void *stream);

// ---- measured roofs (roofs.hip) ----
// kind 0: i8 MFMA, random bytes; 1: i8 MFMA, zeros; 2: f32 MFMA, random;
// rate in TOP/s or TFLOP/s over `cus` workgroups of eight waves.
hipError_t measure_peak_mfma(int kind, int cus, double *rate, hipStream_t s);
// GB/s over arrays of bytes_per_array: gbs[0] STREAM triad, [1] copy, [2]
// read only, [3] write only.
hipError_t measure_bandwidth(long bytes_per_array, double gbs[4], hipStream_t s);
// GB/s into LDS of the operand stream of a 128x128-tile INT8 GEMM (M, N, K
// multiples of 128; M*K and N*K below 2^31), no products.
// vgpr: the same stream read into registers (8 waves, 2 K tiles in flight)
hipError_t measure_lds_feed(int M, int N, int K, double *gbs, hipStream_t s, bool vgpr = false);

// ---- GEMV (gemv.hip) ----
GemvPlan plan_sgemv(int w_trans, int M, int N, int K);
// Grouped GEMV: one launch over independent products. Device descriptor of
// one product's work item (validated by the shim); out_mode of GG_U8S8: 0
// int32, 1 float(v)*sb[n], 2 float(v)*(sa[m]*sb[n]); xld: staged activation
// row stride (elements) = gg_stage_ld(kind, K); strip: the item's strip of
// gg_strip_rows(kind) outputs. The launch takes one descriptor per work item;
// lds_bytes = max over products of gg_lds_bytes(kind, K, mr); mr in {1, 2, 4,
// 8} >= every product's M.
enum { GG_F32_N = 0, GG_F32_T = 1, GG_U8S8 = 2 };
struct GgDesc {
    int kind, M, N, K;
    const void *X;
    long ldx;
    const void *W;
    long ldw;
    const float *bias;
    const int32_t *col_off;
    const float *sa, *sb;
    void *Y;
    long ldy;
    int accumulate, out_mode, xld;
    int strip;  // the work item's strip (one descriptor per work item)
};
int gg_strip_rows(int kind);
int gg_stage_ld(int kind, int K);
// dynamic LDS a product needs in a group whose largest M rounds to mr
size_t gg_lds_bytes(int kind, int K, int mr);
// all_u8s8: every product is GG_U8S8 (a kernel with only that path)
hipError_t launch_gemv_group(const GgDesc *flat, int n_items, int mr,
                             size_t lds_bytes, bool all_u8s8, hipStream_t s);
// One INT8 GEMV (M <= 8 rows) on the matrix-core path of the grouped kernel:
// whole-K blocks of 64 weight rows, no split, no workspace. Applicable when
// igemv_mfma_fits (32-bit row offsets, packed rows ldb >= roundup(K, 256),
// staged operands within 64 KB of LDS).
bool igemv_mfma_fits(int M, int N, int K, long ldb);
hipError_t launch_igemv_mfma(int out_mode, int M, int N, int K, const uint8_t *X, long ldx,
                             const int8_t *Bpk, long ldb, const int32_t *col_off, const float *sa,
                             const float *sb, void *Y, long ldy, hipStream_t s);
// Size of the static split-K scratch of the allocation-free GEMV entry point,
// and its device address on the current device (hipGetSymbolAddress).
constexpr size_t GEMV_NOALLOC_SCRATCH_BYTES = (size_t)4 << 20;
hipError_t gemv_noalloc_scratch(void **dev_ptr);
// Column sums of a K x N matrix (bias_bwd): plan for launch_sgemv with x_ones.
GemvPlan plan_bias_bwd(int N, int K);
GemvPlan plan_igemv(int M, int N, int K);
// Y(M,N) = (accumulate ? Y : 0) + X(M,K) . op(W) + bias; M <= 8.
// x_ones: X is the all-ones row (bias_bwd), X/ldx unused and M must be 1.
hipError_t launch_sgemv(const GemvPlan &p, int w_trans, int M, int N, int K, const float *X,
                        long ldx, bool x_ones, const float *W, long ldw, const float *bias,
                        int accumulate, float *Y, long ldy, const Workspace &ws,
                        hipStream_t stream);
// One activation row (M = 1, X of K floats, Y of N floats) through a transform
// applied as the row is staged: xf 0 none, 1 LayerNorm over the row (g, b of
// K floats; generate.c:106-114), 2 tanh-GELU; then the N x K-weight GEMV of
// launch_sgemv (plan from plan_sgemv(1, 1, N, K)).
hipError_t launch_sgemv_xf(const GemvPlan &p, int xf, int N, int K, const float *X,
                           const float *W, long ldw, const float *g, const float *b,
                           const float *bias, int accumulate, float *Y, const Workspace &ws,
                           hipStream_t stream);
// Decode INT8 GEMV of one fp32 row: qx 0 none, 1 LayerNorm (g, b), 2
// GELU(x + b); the row quantised per row in-kernel; packed weights N x Kp
// (Kp % 256 == 0, K <= Kp <= IGEMV_Q_MAX_K); epi 0: Y = v * scale * sb[n],
// epi 1: Y += v * scale * sb[n] + bias[n].
constexpr int IGEMV_Q_MAX_K = 8192;
// A verification tap (all members null in normal use): where the kernel also
// records the quantised row it used (as u8 = q + 128, Kp bytes), that row's
// scale, and the dequantised product v * scale * sb[n] before bias and
// residual (N floats).
struct GemvTap {
    uint8_t *xq = nullptr;
    float *sa = nullptr;
    float *y = nullptr;
};
hipError_t launch_igemv_q(int qx, int epi, const float *X, const float *g, const float *b, int K,
                          const int8_t *B, int Kp, const float *sb, const float *bias, float *Y,
                          int N, hipStream_t s, const GemvTap &tap = GemvTap{});
// Its fp32 twin over weights stored N x K (rows of K floats, K % 4 == 0,
// 16-byte aligned, K <= SGEMV_Q_MAX_K): same transforms; epi 0: Y = s + bias,
// epi 1: Y += s + bias (bias may be NULL).
constexpr int SGEMV_Q_MAX_K = 16384;
hipError_t launch_sgemv_q(int qx, int epi, const float *X, const float *g, const float *b, int K,
                          const float *W, const float *bias, float *Y, int N, hipStream_t s);
// INT8 GEMV over the packed layout (ldb = Kp); out_mode as in launch_igemm.
hipError_t launch_igemv(const GemvPlan &p, int out_mode, int M, int N, int K, const uint8_t *X,
                        long ldx, const int8_t *Bpk, long ldb, const int32_t *col_off,
                        const float *sa, const float *sb, void *Y, long ldy, const Workspace &ws,
                        hipStream_t stream);

// ---- quantisers and packers (quant.hip) ----
// The activation/weight rule (gemm_bench.c:225-259 as built): amax starts at
// 1e-8f, scale = amax * fl(1/127), q = clamp(roundf(x * (1/scale)), +-127).
constexpr float AMAX_INIT = 1e-8f;
constexpr float RCP127 = 1.0f / 127.0f;  // rounded to fp32 at compile time
__device__ __forceinline__ int quant_q(float x, float inv) {
    int q = (int)roundf(x * inv);
    return q > 127 ? 127 : (q < -127 ? -127 : q);
}
hipError_t launch_quantize_a_tensor(const float *A, int M, int K, uint8_t *Au, int Kpad,
                                    float *scale_dev, unsigned *amax_bits, hipStream_t stream);
hipError_t launch_quantize_a_rows(const float *A, int M, int K, uint8_t *Au, int Kpad, float *sa,
                                  hipStream_t stream);
// layout 0: native packed (N rows of ldb bytes); 1: reference VNNI (Kpad)
hipError_t launch_quantize_b_cols(const float *B, int K, int N, int layout, int8_t *dst, long ldb,
                                  int Kpad, float *bscale, int32_t *colsum, hipStream_t stream);
hipError_t launch_pack_b_s8(const int8_t *B, long ldb_in, int K, int N, int8_t *Bpk, long ldb,
                            int32_t *colsum, hipStream_t stream);
hipError_t launch_pack_b_vnni(const int8_t *Bp, int K, int Kpad, int N, int8_t *Bpk, long ldb,
                              int32_t *colsum, hipStream_t stream);
// off[n] = 128*colsum[n] - corr[n]  (wrap-around int32)
hipError_t launch_corr_to_offset(const int32_t *colsum, const int32_t *corr, int32_t *off, int N,
                                 hipStream_t stream);

}  // namespace pcl

// ---- helpers shared by the kernels ----
namespace pcl {

// Compile-time loop: f(IC<I>{}) for I = LO .. HI-1.
template <int V>
struct IC {
    static constexpr int value = V;
};
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(IC<I>{});
        static_for<I + 1, N>(f);
    }
}

// A global-memory view of a device pointer. Accesses through a pointer the
// compiler cannot trace to a kernel argument (a field of a descriptor read
// from memory, a value passed through inline asm) are otherwise flat
// instructions, which count in lgkmcnt as well as vmcnt: every later wait for
// an LDS access then also waits for them, which serialises a weight prefetch
// with the LDS work it is meant to overlap. Only for pointers into device
// memory (never LDS).
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T *gbl(T *p) {
    return (__attribute__((address_space(1))) T *)p;
}
// The same view re-typed to V (a vector of T's elements, for 16-byte accesses).
template <typename V, typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) V *gvec(const __attribute__((address_space(1))) T *p) {
    return (const __attribute__((address_space(1))) V *)p;
}

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X
// (workgroup i runs on XCD i % 8). Renumber them so that each XCD receives a
// contiguous range of logical tiles; with the grouped tile order below those
// tiles share A rows and B columns in that XCD's private L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblk) {
    const int NX = 8;
    int xcd = bid % NX, idx = bid / NX;
    int q = nblk / NX, rem = nblk % NX;
    return xcd * q + (xcd < rem ? xcd : rem) + idx;
}

// Grouped ("super-tile") order: walk GM tile-rows down a column strip before
// moving right, so a wave of concurrent workgroups reuses a band of A and B.
__device__ __forceinline__ void tile_coords(int logical, int nbm, int nbn, int GM, int &bm,
                                            int &bn) {
    int per_group = GM * nbn;
    int group = logical / per_group;
    int first_m = group * GM;
    int gsz = nbm - first_m < GM ? nbm - first_m : GM;
    int r = logical % per_group;
    bm = first_m + r % gsz;
    bn = r / gsz;
}

}  // namespace pcl
