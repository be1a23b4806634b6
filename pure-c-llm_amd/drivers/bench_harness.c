/*
 * bench_harness.c -- timing loops for bench.py, in C so that the launch rate
 * of back-to-back kernels is set by the GPU, not by Python.
 *
 * Each pcl_bench_* call allocates its operands in HBM, fills them with
 * synthetic data (xorshift32, the generator of train.c:73-78), runs `warmup`
 * untimed steps, then times `steps` steps between two HIP events recorded on
 * the library's stream, with the device synchronised before and after. One
 * step is one call of the hot path (one kernel launch for GEMM/GEMV).
 * Weight copies can be rotated (`copies` > 1) so a memory-bound kernel reads
 * HBM rather than the 256 MB Infinity Cache.
 *
 * Built into libpcl_bench.so (see ../Makefile); only bench.py loads it.
 */
#define _POSIX_C_SOURCE 199309L /* clock_gettime */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "pcl_hip.h"

#define TRY(x)                          \
    do {                                \
        int s_ = (x);                   \
        if (s_ != PCL_OK) {             \
            rc = s_;                    \
            goto done;                  \
        }                               \
    } while (0)

static uint32_t xs32(uint32_t *s) {
    uint32_t x = *s;
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    return *s = x;
}

static void fill_f32(float *p, size_t n, uint32_t seed, float lo, float hi) {
    uint32_t s = seed ? seed : 1u;
    for (size_t i = 0; i < n; i++)
        p[i] = lo + (hi - lo) * ((float)(xs32(&s) & 0xFFFFFFu) / 16777216.0f);
}

static void fill_bytes(uint8_t *p, size_t n, uint32_t seed) {
    uint32_t s = seed ? seed : 1u;
    size_t i = 0;
    for (; i + 4 <= n; i += 4) {
        uint32_t v = xs32(&s);
        memcpy(p + i, &v, 4);
    }
    for (; i < n; i++) p[i] = (uint8_t)xs32(&s);
}

/* device buffer filled from a host staging copy */
static void *dev_f32(size_t n, uint32_t seed, float lo, float hi) {
    float *h = malloc(n * sizeof(float) + 16);
    if (!h) return NULL;
    fill_f32(h, n, seed, lo, hi);
    void *d = pcl_malloc(n * sizeof(float));
    if (d && pcl_memcpy_h2d(d, h, n * sizeof(float)) != PCL_OK) {
        pcl_free(d);
        d = NULL;
    }
    free(h);
    return d;
}

static void *dev_bytes(size_t n, uint32_t seed) {
    uint8_t *h = malloc(n + 16);
    if (!h) return NULL;
    fill_bytes(h, n, seed);
    void *d = pcl_malloc(n);
    if (d && pcl_memcpy_h2d(d, h, n) != PCL_OK) {
        pcl_free(d);
        d = NULL;
    }
    free(h);
    return d;
}

typedef int (*step_fn)(void *ctx, int i);

/* warmup + timed loop shared by every benchmark */
/* Untimed warm-up: the `warmup` steps asked for, then more until the part has
 * been busy for at least WARM_MIN_MS. An MI355X brought out of idle (or out of
 * the host-side set-up between two measurements) raises its clock over ~10-20 ms
 * of load; steps timed before that read 5-15% slow. *next = the index of the
 * first timed step (weight copies keep rotating through the warm-up). */
#define WARM_MIN_MS 20.0
static double now_ms(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec * 1e3 + (double)t.tv_nsec * 1e-6;
}

static int warm_up(step_fn fn, void *ctx, int warmup, int *next) {
    int rc = PCL_OK, i = 0;
    const double t0 = now_ms();
    for (; i < warmup; i++) TRY(fn(ctx, i));
    TRY(pcl_stream_synchronize());
    while (now_ms() - t0 < WARM_MIN_MS) {
        for (int j = 0; j < 8; j++, i++) TRY(fn(ctx, i));
        TRY(pcl_stream_synchronize());
    }
done:
    *next = i;
    return rc;
}

static int time_steps(step_fn fn, void *ctx, int warmup, int steps, double *ms_total) {
    int rc = PCL_OK, first = 0;
    void *e0 = NULL, *e1 = NULL;
    float ms = 0.f;
    TRY(warm_up(fn, ctx, warmup, &first));
    e0 = pcl_event_create();
    e1 = pcl_event_create();
    if (!e0 || !e1) {
        rc = PCL_ERR_HIP;
        goto done;
    }
    TRY(pcl_event_record(e0));
    for (int i = 0; i < steps; i++) TRY(fn(ctx, first + i));
    TRY(pcl_event_record(e1));
    TRY(pcl_event_elapsed_ms(e0, e1, &ms));
    TRY(pcl_stream_synchronize());
    *ms_total = ms;
done:
    if (e0) pcl_event_destroy(e0);
    if (e1) pcl_event_destroy(e1);
    return rc;
}

/* Each of `steps` steps between its own pair of events (recorded on the
 * stream right before and after the step's launch): the average duration of
 * one launch as a kernel trace sees it, without the gaps between launches. */
static int time_each(step_fn fn, void *ctx, int warmup, int steps, double *us_avg) {
    int rc = PCL_OK, first = 0;
    void **ev = calloc((size_t)2 * steps, sizeof(void *));
    double tot = 0;
    if (!ev) return PCL_ERR_OOM;
    TRY(warm_up(fn, ctx, warmup, &first));
    for (int i = 0; i < 2 * steps; i++)
        if (!(ev[i] = pcl_event_create())) {
            rc = PCL_ERR_HIP;
            goto done;
        }
    TRY(pcl_stream_synchronize());
    for (int i = 0; i < steps; i++) {
        TRY(pcl_event_record(ev[2 * i]));
        TRY(fn(ctx, first + i));
        TRY(pcl_event_record(ev[2 * i + 1]));
    }
    TRY(pcl_stream_synchronize());
    for (int i = 0; i < steps; i++) {
        float ms = 0.f;
        TRY(pcl_event_elapsed_ms(ev[2 * i], ev[2 * i + 1], &ms));
        tot += ms;
    }
    *us_avg = 1e3 * tot / steps;
done:
    for (int i = 0; i < 2 * steps; i++)
        if (ev[i]) pcl_event_destroy(ev[i]);
    free(ev);
    return rc;
}

/* ------------------------------------------------------------ INT8 GEMM ---- */
typedef struct {
    int M, N, K, out_mode, copies;
    void *A, *Bq, *Bpk[8], *sa, *sb, *C;
} igemm_ctx;

static int igemm_step(void *c_, int i) {
    igemm_ctx *c = c_;
    void *B = c->Bpk[i % c->copies];
    if (c->out_mode == 0)
        return pcl_gemm_u8s8_i32(c->A, c->K, B, c->C, c->N, c->M, c->N, c->K, NULL);
    return pcl_gemm_u8s8_dq(c->A, c->K, B, NULL, c->out_mode == 2 ? c->sa : NULL, c->sb, c->C,
                            c->N, c->M, c->N, c->K, NULL);
}

/* out_mode: 0 int32 out, 1 per-column dequant, 2 per-row x per-column dequant.
 * ms_total: `steps` back-to-back launches; us_each (may be NULL): then the
 * average of `steps` launches each timed on its own (time_each). */
int pcl_bench_igemm_ex(int M, int N, int K, int out_mode, int copies, int warmup, int steps,
                       double *ms_total, double *us_each) {
    int rc = PCL_OK;
    igemm_ctx c;
    memset(&c, 0, sizeof c);
    c.M = M, c.N = N, c.K = K, c.out_mode = out_mode;
    c.copies = copies < 1 ? 1 : (copies > 8 ? 8 : copies);
    c.A = dev_bytes((size_t)M * K, 11);
    c.Bq = dev_bytes((size_t)K * N, 12);
    c.sa = dev_f32(M, 13, 1e-3f, 1e-2f);
    c.sb = dev_f32(N, 14, 1e-3f, 1e-2f);
    c.C = pcl_malloc((size_t)M * N * 4);
    if (!c.A || !c.Bq || !c.sa || !c.sb || !c.C) {
        rc = PCL_ERR_OOM;
        goto done;
    }
    for (int j = 0; j < c.copies; j++) {
        c.Bpk[j] = pcl_malloc(pcl_s8_packed_bytes(K, N));
        if (!c.Bpk[j]) {
            rc = PCL_ERR_OOM;
            goto done;
        }
        TRY(pcl_pack_b_s8(c.Bq, N, K, N, c.Bpk[j], NULL, NULL));
    }
    TRY(time_steps(igemm_step, &c, warmup, steps, ms_total));
    if (us_each) TRY(time_each(igemm_step, &c, 0, steps, us_each));
done:
    pcl_free(c.A), pcl_free(c.Bq), pcl_free(c.sa), pcl_free(c.sb), pcl_free(c.C);
    for (int j = 0; j < 8; j++) pcl_free(c.Bpk[j]);
    return rc;
}

int pcl_bench_igemm(int M, int N, int K, int out_mode, int copies, int warmup, int steps,
                    double *ms_total) {
    return pcl_bench_igemm_ex(M, N, K, out_mode, copies, warmup, steps, ms_total, NULL);
}

/* ------------------------------------------------------------ FP32 GEMM ---- */
typedef struct {
    int opA, opB, M, N, K, accumulate;
    void *A, *B, *C;
} sgemm_ctx;

static int sgemm_step(void *c_, int i) {
    sgemm_ctx *c = c_;
    (void)i;
    int lda = c->opA == PCL_OP_N ? c->K : c->M, ldb = c->opB == PCL_OP_N ? c->N : c->K;
    return pcl_sgemm(c->opA, c->opB, c->M, c->N, c->K, c->A, lda, c->B, ldb, NULL, c->accumulate,
                     c->C, c->N, NULL);
}

int pcl_bench_sgemm(int opA, int opB, int M, int N, int K, int accumulate, int warmup, int steps,
                    double *ms_total) {
    int rc = PCL_OK;
    sgemm_ctx c = {opA, opB, M, N, K, accumulate, NULL, NULL, NULL};
    c.A = dev_f32((size_t)M * K, 21, -1.f, 1.f);
    c.B = dev_f32((size_t)K * N, 22, -1.f, 1.f);
    c.C = dev_f32((size_t)M * N, 23, -1e-3f, 1e-3f);
    if (!c.A || !c.B || !c.C) {
        rc = PCL_ERR_OOM;
        goto done;
    }
    TRY(time_steps(sgemm_step, &c, warmup, steps, ms_total));
done:
    pcl_free(c.A), pcl_free(c.B), pcl_free(c.C);
    return rc;
}

/* --------------------------------------------------- GEMM + epilogue ---- */
/* One step = the product with its elementwise epilogue, either fused
 * (pcl_sgemm_ex, one kernel) or as the reference sequences it: pcl_sgemm then
 * gelu_fwd / vec_add / gelu_bwd (two kernels, the product round-tripping HBM). */
typedef struct {
    int opA, opB, M, N, K, epi, fused;
    void *A, *B, *bias, *C, *aux, *tmp;
} sgemm_ex_ctx;

static int sgemm_ex_step(void *c_, int i) {
    sgemm_ex_ctx *c = c_;
    (void)i;
    const int lda = c->opA == PCL_OP_N ? c->K : c->M, ldb = c->opB == PCL_OP_N ? c->N : c->K;
    const long mn = (long)c->M * c->N;
    if (c->fused)
        return pcl_sgemm_ex(c->opA, c->opB, c->M, c->N, c->K, c->A, lda, c->B, ldb, c->bias, c->epi,
                            c->epi == PCL_EPI_GELU ? NULL : c->aux,
                            c->epi == PCL_EPI_GELU ? c->aux : NULL, c->N, c->C, c->N, NULL);
    void *prod = c->epi == PCL_EPI_GELU ? c->aux : c->tmp;
    int rc = pcl_sgemm(c->opA, c->opB, c->M, c->N, c->K, c->A, lda, c->B, ldb, c->bias, 0, prod, c->N,
                       NULL);
    if (rc != PCL_OK) return rc;
    if (c->epi == PCL_EPI_GELU) return pcl_gelu_fwd(c->C, prod, mn, NULL);
    if (c->epi == PCL_EPI_RESID) return pcl_vec_add(c->C, c->aux, prod, mn, NULL);
    return pcl_gelu_bwd(c->C, prod, c->aux, mn, NULL);
}

int pcl_bench_sgemm_ex(int opA, int opB, int M, int N, int K, int epi, int fused, int warmup,
                       int steps, double *ms_total) {
    int rc = PCL_OK;
    sgemm_ex_ctx c = {opA, opB, M, N, K, epi, fused, NULL, NULL, NULL, NULL, NULL, NULL};
    c.A = dev_f32((size_t)M * K, 21, -1.f, 1.f);
    c.B = dev_f32((size_t)K * N, 22, -0.05f, 0.05f);
    c.bias = dev_f32((size_t)N, 24, -0.1f, 0.1f);
    c.C = pcl_malloc((size_t)M * N * sizeof(float));
    c.aux = dev_f32((size_t)M * N, 25, -1.f, 1.f);
    c.tmp = pcl_malloc((size_t)M * N * sizeof(float));
    if (!c.A || !c.B || !c.bias || !c.C || !c.aux || !c.tmp) {
        rc = PCL_ERR_OOM;
        goto done;
    }
    TRY(time_steps(sgemm_ex_step, &c, warmup, steps, ms_total));
done:
    pcl_free(c.A), pcl_free(c.B), pcl_free(c.bias), pcl_free(c.C), pcl_free(c.aux), pcl_free(c.tmp);
    return rc;
}

/* ------------------------------------------------------------ attention ---- */
/* One step = one pcl_attn_fwd over B sequences of T tokens, H heads of dh
 * (Q, K, V ~ N-ish(0,1) as U[-1.7,1.7]); probs stored when with_probs. */
typedef struct {
    int B, T, H, dh, with_probs;
    void *Q, *K, *V, *O, *P;
} attn_ctx;

static int attn_step(void *c_, int i) {
    attn_ctx *c = c_;
    (void)i;
    const int D = c->H * c->dh;
    return pcl_attn_fwd(c->Q, c->K, c->V, D, c->O, D, c->with_probs ? c->P : NULL, c->B, c->T, c->H,
                        c->dh, NULL);
}

int pcl_bench_attn(int B, int T, int H, int dh, int with_probs, int warmup, int steps,
                   double *ms_total) {
    int rc = PCL_OK;
    attn_ctx c = {B, T, H, dh, with_probs, NULL, NULL, NULL, NULL, NULL};
    const size_t act = (size_t)B * T * H * dh;
    c.Q = dev_f32(act, 31, -1.7f, 1.7f);
    c.K = dev_f32(act, 32, -1.7f, 1.7f);
    c.V = dev_f32(act, 33, -1.7f, 1.7f);
    c.O = pcl_malloc(act * sizeof(float));
    if (with_probs) c.P = pcl_malloc((size_t)B * H * T * T * sizeof(float));
    if (!c.Q || !c.K || !c.V || !c.O || (with_probs && !c.P)) {
        rc = PCL_ERR_OOM;
        goto done;
    }
    TRY(time_steps(attn_step, &c, warmup, steps, ms_total));
done:
    pcl_free(c.Q), pcl_free(c.K), pcl_free(c.V), pcl_free(c.O), pcl_free(c.P);
    return rc;
}

/* One step = one pcl_attn_bwd (both kernels) from stored probabilities,
 * gradients set; dS goes to a caller scratch of B*H*T*T floats. */
typedef struct {
    int B, T, H, dh, with_att;
    void *dO, *Q, *K, *V, *P, *S, *dQ, *dK, *dV, *O;
} attn_bwd_ctx;

static int attn_bwd_step(void *c_, int i) {
    attn_bwd_ctx *c = c_;
    (void)i;
    const int D = c->H * c->dh;
    if (c->with_att)
        return pcl_attn_bwd_ex(c->dQ, c->dK, c->dV, D, c->S, c->dO, D, c->Q, c->K, c->V, D, c->P, c->O,
                               D, c->B, c->T, c->H, c->dh, 0, NULL);
    return pcl_attn_bwd(c->dQ, c->dK, c->dV, D, c->S, c->dO, D, c->Q, c->K, c->V, D, c->P, c->B,
                        c->T, c->H, c->dh, 0, NULL);
}

/* with_att: pcl_attn_bwd_ex, handed the forward's output */
int pcl_bench_attn_bwd_ex(int B, int T, int H, int dh, int with_att, int warmup, int steps,
                          double *ms_total) {
    int rc = PCL_OK;
    attn_bwd_ctx c = {B, T, H, dh, with_att, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL};
    const size_t act = (size_t)B * T * H * dh, pb = (size_t)B * H * T * T;
    c.dO = dev_f32(act, 34, -1.7f, 1.7f);
    c.Q = dev_f32(act, 31, -1.7f, 1.7f);
    c.K = dev_f32(act, 32, -1.7f, 1.7f);
    c.V = dev_f32(act, 33, -1.7f, 1.7f);
    c.P = pcl_malloc(pb * sizeof(float));
    c.S = pcl_malloc(pb * sizeof(float));
    c.dQ = pcl_malloc(act * sizeof(float));
    c.dK = pcl_malloc(act * sizeof(float));
    c.dV = pcl_malloc(act * sizeof(float));
    c.O = pcl_malloc(act * sizeof(float));
    if (!c.dO || !c.Q || !c.K || !c.V || !c.P || !c.S || !c.dQ || !c.dK || !c.dV || !c.O) {
        rc = PCL_ERR_OOM;
        goto done;
    }
    /* real probabilities and output of these inputs */
    TRY(pcl_attn_fwd(c.Q, c.K, c.V, H * dh, c.O, H * dh, c.P, B, T, H, dh, NULL));
    TRY(time_steps(attn_bwd_step, &c, warmup, steps, ms_total));
done:
    pcl_free(c.dO), pcl_free(c.Q), pcl_free(c.K), pcl_free(c.V), pcl_free(c.P), pcl_free(c.S);
    pcl_free(c.dQ), pcl_free(c.dK), pcl_free(c.dV), pcl_free(c.O);
    return rc;
}

int pcl_bench_attn_bwd(int B, int T, int H, int dh, int warmup, int steps, double *ms_total) {
    return pcl_bench_attn_bwd_ex(B, T, H, dh, 0, warmup, steps, ms_total);
}

/* ----------------------------------------------------------------- GEMV ---- */
/* A decode sweep: per step, one GEMV per weight in `shapes` (K_i x N_i), as
 * the layers of a model are visited, with `copies` rotating copies of the
 * whole weight set. kind 0: FP32 K x N weights (matvec); 1: FP32 N x K
 * (head-style); 2: INT8 packed weights with per-token x per-channel dequant. */
/* kinds[s]: 0 = FP32 W (K x N), 1 = FP32 W (N x K, the tied head),
 * 2 = INT8 packed weights with dequant */
typedef struct {
    int M, nshapes, copies;
    const int *kinds, *Ks, *Ns;
    void **W;  /* [copies * nshapes] */
    void *X, *Xu8, *Y, *sa, *sb;
} gemv_ctx;

static int gemv_step(void *c_, int i) {
    gemv_ctx *c = c_;
    int copy = i % c->copies;
    for (int s = 0; s < c->nshapes; s++) {
        int K = c->Ks[s], N = c->Ns[s], rc;
        void *W = c->W[copy * c->nshapes + s];
        if (c->kinds[s] == 0)
            rc = pcl_sgemv(PCL_OP_N, c->M, N, K, c->X, K, W, N, NULL, 0, c->Y, N, NULL);
        else if (c->kinds[s] == 1)
            rc = pcl_sgemv(PCL_OP_T, c->M, N, K, c->X, K, W, K, NULL, 0, c->Y, N, NULL);
        else
            rc = pcl_gemv_u8s8_dq(c->Xu8, K, W, NULL, c->sa, c->sb, c->Y, N, c->M, N, K, NULL);
        if (rc != PCL_OK) return rc;
    }
    return PCL_OK;
}

/* One token step of a decode sweep as a captured graph: a graph per weight
 * copy, replayed in rotation (one launch per step). */
typedef struct {
    void **graphs;
    int n;
} graph_ctx;

static int graph_step(void *c_, int i) {
    graph_ctx *c = c_;
    return pcl_graph_launch(c->graphs[i % c->n]);
}

/* use_graph: 0 = one call per product, 1 = the step captured once per weight
 * copy and replayed (needs a stream of its own, created here). */
int pcl_bench_gemv(const int *kinds, int M, int nshapes, const int *Ks, const int *Ns, int copies,
                   int warmup, int steps, int use_graph, double *ms_total, double *bytes_per_step) {
    int rc = PCL_OK;
    gemv_ctx c;
    memset(&c, 0, sizeof c);
    c.kinds = kinds, c.M = M, c.nshapes = nshapes, c.Ks = Ks, c.Ns = Ns;
    c.copies = copies < 1 ? 1 : copies;
    int kmax = 0, nmax = 0;
    double bytes = 0;
    for (int s = 0; s < nshapes; s++) {
        if (Ks[s] > kmax) kmax = Ks[s];
        if (Ns[s] > nmax) nmax = Ns[s];
        const int i8 = kinds[s] == 2;
        double wb = i8 ? (double)Ns[s] * pcl_s8_kpad(Ks[s]) : 4.0 * Ks[s] * Ns[s];
        double xb = i8 ? (double)M * Ks[s] : 4.0 * M * Ks[s];
        bytes += wb + xb + 4.0 * M * Ns[s] + (i8 ? 4.0 * (Ns[s] + M) : 0.0);
    }
    *bytes_per_step = bytes;
    c.W = calloc((size_t)c.copies * nshapes, sizeof(void *));
    c.X = dev_f32((size_t)M * kmax, 31, -1.f, 1.f);
    c.Xu8 = dev_bytes((size_t)M * kmax, 32);
    c.Y = pcl_malloc((size_t)M * nmax * 4);
    c.sa = dev_f32(M, 33, 1e-3f, 1e-2f);
    c.sb = dev_f32(nmax, 34, 1e-3f, 1e-2f);
    if (!c.W || !c.X || !c.Xu8 || !c.Y || !c.sa || !c.sb) {
        rc = PCL_ERR_OOM;
        goto done;
    }
    for (int cp = 0; cp < c.copies; cp++)
        for (int s = 0; s < nshapes; s++) {
            void **slot = &c.W[cp * nshapes + s];
            if (kinds[s] == 2) {
                void *Bq = dev_bytes((size_t)Ks[s] * Ns[s], 40 + s);
                *slot = pcl_malloc(pcl_s8_packed_bytes(Ks[s], Ns[s]));
                if (!Bq || !*slot) {
                    pcl_free(Bq);
                    rc = PCL_ERR_OOM;
                    goto done;
                }
                rc = pcl_pack_b_s8(Bq, Ns[s], Ks[s], Ns[s], *slot, NULL, NULL);
                pcl_stream_synchronize();
                pcl_free(Bq);
                if (rc != PCL_OK) goto done;
            } else {
                *slot = dev_f32((size_t)Ks[s] * Ns[s], 40 + s, -0.02f, 0.02f);
                if (!*slot) {
                    rc = PCL_ERR_OOM;
                    goto done;
                }
            }
        }
    if (!use_graph) {
        TRY(time_steps(gemv_step, &c, warmup, steps, ms_total));
    } else {
        void *prev = pcl_get_stream();
        void *st = pcl_stream_create();
        graph_ctx g = {calloc((size_t)c.copies, sizeof(void *)), c.copies};
        if (!st || !g.graphs) {
            rc = st ? PCL_ERR_OOM : pcl_last_status();
        } else {
            pcl_set_stream(st);
            gemv_step(&c, 0); /* eager pass: sizes the stream's scratch */
            rc = pcl_stream_synchronize();
            for (int cp = 0; rc == PCL_OK && cp < c.copies; cp++) {
                rc = pcl_graph_begin();
                if (rc == PCL_OK) {
                    int r1 = gemv_step(&c, cp);
                    int r2 = pcl_graph_end(&g.graphs[cp]);
                    rc = r1 != PCL_OK ? r1 : r2;
                }
            }
            if (rc == PCL_OK) rc = time_steps(graph_step, &g, warmup, steps, ms_total);
            for (int cp = 0; cp < c.copies; cp++)
                if (g.graphs[cp]) pcl_graph_destroy(g.graphs[cp]);
            pcl_set_stream(prev);
            pcl_stream_destroy(st);
        }
        free(g.graphs);
        if (rc != PCL_OK) goto done;
    }
done:
    if (c.W)
        for (int j = 0; j < c.copies * nshapes; j++) pcl_free(c.W[j]);
    free(c.W);
    pcl_free(c.X), pcl_free(c.Xu8), pcl_free(c.Y), pcl_free(c.sa), pcl_free(c.sb);
    return rc;
}

/* The same sweep as one grouped launch per step (pcl_gemv_group_*): every
 * product of the step is independent (own output rows), one group per weight
 * copy, rotated as above. kinds: 0 = FP32 W K x N, 1 = FP32 W N x K, 2 = INT8
 * packed (dequantised per row x per column). */
typedef struct {
    void **groups;
    int n;
} group_ctx;

static int group_step(void *c_, int i) {
    group_ctx *c = c_;
    return pcl_gemv_group_run(c->groups[i % c->n], NULL);
}

int pcl_bench_gemv_group(const int *kinds, int M, int nshapes, const int *Ks, const int *Ns,
                         int copies, int warmup, int steps, double *ms_total,
                         double *bytes_per_step) {
    int rc = PCL_OK;
    copies = copies < 1 ? 1 : copies;
    int kmax = 0, nmax = 0;
    long ytot = 0;
    double bytes = 0;
    for (int s = 0; s < nshapes; s++) {
        if (Ks[s] > kmax) kmax = Ks[s];
        if (Ns[s] > nmax) nmax = Ns[s];
        ytot += (long)M * Ns[s];
        const int i8 = kinds[s] == 2;
        double wb = i8 ? (double)Ns[s] * pcl_s8_kpad(Ks[s]) : 4.0 * Ks[s] * Ns[s];
        double xb = i8 ? (double)M * Ks[s] : 4.0 * M * Ks[s];
        bytes += wb + xb + 4.0 * M * Ns[s] + (i8 ? 4.0 * (Ns[s] + M) : 0.0);
    }
    *bytes_per_step = bytes;
    void **W = calloc((size_t)copies * nshapes, sizeof(void *));
    pcl_gemv_desc *d = calloc((size_t)nshapes, sizeof(pcl_gemv_desc));
    group_ctx g = {calloc((size_t)copies, sizeof(void *)), copies};
    void *X = dev_f32((size_t)M * kmax, 31, -1.f, 1.f);
    void *Xu8 = dev_bytes((size_t)M * kmax, 32);
    float *Y = pcl_malloc((size_t)ytot * 4);
    void *sa = dev_f32(M, 33, 1e-3f, 1e-2f);
    void *sb = dev_f32(nmax, 34, 1e-3f, 1e-2f);
    if (!W || !d || !g.groups || !X || !Xu8 || !Y || !sa || !sb) {
        rc = PCL_ERR_OOM;
        goto done;
    }
    for (int cp = 0; cp < copies; cp++) {
        long yoff = 0;
        for (int s = 0; s < nshapes; s++) {
            void **slot = &W[cp * nshapes + s];
            const int i8 = kinds[s] == 2;
            if (i8) {
                void *Bq = dev_bytes((size_t)Ks[s] * Ns[s], 40 + s);
                *slot = pcl_malloc(pcl_s8_packed_bytes(Ks[s], Ns[s]));
                if (!Bq || !*slot) {
                    pcl_free(Bq);
                    rc = PCL_ERR_OOM;
                    goto done;
                }
                rc = pcl_pack_b_s8(Bq, Ns[s], Ks[s], Ns[s], *slot, NULL, NULL);
                pcl_stream_synchronize();
                pcl_free(Bq);
                if (rc != PCL_OK) goto done;
            } else {
                *slot = dev_f32((size_t)Ks[s] * Ns[s], 40 + s, -0.02f, 0.02f);
                if (!*slot) {
                    rc = PCL_ERR_OOM;
                    goto done;
                }
            }
            pcl_gemv_desc *q = &d[s];
            memset(q, 0, sizeof *q);
            q->kind = i8 ? PCL_GEMV_U8S8 : (kinds[s] == 1 ? PCL_GEMV_F32_T : PCL_GEMV_F32_N);
            q->M = M, q->N = Ns[s], q->K = Ks[s];
            q->X = i8 ? Xu8 : X;
            q->ldx = Ks[s];
            q->W = *slot;
            q->ldw = i8 ? pcl_s8_kpad(Ks[s]) : (kinds[s] == 1 ? Ks[s] : Ns[s]);
            if (i8) q->sa = sa, q->sb = sb;
            q->Y = Y + yoff;
            q->ldy = Ns[s];
            yoff += (long)M * Ns[s];
        }
        TRY(pcl_gemv_group_create(d, nshapes, (pcl_gemv_group **)&g.groups[cp]));
    }
    TRY(time_steps(group_step, &g, warmup, steps, ms_total));
done:
    if (g.groups)
        for (int cp = 0; cp < copies; cp++) pcl_gemv_group_free(g.groups[cp]);
    free(g.groups);
    if (W)
        for (int j = 0; j < copies * nshapes; j++) pcl_free(W[j]);
    free(W);
    free(d);
    pcl_free(X), pcl_free(Xu8), pcl_free(Y), pcl_free(sa), pcl_free(sb);
    return rc;
}

/* Tied head + cross-entropy (350M: M=4096 tokens, D=1024, V=50257).
 * mode 0: one pcl_head_ce (logits, CE in place, d_lnf set, dwte accumulated)
 *         over chunks of at most chunk_bytes of logits;
 * mode 1: pcl_cross_entropy alone, M x V logits -> a separate dlogits. */
typedef struct {
    int M, D, V, mode;
    long chunk;
    void *x, *w, *t, *loss, *dx, *dw, *lg, *dl;
} head_ctx;

static int head_step(void *c_, int i) {
    head_ctx *c = c_;
    (void)i;
    if (c->mode == 0)
        return pcl_head_ce(c->x, c->w, c->t, c->M, c->D, c->V, c->loss, c->dx, c->dw, c->chunk, NULL);
    return pcl_cross_entropy(c->lg, c->V, c->t, c->dl, c->V, c->M, c->V, c->loss, NULL);
}

int pcl_bench_head_ce(int M, int D, int V, long chunk_bytes, int mode, int warmup, int steps,
                      double *ms_total) {
    int rc = PCL_OK;
    head_ctx c = {M, D, V, mode, chunk_bytes, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL};
    int *ht = malloc(sizeof(int) * (size_t)M);
    c.t = pcl_malloc(sizeof(int) * (size_t)M);
    c.loss = dev_f32(1, 40, 0.f, 0.f);
    if (!ht || !c.t || !c.loss) {
        rc = PCL_ERR_OOM;
        goto done;
    }
    for (int m = 0; m < M; m++) ht[m] = (int)((long)m * 7919 % V);
    TRY(pcl_memcpy_h2d(c.t, ht, sizeof(int) * (size_t)M));
    if (mode == 0) {
        c.x = dev_f32((size_t)M * D, 41, -1.f, 1.f);
        c.w = dev_f32((size_t)V * D, 42, -0.05f, 0.05f);
        c.dx = pcl_malloc(sizeof(float) * (size_t)M * D);
        c.dw = dev_f32((size_t)V * D, 43, 0.f, 0.f);
        if (!c.x || !c.w || !c.dx || !c.dw) {
            rc = PCL_ERR_OOM;
            goto done;
        }
    } else {
        c.lg = dev_f32((size_t)M * V, 44, -4.f, 4.f);
        c.dl = pcl_malloc(sizeof(float) * (size_t)M * V);
        if (!c.lg || !c.dl) {
            rc = PCL_ERR_OOM;
            goto done;
        }
    }
    TRY(time_steps(head_step, &c, warmup, steps, ms_total));
done:
    free(ht);
    pcl_free(c.t), pcl_free(c.loss), pcl_free(c.x), pcl_free(c.w), pcl_free(c.dx), pcl_free(c.dw);
    pcl_free(c.lg), pcl_free(c.dl);
    return rc;
}
