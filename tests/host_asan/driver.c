/* driver.c -- exercises the host bookkeeping of libpcl_hip (per-stream scratch
 * grow and retire, graph pinning, scratch release, the thread-local staging
 * slots of the host-pointer drop-ins, the realigned FP32 operands, the bench
 * harness's decode sweep) on a CPU, against the mock HIP runtime, under
 * AddressSanitizer / UndefinedBehaviorSanitizer. Test infrastructure only. */
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pcl_hip.h"

int pcl_bench_gemv(const int *kinds, int M, int nshapes, const int *Ks, const int *Ns, int copies, int warmup,
                   int steps, int use_graph, double *ms_total, double *bytes_per_step);
int pcl_bench_gemv_group(const int *kinds, int M, int nshapes, const int *Ks, const int *Ns, int copies,
                         int warmup, int steps, double *ms_total, double *bytes_per_step);

static void chk(int st, const char *what) {
    if (st != PCL_OK) {
        fprintf(stderr, "FAIL %s: status %d: %s\n", what, st, pcl_last_error());
        exit(1);
    }
}

static float *dalloc(size_t n) {
    float *p = pcl_malloc(n * sizeof(float));
    if (!p) { fprintf(stderr, "FAIL alloc\n"); exit(1); }
    memset(p, 0, n * sizeof(float));
    return p;
}

/* split-K GEMVs of growing K and rows on the thread's stream: the workspace
 * grows (and, on a stream a graph was captured on, is retired, not freed) */
static void gemv_sweep(int rounds) {
    for (int r = 0; r < rounds; r++) {
        const int M = 1 + r % 8, N = 512 + 64 * r, K = 2048 + 1024 * r;
        float *X = dalloc((size_t)M * K), *W = dalloc((size_t)K * N), *Y = dalloc((size_t)M * N);
        chk(pcl_sgemv(PCL_OP_N, M, N, K, X, K, W, N, NULL, 0, Y, N, NULL), "sgemv");
        chk(pcl_sgemv(PCL_OP_T, M, N, K, X, K, W, K, NULL, 0, Y, N, NULL), "sgemv T");
        chk(pcl_stream_synchronize(), "sync");
        pcl_free(X), pcl_free(W), pcl_free(Y);
    }
}

static void *thread_main(void *arg) {
    const int id = (int)(long)arg;
    void *st = id % 2 ? pcl_stream_create() : NULL;  /* half on the shared null stream */
    if (id % 2 && !st) { fprintf(stderr, "FAIL stream\n"); exit(1); }
    chk(pcl_set_stream(st), "set stream");
    for (int rep = 0; rep < 3; rep++) {
        gemv_sweep(4);
        /* host drop-ins: the thread's staging slots grow */
        const int M = 16 + 32 * rep, K = 64 + 16 * rep, N = 48 + 8 * rep;
        float *A = calloc((size_t)M * K, 4), *B = calloc((size_t)K * N, 4), *C = calloc((size_t)M * N, 4);
        matmul(A, B, C, M, K, N);
        chk(pcl_last_status(), "matmul");
        free(A), free(B), free(C);
    }
    if (st) {
        chk(pcl_release_scratch(st), "release");
        gemv_sweep(2);
        chk(pcl_set_stream(NULL), "reset stream");
        chk(pcl_stream_destroy(st), "destroy");
    }
    return NULL;
}

int main(void) {
    chk(pcl_init(), "init");
    /* 1. graphs: capture on a created stream with the workspace growing inside
     * the capture, grow it again eagerly (the old buffer is retired), release
     * refused while pinned, destroy frees everything */
    void *st = pcl_stream_create();
    chk(pcl_set_stream(st), "set stream");
    gemv_sweep(2);
    chk(pcl_graph_begin(), "graph begin");
    {
        const int M = 8, N = 2048, K = 16384;
        float *X = dalloc((size_t)M * K), *W = dalloc((size_t)K * N), *Y = dalloc((size_t)M * N);
        chk(pcl_sgemv(PCL_OP_N, M, N, K, X, K, W, N, NULL, 0, Y, N, NULL), "sgemv in capture");
        /* a host drop-in inside the capture is refused and changes nothing */
        float h[4] = {0};
        matmul(h, h, h, 1, 1, 1);
        if (pcl_last_status() != PCL_ERR_INVALID_ARG) { fprintf(stderr, "FAIL no refusal\n"); return 1; }
        void *g = NULL;
        chk(pcl_graph_end(&g), "graph end");
        gemv_sweep(6);  /* larger: retires the captured workspace */
        chk(pcl_graph_launch(g), "graph launch");
        if (pcl_release_scratch(st) != PCL_ERR_INVALID_ARG) { fprintf(stderr, "FAIL release on pinned\n"); return 1; }
        chk(pcl_graph_destroy(g), "graph destroy");
        pcl_free(X), pcl_free(W), pcl_free(Y);
    }
    chk(pcl_set_stream(NULL), "reset stream");
    chk(pcl_stream_destroy(st), "destroy");
    /* 2. misaligned FP32 operands of >= 2^30 multiply-adds: realigned copies in
     * the stream's realign buffer, twice the size the second time; the head +
     * cross-entropy on such operands keeps its logits chunk in its own scratch */
    for (int r = 0; r < 2; r++) {
        const int M = 256 * (r + 1), N = 4096, K = 1022;
        float *A = dalloc((size_t)M * K), *B = dalloc((size_t)N * K), *C = dalloc((size_t)M * N);
        chk(pcl_sgemm(PCL_OP_N, PCL_OP_T, M, N, K, A, K, B, K, NULL, 0, C, N, NULL), "sgemm realigned");
        chk(pcl_sgemm(PCL_OP_T, PCL_OP_N, K, N, M, A, K, C, N, NULL, 1, B, N, NULL), "sgemm TN realigned");
        pcl_free(A), pcl_free(B), pcl_free(C);
    }
    {
        const int M = 512, D = 1022, V = 8192;
        float *x = dalloc((size_t)M * D), *w = dalloc((size_t)V * D), *dx = dalloc((size_t)M * D),
              *dw = dalloc((size_t)V * D), *loss = dalloc(1);
        int *t = (int *)dalloc(M);
        chk(pcl_head_ce(x, w, t, M, D, V, loss, dx, dw, (long)256 * V * 4, NULL), "head_ce chunked");
        chk(pcl_head_ce(x, w, t, M, D, V, loss, dx, dw, 0, NULL), "head_ce whole");
        pcl_free(x), pcl_free(w), pcl_free(dx), pcl_free(dw), pcl_free(loss), pcl_free(t);
    }
    chk(pcl_release_scratch(NULL), "release null stream");
    /* 3. threads: streams of their own and the shared null stream at once */
    pthread_t th[6];
    for (long i = 0; i < 6; i++) pthread_create(&th[i], NULL, thread_main, (void *)i);
    for (int i = 0; i < 6; i++) pthread_join(th[i], NULL);
    /* 4. the bench harness's decode sweep that ended with a heap-corruption
     * report under the profiler (bench.py decode_fp32_m1: 64 FP32 K x N
     * products of the grown model and the N x K head, M = 1, 3 weight copies),
     * eager and as graphs, then the grouped form */
    {
        int kinds[65], Ks[65], Ns[65];
        const int L[4][2] = {{512, 1536}, {512, 512}, {512, 2048}, {2048, 512}};
        for (int i = 0; i < 64; i++) kinds[i] = 0, Ks[i] = L[i % 4][0], Ns[i] = L[i % 4][1];
        kinds[64] = 1, Ks[64] = 512, Ns[64] = 2048;
        double ms = 0, by = 0;
        chk(pcl_bench_gemv(kinds, 1, 65, Ks, Ns, 3, 2, 10, 0, &ms, &by), "bench gemv eager");
        chk(pcl_bench_gemv(kinds, 1, 65, Ks, Ns, 3, 2, 10, 1, &ms, &by), "bench gemv graph");
        for (int i = 0; i < 65; i++) kinds[i] = 2;
        chk(pcl_bench_gemv(kinds, 8, 65, Ks, Ns, 2, 2, 5, 0, &ms, &by), "bench gemv int8");
        chk(pcl_bench_gemv_group(kinds, 8, 65, Ks, Ns, 2, 2, 5, &ms, &by), "bench gemv group");
    }
    /* everything the library keeps per stream is freed: nothing may leak */
    chk(pcl_release_scratch(NULL), "final release");
    printf("host bookkeeping ok\n");
    return 0;
}
