/*
 * decode_gpu.c -- the projection GEMVs of KV-cached decode, in the order
 * generate.c issues them (generate.c:120-183): per layer Q, K, V, O
 * (D x D), FF1 (D x FF), FF2 (FF x D) through matvec with bias, then the
 * tied-head dot loop over wte (V x D). Here they run through the native
 * device-pointer GEMV (pcl_sgemv) for M token rows at once (M=1 is the
 * reference's single-token decode). LayerNorm, attention and GELU are outside
 * the matrix-multiply path and are not run; the activations are synthetic.
 *
 * Reports the achieved weight-streaming bandwidth of the sweep. The weights
 * of the grown model (205 MB FP32) fit the 256 MB Infinity Cache, so
 * `copies` model replicas are rotated to make every sweep read HBM.
 *
 * Usage: decode_gpu [d_model d_ff vocab layers M copies sweeps]
 *        default: the grown model 512 2048 2048 16, M=1, 3 copies, 20 sweeps
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "pcl_hip.h"

#define CHECK(x)                                                                \
    do {                                                                        \
        int s_ = (x);                                                           \
        if (s_ != PCL_OK) {                                                     \
            fprintf(stderr, "%s failed (%d): %s\n", #x, s_, pcl_last_error());  \
            exit(1);                                                            \
        }                                                                       \
    } while (0)

static uint32_t g_rng = 1234u; /* model.c:117 */
static float frand(float scale) {  /* model.c:118-125 */
    g_rng ^= g_rng << 13;
    g_rng ^= g_rng >> 17;
    g_rng ^= g_rng << 5;
    float u = (float)(g_rng & 0x00FFFFFFu) / (float)0x01000000;
    return (u * 2.0f - 1.0f) * scale;
}

static float *dev_rand(size_t n, float scale) {
    float *h = malloc(n * sizeof(float));
    for (size_t i = 0; i < n; i++) h[i] = frand(scale);
    float *d = pcl_malloc(n * sizeof(float));
    if (!d) {
        fprintf(stderr, "device allocation failed: %s\n", pcl_last_error());
        exit(1);
    }
    CHECK(pcl_memcpy_h2d(d, h, n * sizeof(float)));
    free(h);
    return d;
}

typedef struct {
    float *Wq, *Wk, *Wv, *Wo, *W1, *W2, *bq, *bk, *bv, *bo, *b1, *b2;
} Layer;

int main(int argc, char **argv) {
    int D = 512, FF = 2048, V = 2048, L = 16, M = 1, copies = 3, sweeps = 20;
    if (argc == 8) {
        D = atoi(argv[1]), FF = atoi(argv[2]), V = atoi(argv[3]), L = atoi(argv[4]);
        M = atoi(argv[5]), copies = atoi(argv[6]), sweeps = atoi(argv[7]);
    }
    pcl_set_abort_on_error(1);
    CHECK(pcl_init());
    Layer *lay = malloc(sizeof(Layer) * (size_t)L * copies);
    float **wte = malloc(sizeof(float *) * copies);
    for (int c = 0; c < copies; c++) {
        for (int l = 0; l < L; l++) {
            Layer *w = &lay[c * L + l];
            w->Wq = dev_rand((size_t)D * D, 0.02f), w->Wk = dev_rand((size_t)D * D, 0.02f);
            w->Wv = dev_rand((size_t)D * D, 0.02f), w->Wo = dev_rand((size_t)D * D, 0.02f);
            w->W1 = dev_rand((size_t)D * FF, 0.02f), w->W2 = dev_rand((size_t)FF * D, 0.02f);
            w->bq = dev_rand(D, 0.f), w->bk = dev_rand(D, 0.f), w->bv = dev_rand(D, 0.f);
            w->bo = dev_rand(D, 0.f), w->b1 = dev_rand(FF, 0.f), w->b2 = dev_rand(D, 0.f);
        }
        wte[c] = dev_rand((size_t)V * D, 0.02f);
    }
    float *x = dev_rand((size_t)M * FF, 1.0f), *y = dev_rand((size_t)M * FF, 0.f);
    float *logits = dev_rand((size_t)M * V, 0.f);
    double bytes = 0;
    for (int l = 0; l < L; l++)
        bytes += 4.0 * ((4.0 * D * D + 2.0 * D * FF) + M * (10.0 * D + 2.0 * FF) + 5.0 * D + FF);
    bytes += 4.0 * ((double)V * D + (double)M * (D + V));

    void *e0 = pcl_event_create(), *e1 = pcl_event_create();
    /* warm-up sweep */
    for (int s = -1; s < sweeps; s++) {
        if (s == 0) CHECK(pcl_event_record(e0));
        int c = (s + 1) % copies;
        for (int l = 0; l < L; l++) {
            Layer *w = &lay[c * L + l];
            CHECK(pcl_sgemv(PCL_OP_N, M, D, D, x, D, w->Wq, D, w->bq, 0, y, D, NULL));  /* q */
            CHECK(pcl_sgemv(PCL_OP_N, M, D, D, x, D, w->Wk, D, w->bk, 0, y, D, NULL));  /* k row */
            CHECK(pcl_sgemv(PCL_OP_N, M, D, D, x, D, w->Wv, D, w->bv, 0, y, D, NULL));  /* v row */
            CHECK(pcl_sgemv(PCL_OP_N, M, D, D, y, D, w->Wo, D, w->bo, 0, x, D, NULL));  /* o */
            CHECK(pcl_sgemv(PCL_OP_N, M, FF, D, x, D, w->W1, FF, w->b1, 0, y, FF, NULL));
            CHECK(pcl_sgemv(PCL_OP_N, M, D, FF, y, FF, w->W2, D, w->b2, 0, x, D, NULL));
        }
        CHECK(pcl_sgemv(PCL_OP_T, M, V, D, x, D, wte[c], D, NULL, 0, logits, V, NULL));
    }
    CHECK(pcl_event_record(e1));
    float ms;
    CHECK(pcl_event_elapsed_ms(e0, e1, &ms));
    double per = ms / sweeps;
    printf("decode GEMV sweep: d_model=%d d_ff=%d vocab=%d layers=%d M=%d copies=%d\n", D, FF, V, L, M, copies);
    printf("  %.3f ms per token step, %.1f GB/s, %.0f token-steps/s\n", per, bytes / (per * 1e-3) / 1e9,
           1e3 / per);
    return 0;
}
