/*
 * train_step_gpu.c -- the GEMM sequence of one training step, issued through
 * the reference's device-pointer GPU API (gpu_kernels.h:38-51) as
 * train_kaggle.cu's forward (train_kaggle.cu:147-166) and backward
 * (train_kaggle.cu:168-214) issue it, with libpcl_hip behind that API.
 *
 * Per layer, forward: Q, K, V projections via gemm_nn with bias, causal
 * attention via attn_fwd (probabilities kept), the O projection and FF1, FF2
 * via gemm_nn; after the layers the tied head via gemm_nt and the softmax
 * cross-entropy via ce_fwd_bwd (dlogits in place). Backward: d_lnf via
 * gemm_nn and dwte via gemm_tn for the head, then per layer (in reverse)
 * dX = dY.W^T via gemm_nt (accumulating), dW += X^T.dY via gemm_tn plus
 * bias_bwd, and attn_bwd from the stored probabilities. LayerNorm, GELU,
 * embeddings and AdamW are not run: activations are synthetic.
 *
 * Usage: train_step_gpu [d_model d_ff vocab layers tokens steps heads seq]
 *        default: the 350M-class shapes, 1024 4096 50257 24 4096 3 16 1024
 */
#include <math.h>
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

static uint32_t g_rng = 12345u; /* train.c:72 */
static float frand(float scale) {  /* train.c:73-78 */
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

int main(int argc, char **argv) {
    int D = 1024, FF = 4096, V = 50257, L = 24, M = 4096, steps = 3, H = 16, T = 1024;
    if (argc >= 7) {
        D = atoi(argv[1]), FF = atoi(argv[2]), V = atoi(argv[3]), L = atoi(argv[4]);
        M = atoi(argv[5]), steps = atoi(argv[6]);
    }
    if (argc == 9) H = atoi(argv[7]), T = atoi(argv[8]);
    if (T <= 0 || M % T != 0 || H <= 0 || D % H != 0) {
        fprintf(stderr, "tokens must be a multiple of seq, d_model of heads\n");
        return 2;
    }
    const int B = M / T;
    pcl_set_abort_on_error(1);
    gpu_init();
    /* the compile-time dims of gpu_kernels.h (DIM, VOCAB_SIZE, B_SIZE, T_SIZE, N_HEADS) */
    CHECK(pcl_set_model_dims(D, V));
    CHECK(pcl_set_attn_dims(B, T, H));
    printf("train step: d_model=%d d_ff=%d vocab=%d layers=%d tokens=%d (%d x %d), heads=%d\n", D,
           FF, V, L, M, B, T, H);

    /* one set of layer weights reused by every layer keeps memory modest;
     * the GEMM shapes and the call sequence are those of the full model */
    float *Wq = dev_rand((size_t)D * D, 0.02f), *Wk = dev_rand((size_t)D * D, 0.02f);
    float *Wv = dev_rand((size_t)D * D, 0.02f), *Wo = dev_rand((size_t)D * D, 0.02f);
    float *W1 = dev_rand((size_t)D * FF, 0.02f), *W2 = dev_rand((size_t)FF * D, 0.02f);
    float *bD = dev_rand(D, 0.0f), *bF = dev_rand(FF, 0.0f);
    float *wte = dev_rand((size_t)V * D, 0.02f);
    float *x = dev_rand((size_t)M * D, 1.0f), *h = dev_rand((size_t)M * FF, 1.0f);
    float *q = dev_rand((size_t)M * D, 0.0f), *k = dev_rand((size_t)M * D, 0.0f);
    float *v = dev_rand((size_t)M * D, 0.0f), *o = dev_rand((size_t)M * D, 0.0f);
    float *logits = dev_rand((size_t)M * V, 0.0f);
    float *dY = dev_rand((size_t)M * FF, 1e-3f), *dX = dev_rand((size_t)M * FF, 0.0f);
    float *dWq = dev_rand((size_t)D * D, 0.0f), *dW1 = dev_rand((size_t)D * FF, 0.0f);
    float *dW2 = dev_rand((size_t)FF * D, 0.0f), *db = dev_rand(FF, 0.0f);
    float *dwte = dev_rand((size_t)V * D, 0.0f);
    float *att = dev_rand((size_t)M * D, 0.0f);
    float *probs = dev_rand((size_t)B * H * T * T, 0.0f), *scratch = dev_rand((size_t)B * H * T * T, 0.0f);
    float *dq = dev_rand((size_t)M * D, 0.0f), *dk = dev_rand((size_t)M * D, 0.0f);
    float *dv = dev_rand((size_t)M * D, 0.0f), *loss = dev_rand(1, 0.0f);
    int *targets = pcl_malloc(sizeof(int) * (size_t)M);
    {
        int *ht = malloc(sizeof(int) * (size_t)M);
        if (!targets || !ht) return 1;
        for (int i = 0; i < M; i++) ht[i] = (int)((long)i * 7919 % V);
        CHECK(pcl_memcpy_h2d(targets, ht, sizeof(int) * (size_t)M));
        free(ht);
    }
    const double attn_flop = 4.0 * B * H * (double)(D / H) * T * (T + 1) / 2; /* QK^T + PV, causal */

    void *e0 = pcl_event_create(), *e1 = pcl_event_create();
    double flop = 0;
    float best = 1e30f;
    for (int s = 0; s < steps; s++) {
        flop = 0;
        CHECK(pcl_event_record(e0));
        for (int l = 0; l < L; l++) {
            gemm_nn(x, Wq, bD, q, M, D, D);
            gemm_nn(x, Wk, bD, k, M, D, D);
            gemm_nn(x, Wv, bD, v, M, D, D);
            attn_fwd(q, k, v, att, probs);                   /* train_kaggle.cu:154 */
            gemm_nn(att, Wo, bD, o, M, D, D);
            gemm_nn(o, W1, bF, h, M, D, FF);
            gemm_nn(h, W2, bD, x, M, FF, D);
            flop += 2.0 * M * D * (4.0 * D + 2.0 * FF) + attn_flop;
        }
        gemm_nt(x, wte, logits, M, D, V, 0);                 /* tied head */
        ce_fwd_bwd(logits, targets, logits, loss);           /* train_kaggle.cu:409 */
        gemm_nn(logits, wte, NULL, dX, M, V, D);             /* d_lnf */
        gemm_tn(logits, x, dwte, M, V, D);                   /* dwte += */
        flop += 3 * 2.0 * M * D * V;
        for (int l = L - 1; l >= 0; l--) {
            gemm_nt(dY, W2, dX, M, D, FF, 0);                /* dX of FF2 */
            gemm_tn(h, dY, dW2, M, FF, D);                   /* dW2 += */
            bias_bwd(db, dY, M, D);
            gemm_nt(dY, W1, dX, M, FF, D, 0);                /* dX of FF1 */
            gemm_tn(o, dY, dW1, M, D, FF);                   /* dW1 += */
            bias_bwd(db, dY, M, FF);
            gemm_nt(dY, Wo, dX, M, D, D, 0);                 /* d_att of Wo */
            gemm_tn(att, dY, dWq, M, D, D);
            bias_bwd(db, dY, M, D);
            attn_bwd(dq, dk, dv, scratch, dX, q, k, v, probs); /* train_kaggle.cu:199 */
            for (int p = 0; p < 3; p++) {                    /* Wq, Wk, Wv */
                gemm_nt(p == 0 ? dq : (p == 1 ? dk : dv), Wq, dX, M, D, D, p > 0);
                gemm_tn(x, p == 0 ? dq : (p == 1 ? dk : dv), dWq, M, D, D);
                bias_bwd(db, p == 0 ? dq : (p == 1 ? dk : dv), M, D);
            }
            flop += 2 * 2.0 * M * D * (4.0 * D + 2.0 * FF) + 2 * attn_flop;
        }
        CHECK(pcl_event_record(e1));
        float ms;
        CHECK(pcl_event_elapsed_ms(e0, e1, &ms));
        if (ms < best) best = ms;
        printf("  step %d: %.1f ms, %.1f TFLOP/s over the step's GEMMs and attention\n", s, ms,
               flop / (ms * 1e-3) / 1e12);
    }
    float hl;
    CHECK(pcl_memcpy_d2h(&hl, loss, sizeof hl));
    printf("best step: %.1f ms (%.1f TFLOP/s, %.0f tokens/s); loss accumulated over %d steps %.4f\n",
           best, flop / (best * 1e-3) / 1e12, M / (best * 1e-3), steps, hl);
    return 0;
}
