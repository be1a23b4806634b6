/*
 * generate_gpu.c -- generate.c's greedy decoding (generate.c:222-260 at
 * temperature 0) as a C host program over the C ABI: the CKP1 checkpoint is
 * loaded into device memory once (pcl_model_load_ex, fp32 or INT8 weights),
 * the prompt is fed at positions 0.., and n_new tokens are picked by argmax on
 * the GPU and fed back there, eagerly or as one graph replay per token.
 * The tokenizer (tokenizer.c) is not part of the matrix-multiply path: the
 * prompt is given as token ids and the output is printed as ids.
 *
 * Usage: generate_gpu <ckpt.ckp1> <n_new> <fp32|int8> <eager|graph> <tok> [tok ...]
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "pcl_hip.h"

static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec + 1e-9 * t.tv_nsec;
}

int main(int argc, char **argv) {
    if (argc < 6) {
        fprintf(stderr, "usage: %s <ckpt.ckp1> <n_new> <fp32|int8> <eager|graph> <tok> [tok ...]\n",
                argv[0]);
        return 2;
    }
    const char *path = argv[1];
    const int n_new = atoi(argv[2]);
    const int weights = strcmp(argv[3], "int8") == 0 ? PCL_W_INT8 : PCL_W_FP32;
    const int graph = strcmp(argv[4], "graph") == 0;
    const int n_prompt = argc - 5;
    int *prompt = malloc(sizeof(int) * (size_t)n_prompt);
    int *out = malloc(sizeof(int) * (size_t)(n_new > 0 ? n_new : 1));
    if (!prompt || !out) return 1;
    for (int i = 0; i < n_prompt; i++) prompt[i] = atoi(argv[5 + i]);

    pcl_model *m = pcl_model_load_ex(path, weights);
    if (!m) {
        fprintf(stderr, "pcl_model_load_ex: %s\n", pcl_last_error());
        return 1;
    }
    int hdr[8];
    pcl_model_header(m, hdr);
    printf("model: block %d, d_model %d, heads %d, d_ff %d, layers %d, vocab %d (%s weights)\n",
           hdr[1], hdr[2], hdr[3], hdr[4], hdr[5], hdr[6], weights == PCL_W_INT8 ? "int8" : "fp32");

    /* the first call captures the step graph (graph mode) and warms up */
    int st = pcl_model_generate(m, prompt, n_prompt, n_new, out, graph);
    double t0 = now_s();
    if (st == PCL_OK) st = pcl_model_generate(m, prompt, n_prompt, n_new, out, graph);
    const double dt = now_s() - t0;
    if (st != PCL_OK) {
        fprintf(stderr, "pcl_model_generate: %s\n", pcl_last_error());
        pcl_model_free(m);
        return 1;
    }
    printf("tokens:");
    for (int i = 0; i < n_new; i++) printf(" %d", out[i]);
    printf("\n%d prompt + %d new tokens in %.3f ms: %.1f new tokens/s (%s)\n", n_prompt, n_new,
           1e3 * dt, n_new / dt, graph ? "one graph replay per token" : "eager");
    pcl_model_free(m);
    free(prompt);
    free(out);
    return 0;
}
