/*
 * ref_shim_model.c -- build-time harness around the reference's own
 * transformer.c (pure-c-llm), compiled where it lies. TEST INFRASTRUCTURE
 * ONLY: exports the static decode GEMV proj_token (transformer.c:174-195).
 * model.c's lm_head and tensor.c's matmul are linked into the same library
 * from their own translation units (see Makefile).
 */
#include REF_TRANSFORMER_C

int pcl_ref_model_d_model(void) { return D_MODEL; }
void pcl_ref_proj_token(float *out, const float *in, const float *W, const float *bias, int K, int N) {
    proj_token(out, in, W, bias, K, N);
}
