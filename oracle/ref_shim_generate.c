/*
 * ref_shim_generate.c -- build-time harness around the reference's generate.c
 * (pure-c-llm), compiled where it lies with tokenizer.c (-DTOKENIZER_LIB, as
 * generate.c:8-10 builds it). TEST INFRASTRUCTURE ONLY: exports the
 * checkpoint reader and the KV-cached forward (generate.c:49-76, 118-183).
 */
#include REF_GENERATE_C

int pcl_ref_gen_load(const char *path) {
    load_model(path);
    alloc_state();
    return V;
}
void pcl_ref_gen_forward(int tok, int pos, float *logits) {
    forward(tok, pos);
    memcpy(logits, s_logits, sizeof(float) * (size_t)V);
}
