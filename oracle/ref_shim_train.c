/*
 * ref_shim_train.c -- build-time harness around the reference's own train.c
 * (pure-c-llm), compiled where it lies with small -D dims from the Makefile.
 * TEST INFRASTRUCTURE ONLY: exports its static GEMM and attention functions
 * (train.c:181-252, 339-407, 412-465) under pcl_ref_* names to pin the oracle.
 */
#include REF_TRAIN_C

int pcl_ref_train_d_model(void) { return D_MODEL; }
int pcl_ref_train_vocab(void) { return VOCAB_SIZE; }
void pcl_ref_matmul_forward(float *out, const float *in, const float *Wt, const float *bias, int M, int K, int N) {
    matmul_forward(out, in, Wt, bias, M, K, N);
}
void pcl_ref_matmul_backward(const float *dY, const float *X, const float *Wt, float *dX, float *dW, float *db,
                             int M, int K, int N) {
    matmul_backward(dY, X, Wt, dX, dW, db, M, K, N);
}
void pcl_ref_tied_head_forward(float *logits, const float *lnf, const float *wte, int M) {
    tied_head_forward(logits, lnf, wte, M);
}
void pcl_ref_tied_head_backward(float *d_lnf, float *dwte, const float *d_logits, const float *lnf,
                                const float *wte, int M) {
    tied_head_backward(d_lnf, dwte, d_logits, lnf, wte, M);
}
int pcl_ref_train_n_heads(void) { return N_HEADS; }
int pcl_ref_train_t_size(void) { return T_SIZE; }
void pcl_ref_attention_forward(const float *q, const float *k, const float *v, float *att, float *probs,
                               int B, int T) {
    attention_forward(q, k, v, att, probs, B, T);
}
void pcl_ref_attention_backward(float *dq, float *dk, float *dv, const float *d_att, const float *q,
                                const float *k, const float *v, const float *probs, int B, int T) {
    attention_backward(dq, dk, dv, d_att, q, k, v, probs, B, T);
}
void pcl_ref_gelu_forward(float *out, const float *in, int n) { gelu_forward(out, in, n); }
void pcl_ref_gelu_backward(float *din, const float *dout, const float *in, int n) {
    gelu_backward(din, dout, in, n);
}
float pcl_ref_cross_entropy(const float *logits, const int *targets, float *d_logits, int M) {
    return cross_entropy(logits, targets, d_logits, M);
}
