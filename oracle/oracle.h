/* ORACLE — test infrastructure only.
 *
 * A plain-C CPU restatement of nemoasr-c's per-chunk streaming hot path, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.  The product never
 * links, loads or calls anything here.
 *
 * Every function cites the reference lines it restates.  Activations are f32, weights are
 * bf16 bit patterns widened by <<16 (reference src/safetensors.h:32-36), dot products are
 * accumulated in f32 in increasing k order, and every output is computed by one thread, so the
 * results do not depend on the OpenMP thread count.
 *
 * Parity pinning: each function is checked in tests/test_oracle_*.py against an independent
 * formulation (numpy float64, torch CPU conv2d / LSTMCell, brute force on tiny inputs,
 * closed forms and invariants).  The mel front end lives in oracle/mel_ref.py.
 */
#ifndef NEMO_ORACLE_H
#define NEMO_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kernel-level restatements (reference src/kernels.metal) ------------------------------ */
enum { OR_ACT_NONE = 0, OR_ACT_SILU = 1, OR_ACT_RELU = 2, OR_ACT_GLU = 3 };

/* numerics study switch: GEMM A operand as f32 (0, the reference), bf16 (1), bf16 hi + lo (2) */
void or_set_gemm_a_mode(int mode);
void or_gemm(const float *A, long lda, const uint16_t *W, long ldw, const float *bias,
             float *C, long ldc, int M, int N, int K, int act, int accumulate, float alpha);
void or_layernorm(const float *X, const float *g, const float *b, float *Y, int M, int D, float eps);
void or_layernorm2(const float *X, const float *g1, const float *b1, const float *g2, const float *b2,
                   float *Y1, float *Y2, int M, int D, float eps);
void or_attention_rel(const float *Q, long ldq, const float *K, const float *V, long ldk, const float *P,
                      const float *bu, const float *bv, float *O, int c, int L, int Lmax, int H, int dh, int D,
                      float scale);
void or_dwconv_ln_silu(const float *din, const float *W, const float *g, const float *b, float *Y,
                       int c, int D, int taps, float eps);
void or_conv2d_c1_s2_relu(const float *X, const float *W, const float *bias, float *Y, int T, int F, int T1, int F1, int C);
void or_dwconv2d_s2(const float *X, const float *W, const float *bias, float *Y, int T, int F, int T1, int F1, int C);
void or_flatten_cf(const float *X, float *Y, int T, int F, int C);
void or_lstm_cell(const float *gates, const float *c_in, float *c_out, float *h_out, int H);
/* joint_partial + argmax_reduce: argmax_n W[n].relu(enc+pred) + b[n], lowest n on ties.
   logits (optional, V floats) receives every score. */
int or_joint_argmax(const float *enc, const float *pred, const uint16_t *W, const float *bias, int V, int H,
                    float *best_value, float *logits);
/* relative-position table of one layer: [2*Lmax-1][D] = pe . wpos^T */
void or_ptab(const uint16_t *wpos, int D, int Lmax, float *out);
float or_sigmoid(float v);
float or_silu(float v);

/* ---- model ---------------------------------------------------------------------------------- */
typedef struct {
    int n_layers, d_model, n_heads, head_dim, d_ff, subsampling, sub_channels, conv_kernel, feat_in;
    int num_prompts, prompt_hidden, pred_hidden, vocab_size, blank_id, joint_hidden, num_classes, max_symbols;
    int att_left, max_right;
    float ln_eps;
} or_dims_t;

/* All bf16 tensors as raw bit patterns (uint16), in checkpoint layout. */
typedef struct {
    const uint16_t *conv0_w, *conv0_b, *conv2_w, *conv2_b, *conv3_w, *conv3_b, *conv5_w, *conv5_b, *conv6_w, *conv6_b;
    const uint16_t *pre_out_w, *pre_out_b;
    const uint16_t *prompt_w0, *prompt_b0, *prompt_w2, *prompt_b2;
    const uint16_t *lstm_wx[2], *lstm_wh[2], *lstm_b[2];
    const uint16_t *embed;
    const uint16_t *joint_enc_w, *joint_enc_b, *joint_pred_w, *joint_pred_b, *joint_out_w, *joint_out_b;
} or_global_w_t;

typedef struct {
    const uint16_t *ff1_w1, *ff1_w2, *ff2_w1, *ff2_w2, *wq, *wk, *wv, *wo, *wpos, *pw1, *pw2;
    const uint16_t *ln_ff1_g, *ln_ff1_b, *ln_att_g, *ln_att_b, *ln_conv_g, *ln_conv_b, *ln_ff2_g, *ln_ff2_b;
    const uint16_t *ln_out_g, *ln_out_b, *bn_g, *bn_b, *dw_w, *bias_u, *bias_v;
} or_layer_w_t;

typedef struct or_model or_model_t;
or_model_t *or_model_create(const or_dims_t *dims, const or_global_w_t *g, const or_layer_w_t *layers);
void or_model_free(or_model_t *m);
int or_model_set_language(or_model_t *m, int prompt_index);
const float *or_model_ptab(const or_model_t *m, int layer);
int or_model_lmax(const or_model_t *m);

/* ---- streaming encoder + greedy RNNT decoder (reference src/encoder.c, src/decoder.c) ------- */
typedef struct or_session or_session_t;
or_session_t *or_session_create(or_model_t *m, int right_context);
void or_session_free(or_session_t *s);
void or_session_reset(or_session_t *s);
/* 1: keep per-chunk dumps (per-layer block outputs, prompted rows, joint_enc rows) */
void or_session_set_dump(or_session_t *s, int on);
/* Queue mel frames and run every chunk that is ready (all of them when final). Appends token ids;
   returns the number appended, or -1 on error. */
int or_session_feed_mel(or_session_t *s, const float *mel, size_t nframes, int final, int *tokens, int max_tokens);
size_t or_session_chunks(const or_session_t *s);
size_t or_session_frames(const or_session_t *s);
size_t or_session_joint_steps(const or_session_t *s);
/* dumps: frames x n_layers x D (layer-major per chunk), frames x D, frames x joint_hidden */
const float *or_session_dump_layers(const or_session_t *s);
const float *or_session_dump_prompted(const or_session_t *s);
const float *or_session_dump_joint_enc(const or_session_t *s);
/* per chunk row count c (frames emitted by each chunk that produced rows) */
const int *or_session_dump_chunk_rows(const or_session_t *s);
/* joint evaluation log: for every joint evaluation, best index and top-2 margin */
size_t or_session_joint_log(const or_session_t *s, const int **best, const float **margin);
/* per emitted token, the smallest top-2 joint margin of the decisions that produced it; *tail is the
 * smallest margin of the decisions after the last token (INFINITY when there are none) */
size_t or_session_token_margins(const or_session_t *s, const float **margin, float *tail);
/* committed greedy decisions of the decodes since reset: outcome, runner-up index, top-2 margin */
size_t or_session_decisions(const or_session_t *s, const int **best, const int **second, const float **margin);
/* force committed decision at[i] to token tok[i] in the following decodes (test hook) */
void or_session_force(or_session_t *s, const size_t *at, const int *tok, size_t n);
/* For tests of compaction-independence: the epoch length in chunks (reference CACHE_EPOCH_CHUNKS). */
const char *or_session_error(const or_session_t *s);

/* Encoder-step bookkeeping alone (reference src/encoder.c:213-251): given the state, decide the
   next step. Exposed so host bookkeeping can be compared step by step. */
typedef struct {
    size_t pending_n, consumed, emitted;
    int mel_cache_n, closed;
} or_enc_book_t;
typedef struct {
    int ran;              /* 0: nothing to do; 1: a piece was consumed */
    int take, nwin, lo, hi, c, include_boundary, T3;
} or_enc_plan_t;
or_enc_plan_t or_enc_plan(or_enc_book_t *b, int final, int chunk_mel, int subsampling, int mel_cache);

void or_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
