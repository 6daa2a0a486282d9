/* ORACLE — test infrastructure only (see oracle.h).
 *
 * CPU restatement of the streaming bookkeeping of nemoasr-c:
 *   encoder: src/encoder.c (window/lo/hi rule :213-267, pre-encode :120-142, blocks :144-197,
 *            compaction :199-211);
 *   decoder: src/decoder.c (prediction net :57-77, joint batch :79-90, greedy loop :92-127);
 *   model:   src/model.c (prompt fold :312-322, ptab :286-306).
 *
 * The attention and convolution histories are kept here as explicit sliding windows (the last
 * min(L, att_left) K/V rows and the last conv_kernel-1 GLU rows), not as the reference's
 * append-only buffers with epoch compaction.  Both describe the same sequence of values, so a
 * mismatch against an implementation that uses the append-only layout shows up in parity tests.
 */
#include "oracle.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define OR_MEL_CACHE 16      /* src/encoder.c:10 */
#define OR_DEC_MAX_BATCH 16  /* src/kernel_params.h:17 */

static inline float bf(uint16_t v) {
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)v << 16;
    return c.f;
}
static float *widen(const uint16_t *src, size_t n) {
    float *d = malloc(sizeof(float) * (n ? n : 1));
    for (size_t i = 0; i < n; ++i) d[i] = bf(src[i]);
    return d;
}

typedef struct {
    float *ln_ff1_g, *ln_ff1_b, *ln_att_g, *ln_att_b, *ln_conv_g, *ln_conv_b, *ln_ff2_g, *ln_ff2_b, *ln_out_g, *ln_out_b;
    float *bn_g, *bn_b, *dw_w, *bias_u, *bias_v, *ptab;
    uint16_t *wqkv; /* [3D][D]: q, k, v rows stacked (src/model.c:240-242) */
} or_layer_t;

struct or_model {
    or_dims_t d;
    or_global_w_t g;
    or_layer_w_t *lw;
    or_layer_t *L;
    int Lmax, sub_freq_out;
    float *conv0_w, *conv0_b, *conv2_w, *conv2_b, *conv3_b, *conv5_w, *conv5_b, *conv6_b, *pre_out_b;
    float *prompt_b2, *b0_eff, *lstm_b[2], *joint_enc_b, *joint_pred_b, *joint_out_b;
};

or_model_t *or_model_create(const or_dims_t *dims, const or_global_w_t *g, const or_layer_w_t *layers) {
    or_model_t *m = calloc(1, sizeof *m);
    m->d = *dims;
    m->g = *g;
    const or_dims_t *d = &m->d;
    const size_t D = (size_t)d->d_model, CH = (size_t)d->sub_channels;
    m->lw = malloc(sizeof(or_layer_w_t) * (size_t)d->n_layers);
    memcpy(m->lw, layers, sizeof(or_layer_w_t) * (size_t)d->n_layers);
    /* src/model.c:168: Lmax = att_left + max trained right context + 1 + 2 */
    m->Lmax = d->att_left + d->max_right + 1 + 2;
    int f = d->feat_in;
    for (int i = 0; i < 3; ++i) f = f / 2 + 1; /* src/model.c:226-228 */
    m->sub_freq_out = f;
    m->conv0_w = widen(g->conv0_w, CH * 9); m->conv0_b = widen(g->conv0_b, CH);
    m->conv2_w = widen(g->conv2_w, CH * 9); m->conv2_b = widen(g->conv2_b, CH);
    m->conv3_b = widen(g->conv3_b, CH);
    m->conv5_w = widen(g->conv5_w, CH * 9); m->conv5_b = widen(g->conv5_b, CH);
    m->conv6_b = widen(g->conv6_b, CH);
    m->pre_out_b = widen(g->pre_out_b, D);
    m->prompt_b2 = widen(g->prompt_b2, D);
    m->b0_eff = calloc((size_t)d->prompt_hidden, sizeof(float));
    const size_t P = (size_t)d->pred_hidden;
    for (int l = 0; l < 2; ++l) m->lstm_b[l] = widen(g->lstm_b[l], 4 * P);
    m->joint_enc_b = widen(g->joint_enc_b, (size_t)d->joint_hidden);
    m->joint_pred_b = widen(g->joint_pred_b, (size_t)d->joint_hidden);
    m->joint_out_b = widen(g->joint_out_b, (size_t)d->num_classes);
    m->L = calloc((size_t)d->n_layers, sizeof(or_layer_t));
    const int Prow = 2 * m->Lmax - 1;
    for (int l = 0; l < d->n_layers; ++l) {
        const or_layer_w_t *w = &layers[l];
        or_layer_t *L = &m->L[l];
        L->ln_ff1_g = widen(w->ln_ff1_g, D); L->ln_ff1_b = widen(w->ln_ff1_b, D);
        L->ln_att_g = widen(w->ln_att_g, D); L->ln_att_b = widen(w->ln_att_b, D);
        L->ln_conv_g = widen(w->ln_conv_g, D); L->ln_conv_b = widen(w->ln_conv_b, D);
        L->ln_ff2_g = widen(w->ln_ff2_g, D); L->ln_ff2_b = widen(w->ln_ff2_b, D);
        L->ln_out_g = widen(w->ln_out_g, D); L->ln_out_b = widen(w->ln_out_b, D);
        L->bn_g = widen(w->bn_g, D); L->bn_b = widen(w->bn_b, D);
        L->dw_w = widen(w->dw_w, D * (size_t)d->conv_kernel);
        L->bias_u = widen(w->bias_u, D); L->bias_v = widen(w->bias_v, D);
        L->wqkv = malloc(sizeof(uint16_t) * 3 * D * D);
        memcpy(L->wqkv, w->wq, sizeof(uint16_t) * D * D);
        memcpy(L->wqkv + D * D, w->wk, sizeof(uint16_t) * D * D);
        memcpy(L->wqkv + 2 * D * D, w->wv, sizeof(uint16_t) * D * D);
        L->ptab = malloc(sizeof(float) * (size_t)Prow * D);
        or_ptab(w->wpos, (int)D, m->Lmax, L->ptab);
    }
    return m;
}

void or_model_free(or_model_t *m) {
    if (!m) return;
    for (int l = 0; l < m->d.n_layers; ++l) {
        or_layer_t *L = &m->L[l];
        float *fs[] = { L->ln_ff1_g, L->ln_ff1_b, L->ln_att_g, L->ln_att_b, L->ln_conv_g, L->ln_conv_b, L->ln_ff2_g,
                        L->ln_ff2_b, L->ln_out_g, L->ln_out_b, L->bn_g, L->bn_b, L->dw_w, L->bias_u, L->bias_v, L->ptab };
        for (size_t i = 0; i < sizeof fs / sizeof *fs; ++i) free(fs[i]);
        free(L->wqkv);
    }
    free(m->L);
    free(m->lw);
    float *fs[] = { m->conv0_w, m->conv0_b, m->conv2_w, m->conv2_b, m->conv3_b, m->conv5_w, m->conv5_b, m->conv6_b,
                    m->pre_out_b, m->prompt_b2, m->b0_eff, m->lstm_b[0], m->lstm_b[1], m->joint_enc_b, m->joint_pred_b,
                    m->joint_out_b };
    for (size_t i = 0; i < sizeof fs / sizeof *fs; ++i) free(fs[i]);
    free(m);
}

/* src/model.c:312-322: the one-hot prompt folds into the first prompt layer's bias:
 * b_eff[n] = b0[n] + W0[n][D + idx], both widened from bf16, summed in f32. */
int or_model_set_language(or_model_t *m, int idx) {
    if (idx < 0 || idx >= m->d.num_prompts) return -1;
    const size_t ld = (size_t)m->d.d_model + (size_t)m->d.num_prompts;
    for (int n = 0; n < m->d.prompt_hidden; ++n)
        m->b0_eff[n] = bf(m->g.prompt_b0[n]) + bf(m->g.prompt_w0[(size_t)n * ld + (size_t)m->d.d_model + (size_t)idx]);
    return 0;
}
const float *or_model_ptab(const or_model_t *m, int layer) { return m->L[layer].ptab; }
int or_model_lmax(const or_model_t *m) { return m->Lmax; }

/* ---- session ----------------------------------------------------------------------------- */
struct or_session {
    or_model_t *m;
    int right, chunk_frames, chunk_mel, cmax;
    /* encoder bookkeeping (src/encoder.c:39-82) */
    float *pending;
    size_t pending_n, pending_cap;
    float mel_cache[OR_MEL_CACHE * 128];
    int mel_cache_n;
    size_t consumed, emitted;
    int closed;
    /* sliding histories per layer */
    float **k_hist, **v_hist; /* [att_left][D] each, oldest first */
    int hist_len;
    float **conv_hist;        /* [conv_kernel-1][D], oldest first; zeros at start */
    /* decoder state (src/decoder.c:14-41) */
    float *h[2], *c[2], *hp[2], *cp[2], *pred_out;
    int last_token, pred_valid;
    /* stats + dumps */
    size_t chunks, frames, joint_steps;
    int dump;
    float *d_layers, *d_prompted, *d_joint;
    size_t d_cap;
    int *d_rows;
    size_t d_nrows_cap, d_nchunks;
    int *jl_best;
    float *jl_margin;
    size_t jl_n, jl_cap;
    /* per emitted token: the smallest top-2 margin over the decisions that produced it (the blank
     * frames passed since the previous token, then the emitting frame); seg_min is the running
     * minimum of the decisions since the last emitted token */
    float *tk_margin;
    size_t tk_n, tk_cap;
    float seg_min;
    /* committed greedy decisions (a blank frame or an emitted token; speculative scores of frames
     * redone after an emission are not counted): outcome, runner-up index, top-2 margin */
    int *cd_best, *cd_second;
    float *cd_margin;
    size_t cd_n, cd_cap;
    /* forced outcomes: committed decision force_at[i] takes token force_tok[i] (test hook: replays a
     * decode that took the other side of a float tie) */
    size_t *force_at;
    int *force_tok;
    size_t nforce;
    char err[256];
};

or_session_t *or_session_create(or_model_t *m, int right) {
    or_session_t *s = calloc(1, sizeof *s);
    s->m = m;
    const or_dims_t *d = &m->d;
    s->right = right;
    s->chunk_frames = right + 1;                      /* src/encoder.c:43-44 */
    s->chunk_mel = s->chunk_frames * d->subsampling;
    s->cmax = s->chunk_frames + 2;                     /* src/encoder.c:45-46 (final boundary window) */
    if (s->cmax < 16) s->cmax = 16;
    const size_t D = (size_t)d->d_model;
    s->k_hist = calloc((size_t)d->n_layers, sizeof(float *));
    s->v_hist = calloc((size_t)d->n_layers, sizeof(float *));
    s->conv_hist = calloc((size_t)d->n_layers, sizeof(float *));
    for (int l = 0; l < d->n_layers; ++l) {
        s->k_hist[l] = calloc((size_t)d->att_left * D, sizeof(float));
        s->v_hist[l] = calloc((size_t)d->att_left * D, sizeof(float));
        s->conv_hist[l] = calloc((size_t)(d->conv_kernel - 1) * D, sizeof(float));
    }
    const size_t P = (size_t)d->pred_hidden;
    for (int l = 0; l < 2; ++l) {
        s->h[l] = calloc(P, sizeof(float)); s->c[l] = calloc(P, sizeof(float));
        s->hp[l] = calloc(P, sizeof(float)); s->cp[l] = calloc(P, sizeof(float));
    }
    s->pred_out = calloc((size_t)d->joint_hidden, sizeof(float));
    or_session_reset(s);
    return s;
}

void or_session_free(or_session_t *s) {
    if (!s) return;
    for (int l = 0; l < s->m->d.n_layers; ++l) { free(s->k_hist[l]); free(s->v_hist[l]); free(s->conv_hist[l]); }
    free(s->k_hist); free(s->v_hist); free(s->conv_hist);
    for (int l = 0; l < 2; ++l) { free(s->h[l]); free(s->c[l]); free(s->hp[l]); free(s->cp[l]); }
    free(s->pred_out);
    free(s->pending);
    free(s->d_layers); free(s->d_prompted); free(s->d_joint); free(s->d_rows);
    free(s->jl_best); free(s->jl_margin); free(s->tk_margin);
    free(s->cd_best); free(s->cd_second); free(s->cd_margin);
    free(s->force_at); free(s->force_tok);
    free(s);
}

/* src/encoder.c:92-103 + src/decoder.c:48-53 */
void or_session_reset(or_session_t *s) {
    const or_dims_t *d = &s->m->d;
    const size_t D = (size_t)d->d_model, P = (size_t)d->pred_hidden;
    s->pending_n = 0;
    s->mel_cache_n = 0;
    s->consumed = s->emitted = 0;
    s->closed = 0;
    s->hist_len = 0;
    for (int l = 0; l < d->n_layers; ++l) memset(s->conv_hist[l], 0, sizeof(float) * (size_t)(d->conv_kernel - 1) * D);
    for (int l = 0; l < 2; ++l) { memset(s->h[l], 0, P * sizeof(float)); memset(s->c[l], 0, P * sizeof(float)); }
    s->last_token = d->blank_id;
    s->pred_valid = 0;
    s->chunks = s->frames = s->joint_steps = 0;
    s->d_nchunks = 0;
    s->jl_n = 0;
    s->tk_n = 0;
    s->cd_n = 0;
    s->seg_min = INFINITY;
}

/* The decisions to force in the next decodes of this session (committed decision index, token);
 * kept across reset.  n = 0 clears them. */
void or_session_force(or_session_t *s, const size_t *at, const int *tok, size_t n) {
    free(s->force_at);
    free(s->force_tok);
    s->force_at = n ? malloc(n * sizeof *s->force_at) : NULL;
    s->force_tok = n ? malloc(n * sizeof *s->force_tok) : NULL;
    for (size_t i = 0; i < n; ++i) { s->force_at[i] = at[i]; s->force_tok[i] = tok[i]; }
    s->nforce = n;
}

size_t or_session_decisions(const or_session_t *s, const int **best, const int **second, const float **margin) {
    *best = s->cd_best;
    *second = s->cd_second;
    *margin = s->cd_margin;
    return s->cd_n;
}

void or_session_set_dump(or_session_t *s, int on) { s->dump = on; }
size_t or_session_chunks(const or_session_t *s) { return s->chunks; }
size_t or_session_frames(const or_session_t *s) { return s->frames; }
size_t or_session_joint_steps(const or_session_t *s) { return s->joint_steps; }
const float *or_session_dump_layers(const or_session_t *s) { return s->d_layers; }
const float *or_session_dump_prompted(const or_session_t *s) { return s->d_prompted; }
const float *or_session_dump_joint_enc(const or_session_t *s) { return s->d_joint; }
const int *or_session_dump_chunk_rows(const or_session_t *s) { return s->d_rows; }
const char *or_session_error(const or_session_t *s) { return s->err; }
size_t or_session_joint_log(const or_session_t *s, const int **best, const float **margin) {
    *best = s->jl_best;
    *margin = s->jl_margin;
    return s->jl_n;
}
size_t or_session_token_margins(const or_session_t *s, const float **margin, float *tail) {
    *margin = s->tk_margin;
    *tail = s->seg_min;
    return s->tk_n;
}

static int sub_len(int n) { return n / 2 + 1; } /* src/encoder.c:118 */

/* src/encoder.c:213-251: which pending mel rows the next step consumes and which encoder rows
 * [lo, hi) of the subsampled window it emits (ConformerStreamingState bookkeeping). */
or_enc_plan_t or_enc_plan(or_enc_book_t *b, int final, int chunk_mel, int subsampling, int mel_cache) {
    or_enc_plan_t p;
    memset(&p, 0, sizeof p);
    if (b->closed) return p;
    if (b->pending_n == 0) { if (final) b->closed = 1; return p; }
    if ((int)b->pending_n < chunk_mel && !final) return p;
    size_t take = (size_t)chunk_mel < b->pending_n ? (size_t)chunk_mel : b->pending_n;
    p.include_boundary = final && b->pending_n == take;
    p.ran = 1;
    p.take = (int)take;
    p.nwin = b->mel_cache_n + (int)take;
    const size_t end = b->consumed + take;
    const size_t base = (b->consumed - (size_t)b->mel_cache_n) / (size_t)subsampling;
    const size_t lo = b->emitted - base;
    p.T3 = sub_len(sub_len(sub_len(p.nwin)));
    const size_t hi = p.include_boundary ? (size_t)p.T3 : end / (size_t)subsampling - base;
    b->consumed = end;
    b->mel_cache_n = p.nwin < mel_cache ? p.nwin : mel_cache;
    b->pending_n -= take;
    if (final && b->pending_n == 0) b->closed = 1;
    p.lo = (int)lo;
    p.hi = (int)hi;
    if (hi <= lo) {
        b->emitted = base + (lo > hi ? lo : hi);
        p.c = 0;
    } else {
        b->emitted = base + hi;
        p.c = (int)(hi - lo);
    }
    return p;
}

static void dump_grow(or_session_t *s, size_t rows_needed) {
    const or_dims_t *d = &s->m->d;
    if (rows_needed <= s->d_cap) return;
    size_t cap = s->d_cap ? s->d_cap : 64;
    while (cap < rows_needed) cap *= 2;
    s->d_layers = realloc(s->d_layers, cap * (size_t)d->n_layers * (size_t)d->d_model * sizeof(float));
    s->d_prompted = realloc(s->d_prompted, cap * (size_t)d->d_model * sizeof(float));
    s->d_joint = realloc(s->d_joint, cap * (size_t)d->joint_hidden * sizeof(float));
    s->d_cap = cap;
}

/* pre-encode of a window of nwin mel rows: src/encoder.c:120-142; returns T3 rows in out */
static int pre_encode(or_session_t *s, const float *win, int nwin, float **out) {
    or_model_t *m = s->m;
    const or_dims_t *d = &m->d;
    const int CH = d->sub_channels, F = d->feat_in;
    const int T1 = sub_len(nwin), F1 = F / 2 + 1, T2 = T1 / 2 + 1, F2 = F1 / 2 + 1, T3 = T2 / 2 + 1, F3 = F2 / 2 + 1;
    const int D = d->d_model;
    float *c0 = malloc(sizeof(float) * (size_t)T1 * F1 * CH);
    float *c1 = malloc(sizeof(float) * (size_t)T2 * F2 * CH);
    float *c2 = malloc(sizeof(float) * (size_t)T2 * F2 * CH);
    float *c3 = malloc(sizeof(float) * (size_t)T3 * F3 * CH);
    float *c4 = malloc(sizeof(float) * (size_t)T3 * F3 * CH);
    float *flat = malloc(sizeof(float) * (size_t)T3 * F3 * CH);
    float *po = malloc(sizeof(float) * (size_t)T3 * D);
    or_conv2d_c1_s2_relu(win, m->conv0_w, m->conv0_b, c0, nwin, F, T1, F1, CH);
    or_dwconv2d_s2(c0, m->conv2_w, m->conv2_b, c1, T1, F1, T2, F2, CH);
    or_gemm(c1, CH, m->g.conv3_w, CH, m->conv3_b, c2, CH, T2 * F2, CH, CH, OR_ACT_RELU, 0, 1.0f);
    or_dwconv2d_s2(c2, m->conv5_w, m->conv5_b, c3, T2, F2, T3, F3, CH);
    or_gemm(c3, CH, m->g.conv6_w, CH, m->conv6_b, c4, CH, T3 * F3, CH, CH, OR_ACT_RELU, 0, 1.0f);
    or_flatten_cf(c4, flat, T3, F3, CH);
    or_gemm(flat, (long)CH * F3, m->g.pre_out_w, (long)CH * F3, m->pre_out_b, po, D, T3, D, CH * F3, OR_ACT_NONE, 0, 1.0f);
    free(c0); free(c1); free(c2); free(c3); free(c4); free(flat);
    *out = po;
    return T3;
}

/* 24 conformer blocks + prompt + joint encoder projection on c rows: src/encoder.c:144-197.
 * Writes joint_enc [c][joint_hidden] (and prompted [c][D]). */
static void run_blocks(or_session_t *s, float *h, int c, float *prompted, float *joint_enc, float *dump_layers) {
    or_model_t *m = s->m;
    const or_dims_t *d = &m->d;
    const int D = d->d_model, FF = d->d_ff, H = d->n_heads, dh = d->head_dim, taps = d->conv_kernel;
    const int ch = taps - 1;
    const float eps = d->ln_eps;
    const int L = s->hist_len + c;
    const size_t rowb = sizeof(float) * (size_t)D;
    float *t = malloc(rowb * c), *t2 = malloc(rowb * c), *ff = malloc(sizeof(float) * (size_t)c * FF);
    float *qkv = malloc(3 * rowb * c), *att = malloc(rowb * c), *y = malloc(rowb * c);
    float *Kall = malloc(rowb * L), *Vall = malloc(rowb * L), *din = malloc(rowb * (ch + c));
    for (int l = 0; l < d->n_layers; ++l) {
        or_layer_t *W = &m->L[l];
        const or_layer_w_t *w = &m->lw[l];
        /* FF1 half step; for l > 0 the LN was produced by the previous paired LN (src/encoder.c:154-157) */
        if (l == 0) or_layernorm(h, W->ln_ff1_g, W->ln_ff1_b, t2, c, D, eps);
        or_gemm(t2, D, w->ff1_w1, D, NULL, ff, FF, c, FF, D, OR_ACT_SILU, 0, 1.0f);
        or_gemm(ff, FF, w->ff1_w2, FF, NULL, h, D, c, D, FF, OR_ACT_NONE, 1, 0.5f);
        /* attention (src/encoder.c:158-166) */
        or_layernorm(h, W->ln_att_g, W->ln_att_b, t, c, D, eps);
        or_gemm(t, D, W->wqkv, D, NULL, qkv, 3 * D, c, 3 * D, D, OR_ACT_NONE, 0, 1.0f);
        memcpy(Kall, s->k_hist[l], rowb * (size_t)s->hist_len);
        memcpy(Vall, s->v_hist[l], rowb * (size_t)s->hist_len);
        for (int i = 0; i < c; ++i) {
            memcpy(Kall + (size_t)(s->hist_len + i) * D, qkv + (size_t)i * 3 * D + D, rowb);
            memcpy(Vall + (size_t)(s->hist_len + i) * D, qkv + (size_t)i * 3 * D + 2 * D, rowb);
        }
        or_attention_rel(qkv, 3 * D, Kall, Vall, D, W->ptab, W->bias_u, W->bias_v, att, c, L, m->Lmax, H, dh, D,
                         1.0f / sqrtf((float)dh));
        or_gemm(att, D, w->wo, D, NULL, h, D, c, D, D, OR_ACT_NONE, 1, 1.0f);
        /* keep the last min(L, att_left) rows as the next chunk's K/V cache (src/encoder.c:196) */
        const int keep = L < d->att_left ? L : d->att_left;
        memmove(s->k_hist[l], Kall + (size_t)(L - keep) * D, rowb * (size_t)keep);
        memmove(s->v_hist[l], Vall + (size_t)(L - keep) * D, rowb * (size_t)keep);
        /* convolution module (src/encoder.c:167-175) */
        or_layernorm(h, W->ln_conv_g, W->ln_conv_b, t, c, D, eps);
        memcpy(din, s->conv_hist[l], rowb * (size_t)ch);
        or_gemm(t, D, w->pw1, D, NULL, din + (size_t)ch * D, D, c, 2 * D, D, OR_ACT_GLU, 0, 1.0f);
        or_dwconv_ln_silu(din, W->dw_w, W->bn_g, W->bn_b, y, c, D, taps, eps);
        memcpy(s->conv_hist[l], din + (size_t)c * D, rowb * (size_t)ch);
        or_gemm(y, D, w->pw2, D, NULL, h, D, c, D, D, OR_ACT_NONE, 1, 1.0f);
        /* FF2 half step + output norm (src/encoder.c:176-187) */
        or_layernorm(h, W->ln_ff2_g, W->ln_ff2_b, t, c, D, eps);
        or_gemm(t, D, w->ff2_w1, D, NULL, ff, FF, c, FF, D, OR_ACT_SILU, 0, 1.0f);
        or_gemm(ff, FF, w->ff2_w2, FF, NULL, h, D, c, D, FF, OR_ACT_NONE, 1, 0.5f);
        if (l + 1 < d->n_layers) {
            or_layer_t *Wn = &m->L[l + 1];
            or_layernorm2(h, W->ln_out_g, W->ln_out_b, Wn->ln_ff1_g, Wn->ln_ff1_b, t, t2, c, D, eps);
        } else {
            or_layernorm(h, W->ln_out_g, W->ln_out_b, t, c, D, eps);
        }
        memcpy(h, t, rowb * (size_t)c);
        if (dump_layers)
            for (int i = 0; i < c; ++i) memcpy(dump_layers + ((size_t)i * d->n_layers + l) * D, h + (size_t)i * D, rowb);
    }
    s->hist_len = L < d->att_left ? L : d->att_left;
    /* prompt (one-hot folded into the bias) + joint encoder projection (src/encoder.c:189-194) */
    const int PH = d->prompt_hidden, NP = d->num_prompts, JH = d->joint_hidden;
    float *ph = malloc(sizeof(float) * (size_t)c * PH);
    or_gemm(h, D, m->g.prompt_w0, D + NP, m->b0_eff, ph, PH, c, PH, D, OR_ACT_RELU, 0, 1.0f);
    or_gemm(ph, PH, m->g.prompt_w2, PH, m->prompt_b2, prompted, D, c, D, PH, OR_ACT_NONE, 0, 1.0f);
    or_gemm(prompted, D, m->g.joint_enc_w, D, m->joint_enc_b, joint_enc, JH, c, JH, D, OR_ACT_NONE, 0, 1.0f);
    free(ph);
    free(t); free(t2); free(ff); free(qkv); free(att); free(y); free(Kall); free(Vall); free(din);
}

/* prediction network: src/decoder.c:57-77 */
static void encode_pred(or_session_t *s) {
    or_model_t *m = s->m;
    const or_dims_t *d = &m->d;
    const int P = d->pred_hidden, J = d->joint_hidden;
    float *x = calloc((size_t)P, sizeof(float)), *gates = malloc(sizeof(float) * 4 * (size_t)P);
    if (s->last_token != d->blank_id)
        for (int i = 0; i < P; ++i) x[i] = bf(m->g.embed[(size_t)s->last_token * P + i]);
    const float *in = x;
    for (int l = 0; l < 2; ++l) {
        or_gemm(in, P, m->g.lstm_wx[l], P, m->lstm_b[l], gates, 4 * P, 1, 4 * P, P, OR_ACT_NONE, 0, 1.0f);
        or_gemm(s->h[l], P, m->g.lstm_wh[l], P, NULL, gates, 4 * P, 1, 4 * P, P, OR_ACT_NONE, 1, 1.0f);
        or_lstm_cell(gates, s->c[l], s->cp[l], s->hp[l], P);
        in = s->hp[l];
    }
    or_gemm(s->hp[1], P, m->g.joint_pred_w, P, m->joint_pred_b, s->pred_out, J, 1, J, P, OR_ACT_NONE, 0, 1.0f);
    free(x);
    free(gates);
}

static void jlog(or_session_t *s, int best, float margin) {
    if (s->jl_n == s->jl_cap) {
        s->jl_cap = s->jl_cap ? 2 * s->jl_cap : 1024;
        s->jl_best = realloc(s->jl_best, s->jl_cap * sizeof(int));
        s->jl_margin = realloc(s->jl_margin, s->jl_cap * sizeof(float));
    }
    s->jl_best[s->jl_n] = best;
    s->jl_margin[s->jl_n] = margin;
    s->jl_n++;
}

/* greedy RNNT over `frames` rows of joint_enc: src/decoder.c:92-127 */
static int decode(or_session_t *s, const float *joint_enc, int frames, int *out, int max_out) {
    or_model_t *m = s->m;
    const or_dims_t *d = &m->d;
    const int J = d->joint_hidden, V = d->num_classes;
    float *logits = malloc(sizeof(float) * (size_t)V);
    int n = 0, t = 0, symbols = 0;
    while (t < frames) {
        int rows = frames - t;
        if (rows > OR_DEC_MAX_BATCH) rows = OR_DEC_MAX_BATCH;
        if (!s->pred_valid) encode_pred(s);
        int res[OR_DEC_MAX_BATCH], res2[OR_DEC_MAX_BATCH];
        for (int i = 0; i < rows; ++i) {
            float bv;
            res[i] = or_joint_argmax(joint_enc + (size_t)(t + i) * J, s->pred_out, m->g.joint_out_w, m->joint_out_b, V, J,
                                     &bv, logits);
            float second = -INFINITY;
            res2[i] = -1;
            for (int k = 0; k < V; ++k)
                if (k != res[i] && logits[k] > second) { second = logits[k]; res2[i] = k; }
            jlog(s, res[i], bv - second);
        }
        s->joint_steps++;
        s->pred_valid = 1;
        int i = 0;
        for (; i < rows; ++i) {
            int pred = res[i];
            const float mg = s->jl_margin[s->jl_n - (size_t)rows + (size_t)i];
            for (size_t f = 0; f < s->nforce; ++f)
                if (s->force_at[f] == s->cd_n) pred = s->force_tok[f];
            if (s->cd_n == s->cd_cap) {
                s->cd_cap = s->cd_cap ? 2 * s->cd_cap : 1024;
                s->cd_best = realloc(s->cd_best, s->cd_cap * sizeof(int));
                s->cd_second = realloc(s->cd_second, s->cd_cap * sizeof(int));
                s->cd_margin = realloc(s->cd_margin, s->cd_cap * sizeof(float));
            }
            s->cd_best[s->cd_n] = pred;
            s->cd_second[s->cd_n] = res2[i];
            s->cd_margin[s->cd_n] = mg;
            s->cd_n++;
            if (mg < s->seg_min) s->seg_min = mg;
            if (pred == d->blank_id) { symbols = 0; continue; }
            if (s->tk_n == s->tk_cap) {
                s->tk_cap = s->tk_cap ? 2 * s->tk_cap : 1024;
                s->tk_margin = realloc(s->tk_margin, s->tk_cap * sizeof(float));
            }
            s->tk_margin[s->tk_n++] = s->seg_min;
            s->seg_min = INFINITY;
            if (n < max_out) out[n++] = pred;
            s->last_token = pred;
            for (int l = 0; l < 2; ++l) {
                float *tmp = s->h[l]; s->h[l] = s->hp[l]; s->hp[l] = tmp;
                tmp = s->c[l]; s->c[l] = s->cp[l]; s->cp[l] = tmp;
            }
            s->pred_valid = 0;
            symbols++;
            if (symbols >= d->max_symbols) { symbols = 0; i++; }
            break;
        }
        t += i;
    }
    free(logits);
    return n;
}

int or_session_feed_mel(or_session_t *s, const float *mel, size_t nframes, int final, int *tokens, int max_tokens) {
    or_model_t *m = s->m;
    const or_dims_t *d = &m->d;
    const int NM = d->feat_in, D = d->d_model, J = d->joint_hidden;
    if (nframes) {
        if (s->pending_n + nframes > s->pending_cap) {
            s->pending_cap = (s->pending_n + nframes) * 2;
            s->pending = realloc(s->pending, s->pending_cap * (size_t)NM * sizeof(float));
        }
        memcpy(s->pending + s->pending_n * NM, mel, nframes * (size_t)NM * sizeof(float));
        s->pending_n += nframes;
    }
    int ntok = 0;
    for (;;) {
        or_enc_book_t b = { s->pending_n, s->consumed, s->emitted, s->mel_cache_n, s->closed };
        const int cache_before = s->mel_cache_n;
        or_enc_plan_t p = or_enc_plan(&b, final, s->chunk_mel, d->subsampling, OR_MEL_CACHE);
        if (!p.ran) { s->closed = b.closed; break; }
        /* window = mel cache ++ the consumed pending rows (src/encoder.c:223-227) */
        float *win = malloc(sizeof(float) * (size_t)p.nwin * NM);
        memcpy(win, s->mel_cache, sizeof(float) * (size_t)cache_before * NM);
        memcpy(win + (size_t)cache_before * NM, s->pending, sizeof(float) * (size_t)p.take * NM);
        memcpy(s->mel_cache, win + (size_t)(p.nwin - b.mel_cache_n) * NM, sizeof(float) * (size_t)b.mel_cache_n * NM);
        memmove(s->pending, s->pending + (size_t)p.take * NM, (s->pending_n - (size_t)p.take) * NM * sizeof(float));
        s->pending_n = b.pending_n;
        s->consumed = b.consumed;
        s->emitted = b.emitted;
        s->mel_cache_n = b.mel_cache_n;
        s->closed = b.closed;
        if (p.c <= 0) { free(win); continue; }
        if (p.c > s->cmax) {
            snprintf(s->err, sizeof s->err, "chunk of %d rows exceeds buffer %d", p.c, s->cmax);
            free(win);
            return -1;
        }
        float *po;
        pre_encode(s, win, p.nwin, &po);
        free(win);
        const int c = p.c;
        float *h = malloc(sizeof(float) * (size_t)c * D);
        memcpy(h, po + (size_t)p.lo * D, sizeof(float) * (size_t)c * D);
        free(po);
        float *prompted = malloc(sizeof(float) * (size_t)c * D), *je = malloc(sizeof(float) * (size_t)c * J);
        float *dl = NULL;
        if (s->dump) {
            dump_grow(s, s->frames + (size_t)c);
            dl = s->d_layers + s->frames * (size_t)d->n_layers * D;
        }
        run_blocks(s, h, c, prompted, je, dl);
        if (s->dump) {
            memcpy(s->d_prompted + s->frames * (size_t)D, prompted, sizeof(float) * (size_t)c * D);
            memcpy(s->d_joint + s->frames * (size_t)J, je, sizeof(float) * (size_t)c * J);
            if (s->d_nchunks == s->d_nrows_cap) {
                s->d_nrows_cap = s->d_nrows_cap ? 2 * s->d_nrows_cap : 256;
                s->d_rows = realloc(s->d_rows, s->d_nrows_cap * sizeof(int));
            }
            s->d_rows[s->d_nchunks++] = c;
        }
        s->chunks++;
        s->frames += (size_t)c;
        const int n = decode(s, je, c, tokens ? tokens + ntok : NULL, tokens ? max_tokens - ntok : 0);
        ntok += n;
        free(h); free(prompted); free(je);
    }
    return ntok;
}
