/* Cache-aware streaming encoder (see encoder.h).
 *
 * Bookkeeping is that of the reference (src/encoder.c:18-267, mirroring NeMo's
 * ConformerStreamingState): a 16-row mel cache, the window/lo/hi rule, append-only per-layer K/V
 * and conv histories compacted once per epoch.  Device side:
 *   - every layer's K/V rows (q | k | v, 3D floats) live in one buffer [n_layers][cap_rows][3D],
 *     the GLU outputs (conv history) in [n_layers][cap_rows][D]; compaction of all layers is one
 *     launch per buffer;
 *   - the cache position of the chunk is read by the kernels from a small device descriptor
 *     written before the chunk, so one captured hipGraph per chunk shape (c, window length, lo)
 *     replays every chunk of a stream; steady-state chunks replay a single graph.
 */
#include "encoder.h"
#include "nemo_kernels.h"
#include "mel.h"
#include "../kernel_params.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define MEL_CACHE 16 /* src/encoder.c:10 */
#define MAX_GRAPHS 8
#define CHAIN_SPIN_DEFAULT (1u << 20) /* polls before a chain hand-off gives up: about half a second */

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec / 1e6;
}

typedef struct {
    int c, nwin, lo, seen;
    gpu_graph_t *graph;
    unsigned long long last_use;
} gslot_t;

struct encoder {
    model_t *m;
    gpu_t *g;
    int right, chunk_frames, chunk_mel, cmax, Lmax, left, conv_left;
    float *pending;
    size_t pending_n, pending_cap;
    float mel_cache[MEL_CACHE * MEL_NMEL];
    int mel_cache_n;
    size_t consumed, emitted;
    int closed;
    /* device buffers */
    gpu_buf_t *win, *c1, *c2, *c3, *c4, *flat;
    gpu_buf_t *h, *tmp, *t2, *xf, *ff, *att, *y, *ph, *prompted, *joint_enc;
    gpu_buf_t *kv, *din, *desc;
    size_t kv_stride, din_stride; /* floats per layer */
    int cap_rows, pos, cache_len;
    /* pinned staging: window rows then the descriptor */
    float *stage_win;
    int *stage_desc;
    /* graphs */
    int use_graphs, capture_first;
    int fuse; /* single-stream launch fusions (kernels/nk_fuse.hip) */
    /* one-row chunks: all blocks in one persistent launch (kernels/nk_chain.hip) */
    int chain, chain_ok;
    uint32_t chain_spin; /* 0: CHAIN_SPIN_DEFAULT */
    gpu_buf_t *ch_layers, *ch_ll, *ch_abort;
    int *ch_err;        /* pinned host word the chain reports a time-out in */
    unsigned epoch;     /* per-chunk tag base of the chain's hand-offs */
    gslot_t gs[MAX_GRAPHS];
    unsigned long long tick;
    /* dumps */
    int dump;
    gpu_buf_t *dump_dev;
    float *d_layers, *d_prompted, *d_joint;
    size_t d_frames, d_cap;
};

static int sub_len(int n) { return n / 2 + 1; } /* src/encoder.c:118 */

/* The persistent chain serves one-row chunks of the shape it is built for, on a device with
 * enough compute units to hold all its workgroups at once; everything else takes the per-kernel
 * sequence of run_blocks. */
static void chain_init(encoder_t *e) {
    const model_cfg_t *c = &e->m->cfg;
    gpu_t *g = e->g;
    e->chain_ok = c->d_model == NK_CHAIN_D && c->d_ff == NK_CHAIN_FF && c->n_heads == NK_CHAIN_HEADS &&
                  c->head_dim * c->n_heads == c->d_model && c->conv_kernel == NK_CONV_TAPS &&
                  c->n_layers > 0 && c->n_layers * NK_CHAIN_PH < 1024 && e->left + 1 <= NK_CHAIN_MAX_L &&
                  e->left + 1 <= e->Lmax && gpu_cu_count(g) >= NK_CHAIN_G;
    e->chain = e->chain_ok;
    if (!e->chain_ok) return;
    const int nl = c->n_layers;
    NkChainLayer *t = calloc((size_t)nl, sizeof *t);
    for (int l = 0; l < nl; ++l) {
        const layer_dev_t *W = &e->m->L[l];
        t[l] = (NkChainLayer){ W->ff1_w1, W->ff1_w2, W->wqkv, W->wo, W->pw1, W->pw2, W->ff2_w1, W->ff2_w2,
                               W->ln_ff1_g, W->ln_ff1_b, W->ln_att_g, W->ln_att_b, W->ln_conv_g, W->ln_conv_b,
                               W->ln_ff2_g, W->ln_ff2_b, W->ln_out_g, W->ln_out_b, W->bn_g, W->bn_b, W->dw_w,
                               W->bias_u, W->bias_v, W->ptab };
    }
    e->ch_layers = gpu_buf_alloc(g, (size_t)nl * sizeof *t);
    e->ch_ll = gpu_buf_alloc(g, (size_t)NK_CHAIN_SLOTS * NK_CHAIN_SLOT * sizeof(unsigned long long));
    e->ch_abort = gpu_buf_alloc(g, 256);
    e->ch_err = gpu_host_alloc(g, 64);
    if (!e->ch_layers || !e->ch_ll || !e->ch_abort || !e->ch_err || !gpu_host_dptr(g, e->ch_err) ||
        gpu_upload(g, gpu_buf_dptr(e->ch_layers), t, (size_t)nl * sizeof *t))
        e->chain_ok = e->chain = 0;
    free(t);
}

/* all conformer blocks of a one-row chunk: block 0 reads x_in, the last block leaves its residual
 * row (before its output norm) in x_out */
static void run_chain(encoder_t *e, const float *x_in, float *x_out) {
    const model_cfg_t *c = &e->m->cfg;
    gpu_t *g = e->g;
    NkChainArgs a;
    memset(&a, 0, sizeof a);
    a.L = gpu_buf_dptr(e->ch_layers);
    a.x_in = x_in;
    a.x_out = x_out;
    a.kv = gpu_buf_dptr(e->kv);
    a.din = gpu_buf_dptr(e->din);
    a.ll = gpu_buf_dptr(e->ch_ll);
    a.abort_word = gpu_buf_dptr(e->ch_abort);
    a.err_word = gpu_host_dptr(g, e->ch_err);
    a.dump = e->dump ? gpu_buf_dptr(e->dump_dev) : NULL;
    a.desc = gpu_buf_dptr(e->desc);
    a.kv_stride = e->kv_stride;
    a.din_stride = e->din_stride;
    a.n_layers = (uint32_t)c->n_layers;
    a.Lmax = (uint32_t)e->Lmax;
    a.spin_max = e->chain_spin ? e->chain_spin : CHAIN_SPIN_DEFAULT;
    a.eps = c->ln_eps;
    a.scale = 1.0f / sqrtf((float)c->head_dim);
    const double D = NK_CHAIN_D, FF = NK_CHAIN_FF;
    gpu_next_bytes(g, (double)c->n_layers * (4.0 * FF * D + 7.0 * D * D) * 2.0);
    gpu_launch(g, "enc_chain", &a, sizeof a, NK_CHAIN_G, 1, 1, NK_CHAIN_THREADS, 1, 1);
}

encoder_t *encoder_create(model_t *m, int right) {
    encoder_t *e = calloc(1, sizeof *e);
    e->m = m;
    e->g = m->gpu;
    const model_cfg_t *c = &m->cfg;
    e->right = right;
    e->chunk_frames = right + 1;
    e->chunk_mel = e->chunk_frames * c->subsampling;
    e->cmax = e->chunk_frames + 2; /* a final boundary window can yield up to chunk_frames + 2 rows */
    if (e->cmax < NK_FEW_ROWS) e->cmax = NK_FEW_ROWS;
    e->left = c->att_left;
    e->Lmax = m->Lmax;
    e->conv_left = c->conv_kernel - 1;
    const size_t D = (size_t)c->d_model, CH = (size_t)c->sub_channels, F = (size_t)c->feat_in;
    const size_t nwin = MEL_CACHE + (size_t)e->chunk_mel + 1;
    const size_t T1 = nwin / 2 + 1, F1 = F / 2 + 1, T2 = T1 / 2 + 1, F2 = F1 / 2 + 1, T3 = T2 / 2 + 1, F3 = F2 / 2 + 1;
    gpu_t *g = e->g;
    const size_t cm = (size_t)e->cmax, fs = sizeof(float);
    e->win = gpu_buf_alloc(g, nwin * F * fs);
    e->c1 = gpu_buf_alloc(g, T2 * F2 * CH * fs);
    e->c2 = gpu_buf_alloc(g, T2 * F2 * CH * fs);
    e->c3 = gpu_buf_alloc(g, T3 * F3 * CH * fs);
    e->c4 = gpu_buf_alloc(g, T3 * F3 * CH * fs);
    e->flat = gpu_buf_alloc(g, T3 * F3 * CH * fs);
    e->h = gpu_buf_alloc(g, cm * D * fs);
    e->tmp = gpu_buf_alloc(g, cm * D * fs);
    e->t2 = gpu_buf_alloc(g, cm * D * fs);
    e->xf = gpu_buf_alloc(g, cm * D * fs);
    e->ff = gpu_buf_alloc(g, cm * (size_t)c->d_ff * fs);
    e->att = gpu_buf_alloc(g, cm * D * fs);
    e->y = gpu_buf_alloc(g, cm * D * fs);
    e->ph = gpu_buf_alloc(g, cm * (size_t)c->prompt_hidden * fs);
    e->prompted = gpu_buf_alloc(g, cm * D * fs);
    e->joint_enc = gpu_buf_alloc(g, cm * (size_t)c->joint_hidden * fs);
    e->cap_rows = e->left + NK_CACHE_EPOCH_CHUNKS * e->cmax;
    e->kv_stride = (size_t)e->cap_rows * 3 * D;
    e->din_stride = (size_t)e->cap_rows * D;
    e->kv = gpu_buf_alloc(g, (size_t)c->n_layers * e->kv_stride * fs);
    e->din = gpu_buf_alloc(g, (size_t)c->n_layers * e->din_stride * fs);
    e->desc = gpu_buf_alloc(g, NK_DESC_INTS * sizeof(int));
    e->stage_win = gpu_host_alloc(g, nwin * F * fs + NK_DESC_INTS * sizeof(int) + 256);
    e->stage_desc = (int *)((char *)e->stage_win + ((nwin * F * fs + 255) / 256) * 256);
    e->use_graphs = 1;
    e->fuse = 1;
    e->pos = e->conv_left; /* rows [0, conv_left) stay zero: the empty conv history */
    chain_init(e);
    return e;
}

static void drop_graphs(encoder_t *e) {
    for (int i = 0; i < MAX_GRAPHS; ++i) {
        gpu_graph_free(e->gs[i].graph);
        memset(&e->gs[i], 0, sizeof e->gs[i]);
    }
}

void encoder_destroy(encoder_t *e) {
    if (!e) return;
    drop_graphs(e);
    gpu_buf_t *bufs[] = { e->win, e->c1, e->c2, e->c3, e->c4, e->flat, e->h, e->tmp, e->t2, e->xf, e->ff,
                          e->att, e->y, e->ph, e->prompted, e->joint_enc, e->kv, e->din, e->desc, e->dump_dev,
                          e->ch_layers, e->ch_ll, e->ch_abort };
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs; ++i) gpu_buf_free(bufs[i]);
    gpu_host_free(e->stage_win);
    gpu_host_free(e->ch_err);
    free(e->pending);
    free(e->d_layers);
    free(e->d_prompted);
    free(e->d_joint);
    free(e);
}

/* src/encoder.c:92-103: back to the state after create; the conv history rows [0, conv_left)
 * of every layer read as zeros again */
void encoder_reset(encoder_t *e) {
    e->pending_n = 0;
    e->mel_cache_n = 0;
    e->consumed = e->emitted = 0;
    e->closed = 0;
    e->cache_len = 0;
    e->pos = e->conv_left;
    const size_t D = (size_t)e->m->cfg.d_model;
    float *z = calloc((size_t)e->conv_left * D, sizeof(float));
    for (int l = 0; l < e->m->cfg.n_layers; ++l)
        gpu_upload(e->g, (float *)gpu_buf_dptr(e->din) + (size_t)l * e->din_stride, z, (size_t)e->conv_left * D * sizeof(float));
    free(z);
    e->d_frames = 0;
}

int encoder_right(const encoder_t *e) { return e->right; }
int encoder_chunk_frames(const encoder_t *e) { return e->chunk_frames; }
int encoder_chunk_mel(const encoder_t *e) { return e->chunk_mel; }
void encoder_use_graphs(encoder_t *e, int on) {
    e->use_graphs = on;
    if (!on) drop_graphs(e);
}

void encoder_capture_first(encoder_t *e, int on) { e->capture_first = on != 0; }
int encoder_graphs(const encoder_t *e) {
    int n = 0;
    for (int i = 0; i < MAX_GRAPHS; ++i) n += e->gs[i].graph != NULL;
    return n;
}

void encoder_fuse(encoder_t *e, int on) {
    if (e->fuse != on) drop_graphs(e);
    e->fuse = on;
}

void encoder_chain(encoder_t *e, int on) {
    if (e->chain != (on != 0)) drop_graphs(e);
    e->chain = on != 0;
}
int encoder_chain_usable(const encoder_t *e) { return e->chain_ok; }
void encoder_chain_spin(encoder_t *e, uint32_t spin_max) {
    if (e->chain_spin != spin_max) drop_graphs(e); /* captured launches hold the old bound */
    e->chain_spin = spin_max;
}

int encoder_check(encoder_t *e, char *err, size_t errlen) {
    if (e->ch_err && *(volatile int *)e->ch_err) {
        snprintf(err, errlen, "encoder chain: hand-off %d timed out", *(volatile int *)e->ch_err - 1);
        return -1;
    }
    return 0;
}

void encoder_set_dump(encoder_t *e, int on) {
    e->dump = on;
    if (on && !e->dump_dev)
        e->dump_dev = gpu_buf_alloc(e->g, (size_t)e->cmax * (size_t)e->m->cfg.n_layers * (size_t)e->m->cfg.d_model * sizeof(float));
}
size_t encoder_dump_frames(const encoder_t *e) { return e->d_frames; }
const float *encoder_dump_layers(const encoder_t *e) { return e->d_layers; }
const float *encoder_dump_prompted(const encoder_t *e) { return e->d_prompted; }
const float *encoder_dump_joint(const encoder_t *e) { return e->d_joint; }

void encoder_push(encoder_t *e, const float *mel, size_t nframes) {
    if (!nframes) return;
    if (e->pending_n + nframes > e->pending_cap) {
        e->pending_cap = (e->pending_n + nframes) * 2;
        e->pending = realloc(e->pending, e->pending_cap * MEL_NMEL * sizeof(float));
    }
    memcpy(e->pending + e->pending_n * MEL_NMEL, mel, nframes * MEL_NMEL * sizeof(float));
    e->pending_n += nframes;
}

/* src/encoder.c:213-251: ConformerStreamingState._encode_mel_chunk bookkeeping */
enc_plan_t enc_plan_step(enc_book_t *b, int final, int chunk_mel, int subsampling, int mel_cache) {
    enc_plan_t p;
    memset(&p, 0, sizeof p);
    if (b->closed) return p;
    if (b->pending_n == 0) {
        if (final) b->closed = 1;
        return p;
    }
    if ((int)b->pending_n < chunk_mel && !final) return p;
    const size_t take = b->pending_n < (size_t)chunk_mel ? b->pending_n : (size_t)chunk_mel;
    p.ran = 1;
    p.take = (int)take;
    p.include_boundary = final && b->pending_n == take;
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
    } else {
        b->emitted = base + hi;
        p.c = (int)(hi - lo);
    }
    return p;
}

/* subsampling of the window (nwin mel rows): src/encoder.c:120-142.  The output projection runs
 * only on the c rows the chunk emits (rows lo .. lo+c-1 of the subsampled window; the reference
 * projects all T3 rows and copies these, src/encoder.c:142, :258) and writes them into h. */
static void run_pre_encode(encoder_t *e, int nwin, int lo, int c) {
    model_t *m = e->m;
    gpu_t *g = e->g;
    const uint32_t CH = (uint32_t)m->cfg.sub_channels, F = (uint32_t)m->cfg.feat_in;
    const uint32_t T1 = (uint32_t)sub_len(nwin), F1 = F / 2 + 1, T2 = T1 / 2 + 1, F2 = F1 / 2 + 1, T3 = T2 / 2 + 1, F3 = F2 / 2 + 1;
    float *win = gpu_buf_dptr(e->win), *c1 = gpu_buf_dptr(e->c1), *c2 = gpu_buf_dptr(e->c2);
    float *c3 = gpu_buf_dptr(e->c3), *c4 = gpu_buf_dptr(e->c4), *flat = gpu_buf_dptr(e->flat);
    /* conv 0 + ReLU and the first depthwise conv in one launch (conv 0's output is not stored) */
    nk_conv2d_c1_dw_s2_b(g, win, m->conv0_w, m->conv0_b, m->conv2_w, m->conv2_b, c1, (uint32_t)nwin, F, T1, F1, T2,
                         F2, CH, 1);
    nk_gemm(g, c1, CH, m->conv3_w, CH, m->conv3_b, c2, CH, T2 * F2, CH, CH, NK_ACT_RELU, 0, 1.0f);
    nk_dwconv2d_s2(g, c2, m->conv5_w, m->conv5_b, c3, T2, F2, T3, F3, CH);
    nk_gemm(g, c3, CH, m->conv6_w, CH, m->conv6_b, c4, CH, T3 * F3, CH, CH, NK_ACT_RELU, 0, 1.0f);
    nk_flatten_cf(g, c4, flat, T3, F3, CH);
    const uint32_t D = (uint32_t)m->cfg.d_model, K = CH * F3;
    nk_gemm(g, flat + (size_t)lo * K, K, m->pre_out_w, K, m->pre_out_b, gpu_buf_dptr(e->h), D, (uint32_t)c, D, K,
            NK_ACT_NONE, 0, 1.0f);
}

/* 24 conformer blocks + prompt + joint projection on the c rows in e->h: src/encoder.c:144-197.
 * Cache positions come from the device descriptor.  Every LayerNorm in front of a GEMM runs in
 * that GEMM's prologue: the output norm of block l and the FF1 norm of block l+1 run in block
 * l+1's first GEMM, which also writes the normalised residual into the other residual buffer
 * (the reference's h/t swap, src/encoder.c:180-187). */
static void run_blocks(encoder_t *e, int c) {
    model_t *m = e->m;
    gpu_t *g = e->g;
    const model_cfg_t *cf = &m->cfg;
    const uint32_t D = (uint32_t)cf->d_model, FF = (uint32_t)cf->d_ff, H = (uint32_t)cf->n_heads, dh = (uint32_t)cf->head_dim;
    const uint32_t uc = (uint32_t)c, nl = (uint32_t)cf->n_layers;
    const float eps = cf->ln_eps, scale = 1.0f / sqrtf((float)dh);
    const int *desc = gpu_buf_dptr(e->desc);
    const int *rows = desc + NK_DESC_ROWS;
    float *R[2] = { gpu_buf_dptr(e->h), gpu_buf_dptr(e->tmp) };
    float *lnbuf = gpu_buf_dptr(e->t2); /* LayerNorm output when the GEMM cannot take it as a prologue */
    float *xdead = gpu_buf_dptr(e->xf);  /* residual rows after a pending update that nothing reads again */
    float *ff = gpu_buf_dptr(e->ff), *att = gpu_buf_dptr(e->att), *y = gpu_buf_dptr(e->y);
    float *dump = e->dump ? gpu_buf_dptr(e->dump_dev) : NULL;
    if (e->chain && uc == 1) {
        /* one row: every block in the persistent chain; its output row in R[1] */
        run_chain(e, R[0], R[1]);
        const layer_dev_t *Wl = &m->L[nl - 1];
        const uint32_t PH = (uint32_t)cf->prompt_hidden, NP = (uint32_t)cf->num_prompts, JH = (uint32_t)cf->joint_hidden;
        float *ph = gpu_buf_dptr(e->ph), *pr = gpu_buf_dptr(e->prompted);
        float *hn = dump ? R[0] : NULL;
        nk_gemm_ln(g, R[1], D, m->prompt_w0, D + NP, m->prompt_b0_eff, ph, PH, NULL, uc, PH, D, NK_ACT_RELU, 0, 1.0f, 1,
                   Wl->ln_out_g, Wl->ln_out_b, NULL, NULL, hn, lnbuf, eps);
        if (dump) nk_copy2d(g, hn, D, dump + (size_t)(nl - 1) * D, D * nl, uc, D);
        nk_gemm(g, ph, PH, m->prompt_w2, PH, m->prompt_b2, pr, D, uc, D, PH, NK_ACT_NONE, 0, 1.0f);
        nk_gemm(g, pr, D, m->joint_enc_w, D, m->joint_enc_b, gpu_buf_dptr(e->joint_enc), JH, uc, JH, D, NK_ACT_NONE, 0, 1.0f);
        return;
    }
    /* one or two rows per chunk: attention + out_proj and dwconv + pw2 as one launch each */
    const int fuse_att = e->fuse && uc <= 4 && dh == 128 && D % 128 == 0;
    const int fuse_conv = e->fuse && uc <= 2 && D <= 1024 && D % 8 == 0 && cf->conv_kernel == NK_CONV_TAPS;
    int cur = 0;
    /* A residual update may stay pending (its partial rows in the context's scratch: the few-row
     * kernel's K shares, or the fused attention's heads) until the next LayerNorm-fused GEMM, which
     * adds it to the residual in its prologue and writes the updated rows to the other buffer. */
    nk_resid_t pend = { 0 };
#define LN_GEMM(Wt, C, ldc, crow, N, act, g1, b1)                                                          \
    do {                                                                                                   \
        float *xf = pend.nparts ? R[cur ^ 1] : NULL;                                                       \
        nk_gemm_ln_pend(g, R[cur], D, Wt, D, NULL, C, ldc, crow, uc, N, D, act, 0, 1.0f, 1, g1, b1, NULL, NULL, NULL, \
                        lnbuf, eps, &pend, xf);                                                            \
        if (xf) cur ^= 1;                                                                                  \
        pend.nparts = 0;                                                                                   \
    } while (0)
    for (uint32_t l = 0; l < nl; ++l) {
        const layer_dev_t *W = &m->L[l];
        float *kv = (float *)gpu_buf_dptr(e->kv) + (size_t)l * e->kv_stride;
        float *din = (float *)gpu_buf_dptr(e->din) + (size_t)l * e->din_stride;
        /* FF1 half step (LN of block l-1's output, then this block's FF1 norm; block l-1's last
         * update added first) */
        if (l == 0) {
            nk_gemm_ln(g, R[0], D, W->ff1_w1, D, NULL, ff, FF, NULL, uc, FF, D, NK_ACT_SILU, 0, 1.0f, 1, W->ln_ff1_g,
                       W->ln_ff1_b, NULL, NULL, NULL, lnbuf, eps);
        } else {
            const layer_dev_t *Wp = &m->L[l - 1];
            const int prev = cur;
            cur ^= 1;
            nk_gemm_ln_pend(g, R[prev], D, W->ff1_w1, D, NULL, ff, FF, NULL, uc, FF, D, NK_ACT_SILU, 0, 1.0f, 2,
                            Wp->ln_out_g, Wp->ln_out_b, W->ln_ff1_g, W->ln_ff1_b, R[cur], lnbuf, eps, &pend,
                            pend.nparts ? xdead : NULL);
            pend.nparts = 0;
            if (dump) nk_copy2d(g, R[cur], D, dump + (size_t)(l - 1) * D, D * nl, uc, D);
        }
        nk_gemm_pend(g, ff, FF, W->ff1_w2, FF, R[cur], D, uc, D, FF, 0.5f, &pend);
        /* attention: fused q|k|v projection written into cache rows pos .. pos+c-1 */
        LN_GEMM(W->wqkv, kv, 3 * D, rows, 3 * D, NK_ACT_NONE, W->ln_att_g, W->ln_att_b);
        if (fuse_att) {
            /* the heads' partial rows stay pending for the conv module's LN-fused pw1 */
            nk_attention_out_desc_pend(g, kv, 3 * D, desc, W->ptab, W->bias_u, W->bias_v, uc, (uint32_t)e->Lmax, H, dh,
                                       D, scale, W->wo, D, 1.0f, &pend);
        } else {
            nk_attention_rel_desc(g, kv, 3 * D, desc, W->ptab, W->bias_u, W->bias_v, att, uc, (uint32_t)e->Lmax, H, dh,
                                  D, scale);
            nk_gemm_pend(g, att, D, W->wo, D, R[cur], D, uc, D, D, 1.0f, &pend);
        }
        /* convolution module: GLU output appended to the conv history, causal depthwise conv over it */
        LN_GEMM(W->pw1, din, D, rows, 2 * D, NK_ACT_GLU, W->ln_conv_g, W->ln_conv_b);
        if (fuse_conv) {
            nk_dwconv_pw_desc(g, din, desc, W->dw_w, W->bn_g, W->bn_b, eps, W->pw2, D, R[cur], D, uc, D, D, 1, 1.0f);
        } else {
            nk_dwconv_ln_silu_desc(g, din, desc, W->dw_w, W->bn_g, W->bn_b, y, uc, D, (uint32_t)cf->conv_kernel, eps);
            nk_gemm_pend(g, y, D, W->pw2, D, R[cur], D, uc, D, D, 1.0f, &pend);
        }
        /* FF2 half step; its update stays pending for the next block's (or the prompt's) LayerNorm */
        LN_GEMM(W->ff2_w1, ff, FF, NULL, FF, NK_ACT_SILU, W->ln_ff2_g, W->ln_ff2_b);
        nk_gemm_pend(g, ff, FF, W->ff2_w2, FF, R[cur], D, uc, D, FF, 0.5f, &pend);
    }
#undef LN_GEMM
    /* last output norm in the prompt GEMM's prologue, language prompt (one-hot folded into the
     * bias) and joint encoder projection */
    const layer_dev_t *Wl = &m->L[nl - 1];
    const uint32_t PH = (uint32_t)cf->prompt_hidden, NP = (uint32_t)cf->num_prompts, JH = (uint32_t)cf->joint_hidden;
    float *ph = gpu_buf_dptr(e->ph), *pr = gpu_buf_dptr(e->prompted);
    float *hn = dump ? R[cur ^ 1] : NULL;
    nk_gemm_ln_pend(g, R[cur], D, m->prompt_w0, D + NP, m->prompt_b0_eff, ph, PH, NULL, uc, PH, D, NK_ACT_RELU, 0, 1.0f,
                    1, Wl->ln_out_g, Wl->ln_out_b, NULL, NULL, hn, lnbuf, eps, &pend,
                    pend.nparts ? xdead : NULL);
    if (dump) nk_copy2d(g, hn, D, dump + (size_t)(nl - 1) * D, D * nl, uc, D);
    nk_gemm(g, ph, PH, m->prompt_w2, PH, m->prompt_b2, pr, D, uc, D, PH, NK_ACT_NONE, 0, 1.0f);
    nk_gemm(g, pr, D, m->joint_enc_w, D, m->joint_enc_b, gpu_buf_dptr(e->joint_enc), JH, uc, JH, D, NK_ACT_NONE, 0, 1.0f);
}

/* everything a chunk launches after the uploads: pre-encode (its emitted rows into h), blocks */
static void launch_chunk(encoder_t *e, int nwin, int lo, int c) {
    run_pre_encode(e, nwin, lo, c);
    run_blocks(e, c);
}

static gslot_t *graph_slot(encoder_t *e, int c, int nwin, int lo) {
    gslot_t *free_slot = NULL, *lru = &e->gs[0];
    for (int i = 0; i < MAX_GRAPHS; ++i) {
        gslot_t *s = &e->gs[i];
        if (s->seen && s->c == c && s->nwin == nwin && s->lo == lo) return s;
        if (!s->seen && !free_slot) free_slot = s;
        if (s->last_use < lru->last_use) lru = s;
    }
    gslot_t *s = free_slot ? free_slot : lru;
    gpu_graph_free(s->graph);
    memset(s, 0, sizeof *s);
    s->c = c;
    s->nwin = nwin;
    s->lo = lo;
    return s;
}

/* Once per epoch: move the live history to the front of the per-layer buffers
 * (src/encoder.c:199-211).  Regions never overlap because cap_rows >= 2*left + cmax. */
static void compact_caches(encoder_t *e) {
    const uint32_t D = (uint32_t)e->m->cfg.d_model, nl = (uint32_t)e->m->cfg.n_layers;
    const int src_kv = e->pos - e->cache_len, src_din = e->pos - e->conv_left, dst_din = e->cache_len - e->conv_left;
    if (e->cache_len > 0)
        nk_compact(e->g, gpu_buf_dptr(e->kv), e->kv_stride, nl, (uint32_t)e->cache_len, 3 * D, (uint32_t)src_kv, 0);
    nk_compact(e->g, gpu_buf_dptr(e->din), e->din_stride, nl, (uint32_t)e->conv_left, D, (uint32_t)src_din, (uint32_t)dst_din);
    e->pos = e->cache_len;
}

int encoder_step(encoder_t *e, int final, enc_out_t *out, char *err, size_t errlen) {
    memset(out, 0, sizeof *out);
    enc_book_t b = { e->pending_n, e->consumed, e->emitted, e->mel_cache_n, e->closed };
    const int cache_before = e->mel_cache_n;
    const enc_plan_t p = enc_plan_step(&b, final, e->chunk_mel, e->m->cfg.subsampling, MEL_CACHE);
    e->closed = b.closed;
    if (!p.ran) return 0;
    const double t0 = now_ms();
    /* the previous step's uploads read the pinned staging: wait for them before rewriting it */
    gpu_wait_deferred(e->g);
    /* window = mel cache ++ the consumed rows, written into pinned staging */
    float *w = e->stage_win;
    memcpy(w, e->mel_cache, (size_t)cache_before * MEL_NMEL * sizeof(float));
    memcpy(w + (size_t)cache_before * MEL_NMEL, e->pending, (size_t)p.take * MEL_NMEL * sizeof(float));
    memcpy(e->mel_cache, w + (size_t)(p.nwin - b.mel_cache_n) * MEL_NMEL, (size_t)b.mel_cache_n * MEL_NMEL * sizeof(float));
    memmove(e->pending, e->pending + (size_t)p.take * MEL_NMEL, (e->pending_n - (size_t)p.take) * MEL_NMEL * sizeof(float));
    e->pending_n = b.pending_n;
    e->consumed = b.consumed;
    e->emitted = b.emitted;
    e->mel_cache_n = b.mel_cache_n;
    if (p.c <= 0) {
        out->wall_ms = now_ms() - t0;
        return 1;
    }
    const int c = p.c;
    if (c > e->cmax) { snprintf(err, errlen, "chunk of %d rows exceeds buffer %d", c, e->cmax); return -1; }
    gpu_t *g = e->g;
    gpu_begin(g);
    if (e->pos + c > e->cap_rows) compact_caches(e);
    const int L = e->cache_len + c;
    if (L > e->Lmax || e->pos < e->cache_len || e->pos < e->conv_left || e->pos + c > e->cap_rows) {
        snprintf(err, errlen, "cache bookkeeping out of range (pos %d, cache %d, c %d)", e->pos, e->cache_len, c);
        gpu_end(g, NULL, 0);
        return -1;
    }
    int *d = e->stage_desc;
    d[NK_DESC_POS] = e->pos;
    d[NK_DESC_CACHE] = e->cache_len;
    d[NK_DESC_L] = L;
    d[NK_DESC_C] = c;
    for (int i = 0; i < NK_FEW_ROWS; ++i) d[NK_DESC_ROWS + i] = e->pos + (i < c ? i : c - 1);
    e->epoch = e->epoch + 1 < (1u << 22) ? e->epoch + 1 : 1; /* tag base epoch << 10 stays in 32 bits */
    d[NK_DESC_EPOCH] = (int)e->epoch;
    gpu_upload_async(g, gpu_buf_dptr(e->win), w, (size_t)p.nwin * MEL_NMEL * sizeof(float));
    gpu_upload_async(g, gpu_buf_dptr(e->desc), d, NK_DESC_INTS * sizeof(int));
    if (e->use_graphs && !e->dump) {
        gslot_t *s = graph_slot(e, c, p.nwin, p.lo);
        s->last_use = ++e->tick;
        if (!s->graph && (s->seen >= 1 || e->capture_first)) {
            /* second chunk of this shape (first, during warm-up): capture it once, replay from now on */
            if (!gpu_capture_begin(g)) {
                launch_chunk(e, p.nwin, p.lo, c);
                s->graph = gpu_capture_end(g);
            }
        }
        s->seen++;
        if (s->graph) gpu_graph_launch(g, s->graph);
        else launch_chunk(e, p.nwin, p.lo, c);
    } else {
        launch_chunk(e, p.nwin, p.lo, c);
    }
    e->pos += c;
    e->cache_len = L < e->left ? L : e->left;
    if (e->dump ? gpu_end(g, err, errlen) : gpu_end_nowait(g, err, errlen)) return -1;
    if (e->dump) {
        const model_cfg_t *cf = &e->m->cfg;
        const size_t D = (size_t)cf->d_model, nl = (size_t)cf->n_layers, J = (size_t)cf->joint_hidden;
        if (e->d_frames + (size_t)c > e->d_cap) {
            e->d_cap = (e->d_frames + (size_t)c) * 2;
            e->d_layers = realloc(e->d_layers, e->d_cap * nl * D * sizeof(float));
            e->d_prompted = realloc(e->d_prompted, e->d_cap * D * sizeof(float));
            e->d_joint = realloc(e->d_joint, e->d_cap * J * sizeof(float));
        }
        gpu_download(g, e->d_layers + e->d_frames * nl * D, gpu_buf_dptr(e->dump_dev), (size_t)c * nl * D * sizeof(float));
        gpu_download(g, e->d_prompted + e->d_frames * D, gpu_buf_dptr(e->prompted), (size_t)c * D * sizeof(float));
        gpu_download(g, e->d_joint + e->d_frames * J, gpu_buf_dptr(e->joint_enc), (size_t)c * J * sizeof(float));
        e->d_frames += (size_t)c;
    }
    out->frames = c;
    out->prompted = gpu_buf_dptr(e->prompted);
    out->joint_enc = gpu_buf_dptr(e->joint_enc);
    out->gpu_ms = e->dump ? gpu_last_ms(g) : 0.0;
    out->wall_ms = now_ms() - t0;
    return 1;
}

double encoder_take_gpu_ms(encoder_t *e) { return gpu_wait_deferred(e->g); }
