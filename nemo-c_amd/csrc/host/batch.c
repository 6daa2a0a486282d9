/* Multi-stream batching on one GPU (include/nemoasr_batch.h).
 *
 * Every stream keeps the reference's per-stream state: the mel bookkeeping of
 * src/encoder.c:213-251 (through enc_plan_step), a K/V and conv history, and the greedy decoder
 * state of src/decoder.c:14-23 (committed and provisional LSTM states, last token, whether the
 * prediction is valid).  A batched step takes one chunk from every stream that has one:
 *   - windows of equal length are subsampled together (batched conv launches, the 1x1 convs and
 *     the output projection as GEMMs over all their rows), and the rows each stream keeps
 *     ([lo, hi) of its window) are gathered into one matrix of M = sum(c_s) rows;
 *   - the 24 conformer blocks run once on those M rows: every GEMM is one many-row launch, the
 *     fused QKV and GLU GEMMs write each row to its stream's cache row, and attention and the
 *     depthwise conv read each row's stream window through a row table
 *     {cache row, index in chunk, chunk rows, cached rows};
 *   - the greedy RNNT loop then advances every stream's chunk together: one step runs the
 *     prediction network for the streams whose prediction is stale (LSTM layers as GEMMs over
 *     those streams' [x | h] rows with the input and recurrent weights side by side) and the
 *     joint + argmax for up to 16 pending frames of every stream, and the host applies the
 *     reference's rules to each stream's row of results.
 * Device layout: caches [n_layers][S][cap_rows][3D] (K/V) and [n_layers][S][cap_rows][D] (conv
 * history); LSTM states [S][2 sets][h0, c0, h1, c1][P].  The encoder launch sequence of a step
 * depends only on (M, the window groups), so it is captured as a hipGraph and replayed when the
 * same shape recurs (the lockstep steady state of a batch replays one graph). */
#include "nemoasr_batch.h"
#include "encoder.h"
#include "mel.h"
#include "model.h"
#include "nemo_kernels.h"
#include "../kernel_params.h"
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#define MEL_CACHE 16      /* src/encoder.c:10 */
#define DEC_WIN 16        /* frames scored per stream per joint evaluation, src/decoder.c:96-97 */
#define MAX_BGRAPHS 8
#define MAX_SIG_GROUPS 8
#define POOL_MAX 16       /* host threads for the log-mel front end of a step */
#define MEL_RING 512      /* device log-mel rows kept per stream (GPU front end) */

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec / 1e6;
}

static int sub_len(int n) { return n / 2 + 1; } /* src/encoder.c:118 */

typedef struct {
    melfe_t *mel;
    float *aq;                          /* audio queued for the front end */
    size_t aq_n, aq_cap;
    int ended, fe_final;                /* no more input; the front end flushes at the next step */
    float *pending;
    size_t pending_n, pending_cap;
    float mel_cache[MEL_CACHE * MEL_NMEL];
    int mel_cache_n;
    int src;                            /* GPU front end: 0 no input yet, 1 audio, 2 mel rows */
    size_t fr_taken;                    /* frames taken into windows so far */
    size_t fr_lo;                       /* oldest frame a window of the current step may read */
    size_t consumed, emitted;
    int closed, final;
    int pos, cache_len;                 /* cache rows of this stream */
    /* Decoder fields (through cap_tok).  Ownership between the caller's thread and the greedy-loop
     * worker: while a loop is queued or running (dstate != 0) only the worker touches them; the
     * caller's thread sets frames..erow0 for the next loop, and reads or resets any of them, only
     * after dec_drain() has returned (worker idle).  The encoder part of a step touches none of
     * them.  The same rule holds for the stats fields the worker adds to (decoder_ms, tokens,
     * joint_steps). */
    int last_token, pred_valid, cur;    /* cur = committed LSTM slot set */
    int frames, t, symbols, erow0;      /* the chunk in the decoder */
    int *tok;
    size_t n_tok, cap_tok, n_text;
    int printed_any;
    /* the chunk of the current step */
    int c, nwin, lo, row0, cache_before, gk, gj; /* gk, gj: window group and index in it */
    enc_book_t book;
    enc_plan_t plan;
} bstream_t;

typedef struct {
    int M, ng, nwin[MAX_SIG_GROUPS], cnt[MAX_SIG_GROUPS];
    gpu_graph_t *graph;
    int seen;
    unsigned long long last_use;
} bgraph_t;

/* Persistent worker threads: the front end of the streams with queued audio runs in parallel
 * (each stream's state is touched by one thread only). */
typedef struct {
    pthread_t th[POOL_MAX];
    int n, started, quit;
    unsigned gen;
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    int busy;
    int next, count;
    const int *list;
    struct nemoasr_batch *b;
} pool_t;

struct nemoasr_batch {
    pool_t pool;
    int *fe_list;
    model_t *m;
    gpu_t *g;
    int S, latency_ms, right, chunk_frames, chunk_mel, cmax, left, conv_left, Lmax, cap_rows;
    int nwin_max, T1max, T2max, T3max, F1, F2, F3;
    int Mmax;
    bstream_t *st;
    int *order, *gid;              /* streams with a chunk this step, in row order; their group */
    int ng, *g_nwin, *g_cnt, *g_woff, *g_poff, *g_fill, *ord;
    float *wtmp;                   /* host scratch for chunks that emit no rows */
    /* GPU log-mel front end: per-stream rings of mel rows; each step stages the sample spans of the
     * frames its windows take (frames are computed when taken), then one mel_frames launch fills
     * the rings and a row gather builds the windows */
    int gpu_fe;
    gpu_buf_t *ring, *meltab, *span_dev, *ftab_dev, *wmap_dev, *hrow_dev, *hmap_dev;
    float *stage_span, *stage_hrow;
    int *stage_ftab, *stage_wmap, *stage_hmap;
    size_t span_cap, span_n;       /* floats */
    size_t ftab_cap, ftab_n;       /* ints (two per frame) */
    size_t hrow_cap, hrow_n;       /* floats of mel rows given by the host (push_mel) */
    size_t hmap_cap, wmap_cap;     /* ints */
    /* encoder */
    gpu_buf_t *win, *c1, *c2, *c3, *c4, *flat, *pre_out;
    gpu_buf_t *h, *tmp, *lnb, *ff, *att, *y, *ph, *prompted, *joint_enc, *kv, *din, *etab;
    size_t kv_lstride, din_lstride;
    float *stage_win;
    int *stage_tab;
    bgraph_t gr[MAX_BGRAPHS];
    unsigned long long tick;
    int use_graphs, chunk_attn;
    /* decoder */
    int P, J, V, Vp;
    gpu_buf_t *wcat[2], *wout, *bout, *hc, *lin, *gates, *hout, *hout2, *pred, *jin, *logits, *amax, *dtab;
    int *stage_dtab, *stage_amax;
    /* device-resident loop (kernels/nk_bdec.hip) */
    int device_dec, W, tok_ld;
    gpu_buf_t *bst, *bsetup, *btok, *lin1, *tx, *wcati[2], *bi[2], *keys, *brows, *bcnt, *pre0;
    int nkeys;
    NkBDecStream *stage_bst;
    int *stage_bsetup, *stage_btok;
    gpu_graph_t *dgraph[2][6];     /* per joint.enc buffer, per run size (k_brun_steps) */
    /* pipelined greedy loop: a worker thread runs each step's loop on its own GPU context (its own
     * stream) while the caller's next step runs its front end and encoder; the step's joint.enc
     * rows are copied to jdec[parity] for it.  The queue holds one step: the next hand-off waits
     * for the previous loop, and every read of tokens or counters waits for the worker first. */
    gpu_t *gd;
    gpu_buf_t *jdec[2];
    int jpar;
    pthread_t dth;
    pthread_mutex_t dmu;
    pthread_cond_t dcv;
    int dstarted, dquit, dstate, drc; /* dstate: 0 idle, 1 queued, 2 running */
    /* Held by the worker while it captures a graph of the loop, and by the caller's thread for the
     * whole encoder part of a step (its own capture, staging allocations, synchronous copies):
     * a capture on one thread never overlaps allocations, synchronous copies or a capture on the
     * other.  Without it, a staging allocation of the encoder step that met the worker's first
     * capture failed now and then, and some steps decoded other tokens. */
    pthread_mutex_t cmu;
    char derr[256];
    int dnact, *dorder, *dc, *drow0, dbuf;
    double dt0;
    /* accounting */
    double *step_ms;
    size_t n_step, cap_step;
    nemoasr_batch_stats_t stats;
    /* test hook: joint.enc rows per stream */
    int dump;
    float **dj;
    size_t *dj_n, *dj_cap;
};

/* latency -> right context (src/nemoasr.c:58-64) */
static int right_for(int latency_ms) {
    static const int ms[] = { 80, 160, 320, 560, 1120 }, r[] = { 0, 1, 3, 6, 13 };
    for (size_t i = 0; i < sizeof ms / sizeof *ms; ++i)
        if (ms[i] == latency_ms) return r[i];
    return -1;
}

int nemoasr_batch_streams(const nemoasr_batch_t *b) { return b->S; }

static bgraph_t *bgraph_slot(nemoasr_batch_t *b, int M) {
    if (b->ng > MAX_SIG_GROUPS) return NULL;
    bgraph_t *free_slot = NULL, *lru = &b->gr[0];
    for (int i = 0; i < MAX_BGRAPHS; ++i) {
        bgraph_t *s = &b->gr[i];
        if (s->seen && s->M == M && s->ng == b->ng && !memcmp(s->nwin, b->g_nwin, (size_t)b->ng * sizeof(int)) &&
            !memcmp(s->cnt, b->g_cnt, (size_t)b->ng * sizeof(int)))
            return s;
        if (!s->seen && !free_slot) free_slot = s;
        if (s->last_use < lru->last_use) lru = s;
    }
    bgraph_t *s = free_slot ? free_slot : lru;
    gpu_graph_free(s->graph);
    memset(s, 0, sizeof *s);
    s->M = M;
    s->ng = b->ng;
    memcpy(s->nwin, b->g_nwin, (size_t)b->ng * sizeof(int));
    memcpy(s->cnt, b->g_cnt, (size_t)b->ng * sizeof(int));
    return s;
}

static void drop_graphs(nemoasr_batch_t *b) {
    for (int i = 0; i < MAX_BGRAPHS; ++i) {
        gpu_graph_free(b->gr[i].graph);
        memset(&b->gr[i], 0, sizeof b->gr[i]);
    }
}

static void pool_start(pool_t *p, struct nemoasr_batch *b);
static int dec_start(nemoasr_batch_t *b);
static void dec_stop(nemoasr_batch_t *b);
static void pool_stop(pool_t *p);

/* bf16 matrices of the batched decoder: [Wx | Wh] per LSTM layer ([4P][2P]) and the joint output
 * weights padded to a multiple of 64 rows (padding rows zero; the argmax reads the first V) */
static int build_decoder_weights(nemoasr_batch_t *b) {
    model_t *m = b->m;
    gpu_t *g = b->g;
    const size_t P = (size_t)b->P, J = (size_t)b->J, V = (size_t)b->V, Vp = (size_t)b->Vp;
    uint16_t *wx = malloc(4 * P * P * 2), *wh = malloc(4 * P * P * 2), *cat = malloc(4 * P * 2 * P * 2);
    int rc = 0;
    for (int l = 0; l < 2 && !rc; ++l) {
        rc |= gpu_download(g, wx, m->lstm_wx[l], 4 * P * P * 2);
        rc |= gpu_download(g, wh, m->lstm_wh[l], 4 * P * P * 2);
        for (size_t r = 0; r < 4 * P; ++r) {
            memcpy(cat + r * 2 * P, wx + r * P, P * 2);
            memcpy(cat + r * 2 * P + P, wh + r * P, P * 2);
        }
        b->wcat[l] = gpu_buf_alloc(g, 4 * P * 2 * P * 2);
        rc |= gpu_upload(g, gpu_buf_dptr(b->wcat[l]), cat, 4 * P * 2 * P * 2);
        /* the same rows interleaved by unit (row 4u + q = gate q of unit u) for the device loop,
           whose GEMM epilogue applies the LSTM cell, and the bias in the same order */
        uint16_t *ci = malloc(4 * P * 2 * P * 2);
        float *bh = malloc(4 * P * sizeof(float)), *bih = malloc(4 * P * sizeof(float));
        for (size_t u = 0; u < P; ++u)
            for (size_t q = 0; q < 4; ++q) memcpy(ci + (4 * u + q) * 2 * P, cat + (q * P + u) * 2 * P, 2 * P * 2);
        rc |= gpu_download(g, bh, m->lstm_b[l], 4 * P * sizeof(float));
        for (size_t u = 0; u < P; ++u)
            for (size_t q = 0; q < 4; ++q) bih[4 * u + q] = bh[q * P + u];
        b->wcati[l] = gpu_buf_alloc(g, 4 * P * 2 * P * 2);
        b->bi[l] = gpu_buf_alloc(g, 4 * P * sizeof(float));
        rc |= gpu_upload(g, gpu_buf_dptr(b->wcati[l]), ci, 4 * P * 2 * P * 2);
        rc |= gpu_upload(g, gpu_buf_dptr(b->bi[l]), bih, 4 * P * sizeof(float));
        free(ci);
        free(bh);
        free(bih);
    }
    /* layer-0 input table Tx = embed . Wx0^T + b0 (rows interleaved like wcati), one row per token
       and the blank row (zero input: the bias); the device loop looks it up instead of multiplying
       the embedding half of [x | h0] */
    const size_t NT = (size_t)m->cfg.blank_id + 1;
    uint16_t *eb = malloc(NT * P * 2);
    float *ef = malloc(NT * P * sizeof(float));
    gpu_buf_t *edev = gpu_buf_alloc(g, NT * P * sizeof(float));
    b->tx = gpu_buf_alloc(g, NT * 4 * P * sizeof(float));
    rc |= !eb || !ef || !edev || !b->tx;
    if (!rc) {
        rc |= gpu_download(g, eb, m->embed_dev, NT * P * 2);
        for (size_t i = 0; i < NT * P; ++i) {
            const uint32_t u = (uint32_t)eb[i] << 16;
            memcpy(&ef[i], &u, sizeof u);
            if (i / P == (size_t)m->cfg.blank_id) ef[i] = 0.0f;
        }
        rc |= gpu_upload(g, gpu_buf_dptr(edev), ef, NT * P * sizeof(float));
        rc |= gpu_begin(g);
        rc |= nk_gemm(g, gpu_buf_dptr(edev), (uint32_t)P, gpu_buf_dptr(b->wcati[0]), (uint32_t)(2 * P),
                      gpu_buf_dptr(b->bi[0]), gpu_buf_dptr(b->tx), (uint32_t)(4 * P), (uint32_t)NT, (uint32_t)(4 * P),
                      (uint32_t)P, NK_ACT_NONE, 0, 1.0f) < 0;
        rc |= gpu_end(g, NULL, 0);
    }
    free(eb);
    free(ef);
    gpu_buf_free(edev);
    uint16_t *wo = calloc(Vp * J, 2);
    float *bo = calloc(Vp, sizeof(float));
    rc |= gpu_download(g, wo, m->joint_out_w, V * J * 2);
    rc |= gpu_download(g, bo, m->joint_out_b, V * sizeof(float));
    b->wout = gpu_buf_alloc(g, Vp * J * 2);
    b->bout = gpu_buf_alloc(g, Vp * sizeof(float));
    rc |= gpu_upload(g, gpu_buf_dptr(b->wout), wo, Vp * J * 2);
    rc |= gpu_upload(g, gpu_buf_dptr(b->bout), bo, Vp * sizeof(float));
    free(wx);
    free(wh);
    free(cat);
    free(wo);
    free(bo);
    return rc;
}

/* ---- GPU log-mel front end ---------------------------------------------------------------------- */
/* device tables in one buffer: twiddles (2 x 256 double), window [512], filterbank [128][257],
 * filter bin ranges (2 x 128 int), bit reversal [512] u16 */
#define MT_TWR 0
#define MT_TWI (MT_TWR + 256 * 8)
#define MT_WIN (MT_TWI + 256 * 8)
#define MT_FB (MT_WIN + MEL_NFFT * 4)
#define MT_LO (MT_FB + MEL_NMEL * MEL_NBIN * 4)
#define MT_HI (MT_LO + MEL_NMEL * 4)
#define MT_REV (MT_HI + MEL_NMEL * 4)
#define MT_BYTES (MT_REV + MEL_NFFT * 2)

/* grow a pinned staging buffer and its device twin to hold `need` elements of `esz` bytes,
 * keeping the first `keep` elements of the staging buffer */
static int grow_stage(gpu_t *g, void **stage, gpu_buf_t **dev, size_t *cap, size_t need, size_t keep, size_t esz) {
    if (need <= *cap) return 0;
    size_t nc = *cap ? *cap : 1024;
    while (nc < need) nc *= 2;
    void *ns = gpu_host_alloc(g, nc * esz);
    gpu_buf_t *nd = dev ? gpu_buf_alloc(g, nc * esz) : NULL;
    if (!ns || (dev && !nd)) {
        gpu_host_free(ns);
        gpu_buf_free(nd);
        return -1;
    }
    if (keep && *stage) memcpy(ns, *stage, keep * esz);
    gpu_host_free(*stage);
    *stage = ns;
    if (dev) {
        gpu_buf_free(*dev);
        *dev = nd;
    }
    *cap = nc;
    return 0;
}

static int mel_gpu_setup(nemoasr_batch_t *b) {
    gpu_t *g = b->g;
    const size_t S = (size_t)b->S;
    b->gpu_fe = 1;
    b->ring = gpu_buf_alloc(g, S * MEL_RING * MEL_NMEL * sizeof(float));
    b->meltab = gpu_buf_alloc(g, MT_BYTES);
    b->wmap_dev = gpu_buf_alloc(g, S * (size_t)b->nwin_max * sizeof(int));
    b->stage_wmap = gpu_host_alloc(g, S * (size_t)b->nwin_max * sizeof(int));
    b->wmap_cap = S * (size_t)b->nwin_max;
    if (!b->ring || !b->meltab || !b->wmap_dev || !b->stage_wmap) return -1;
    melfe_t *mf = melfe_create();
    melfe_tables_t t;
    melfe_tables(mf, &t);
    char *h = calloc(1, MT_BYTES);
    memcpy(h + MT_TWR, t.tw_re, 256 * 8);
    memcpy(h + MT_TWI, t.tw_im, 256 * 8);
    memcpy(h + MT_WIN, t.win, MEL_NFFT * 4);
    memcpy(h + MT_FB, t.fb, MEL_NMEL * MEL_NBIN * 4);
    memcpy(h + MT_LO, t.fb_lo, MEL_NMEL * 4);
    memcpy(h + MT_HI, t.fb_hi, MEL_NMEL * 4);
    memcpy(h + MT_REV, t.rev, MEL_NFFT * 2);
    const int rc = gpu_upload(g, gpu_buf_dptr(b->meltab), h, MT_BYTES);
    free(h);
    melfe_destroy(mf);
    /* every staging buffer sized at open for one window per stream per step (host mel rows
     * included), so a step allocates nothing while the worker thread may be capturing; growth stays
     * only for a stream that consumes several row-less chunks in one step */
    const size_t fr = S * (size_t)b->nwin_max;
    if (grow_stage(g, (void **)&b->stage_span, &b->span_dev, &b->span_cap, fr * MEL_HOP + S * MEL_NFFT, 0, sizeof(float)) ||
        grow_stage(g, (void **)&b->stage_ftab, &b->ftab_dev, &b->ftab_cap, 2 * fr, 0, sizeof(int)) ||
        grow_stage(g, (void **)&b->stage_hrow, &b->hrow_dev, &b->hrow_cap, fr * MEL_NMEL, 0, sizeof(float)) ||
        grow_stage(g, (void **)&b->stage_hmap, &b->hmap_dev, &b->hmap_cap, fr, 0, sizeof(int)))
        return -1;
    return rc;
}

/* the device loop's GEMMs cover K = 2P <= 1280 and K = P <= 640 in one pass of their wavefronts,
   its decision scores at most 16 frames with at most 64 keys each; other shapes use the host-driven
   loop */
static int device_dec_ok(const nemoasr_batch_t *b) {
    return b->P <= 640 && b->P % 32 == 0 && b->J % 32 == 0 && b->W <= NK_ATTC_MAX_C && b->nkeys <= 64;
}

static void stream_clear(nemoasr_batch_t *b, int s) {
    bstream_t *x = &b->st[s];
    melfe_destroy(x->mel);
    int *tok = x->tok;
    size_t cap = x->cap_tok;
    float *pend = x->pending, *aq = x->aq;
    size_t pcap = x->pending_cap, acap = x->aq_cap;
    memset(x, 0, sizeof *x);
    x->tok = tok;
    x->cap_tok = cap;
    x->pending = pend;
    x->pending_cap = pcap;
    x->aq = aq;
    x->aq_cap = acap;
    x->mel = melfe_create();
    x->pos = b->conv_left; /* rows [0, conv_left) of every layer stay zero: the empty conv history */
    x->last_token = b->m->cfg.blank_id;
    if (b->dump) b->dj_n[s] = 0;
}

/* decoder state of a fresh stream on the device: no valid prediction, last token blank, slot set 0 */
static int bdec_state_reset(nemoasr_batch_t *b, int s) {
    NkBDecStream x;
    memset(&x, 0, sizeof x);
    x.last_token = b->m->cfg.blank_id;
    return gpu_upload(b->g, (NkBDecStream *)gpu_buf_dptr(b->bst) + s, &x, sizeof x);
}

/* device state of one stream back to that after open: zero LSTM states (and so zero hidden halves
 * of layer 0) and conv history */
static int stream_zero_device(nemoasr_batch_t *b, int s) {
    const size_t D = (size_t)b->m->cfg.d_model, P = (size_t)b->P;
    const size_t n = (size_t)b->conv_left * D > 8 * P ? (size_t)b->conv_left * D : 8 * P;
    float *z = calloc(n, sizeof(float));
    int rc = gpu_upload(b->g, (float *)gpu_buf_dptr(b->hc) + (size_t)s * 8 * P, z, 8 * P * sizeof(float));
    rc |= gpu_upload(b->g, (float *)gpu_buf_dptr(b->pre0) + (size_t)s * 8 * P, z, 8 * P * sizeof(float));
    for (int l = 0; l < b->m->cfg.n_layers; ++l)
        rc |= gpu_upload(b->g, (float *)gpu_buf_dptr(b->din) + (size_t)l * b->din_lstride + (size_t)s * b->cap_rows * D, z,
                         (size_t)b->conv_left * D * sizeof(float));
    free(z);
    return rc | bdec_state_reset(b, s);
}

nemoasr_batch_t *nemoasr_batch_open(const char *model_dir, const char *language, int latency_ms, int n_streams,
                                    char *err, size_t errlen) {
    if (errlen) err[0] = 0;
    const int right = right_for(latency_ms);
    if (right < 0) { snprintf(err, errlen, "latency must be one of 80, 160, 320, 560, 1120 ms"); return NULL; }
    if (n_streams < 1 || n_streams > 4096) { snprintf(err, errlen, "n_streams must be 1..4096"); return NULL; }
    nemoasr_batch_t *b = calloc(1, sizeof *b);
    b->m = model_load(model_dir, err, errlen);
    if (!b->m) { free(b); return NULL; }
    model_t *m = b->m;
    if (!model_right_context_trained(m, right)) {
        snprintf(err, errlen, "latency %d ms not trained for this checkpoint", latency_ms);
        nemoasr_batch_close(b);
        return NULL;
    }
    if (model_set_language(m, language ? language : "auto", err, errlen)) { nemoasr_batch_close(b); return NULL; }
    const model_cfg_t *c = &m->cfg;
    b->g = m->gpu;
    gpu_set_many_rows(b->g, 1);
    b->S = n_streams;
    b->latency_ms = latency_ms;
    b->right = right;
    b->chunk_frames = right + 1;
    b->chunk_mel = b->chunk_frames * c->subsampling;
    b->cmax = b->chunk_frames + 2; /* a final boundary window can yield up to chunk_frames + 2 rows */
    b->left = c->att_left;
    b->conv_left = c->conv_kernel - 1;
    b->Lmax = m->Lmax;
    /* compaction moves the live rows to the front; source and destination never overlap when
     * cap_rows >= 2 * left + cmax.  (Regions twice as deep, compacted half as often, measured no
     * faster at 64 and 256 streams.) */
    b->cap_rows = b->left + NK_CACHE_EPOCH_CHUNKS * b->cmax;
    if (b->cap_rows < 2 * b->left + 2 * b->cmax) b->cap_rows = 2 * b->left + 2 * b->cmax;
    b->P = c->pred_hidden;
    b->J = c->joint_hidden;
    b->V = c->num_classes;
    b->Vp = (b->V + 63) / 64 * 64;
    if (b->P % 8 || b->J % 32 || b->P * 2 % 32 || c->d_model % 64 || c->d_ff % 64) {
        snprintf(err, errlen, "batch: unsupported model sizes");
        nemoasr_batch_close(b);
        return NULL;
    }
    const size_t S = (size_t)n_streams, D = (size_t)c->d_model, CH = (size_t)c->sub_channels, F = (size_t)c->feat_in;
    const size_t fs = sizeof(float);
    b->nwin_max = MEL_CACHE + b->chunk_mel;
    b->T1max = sub_len(b->nwin_max);
    b->T2max = sub_len(b->T1max);
    b->T3max = sub_len(b->T2max);
    b->F1 = (int)F / 2 + 1;
    b->F2 = b->F1 / 2 + 1;
    b->F3 = b->F2 / 2 + 1;
    b->Mmax = n_streams * b->cmax;
    const size_t Mm = (size_t)b->Mmax;
    gpu_t *g = b->g;
    b->win = gpu_buf_alloc(g, S * (size_t)b->nwin_max * F * fs);
    b->c1 = gpu_buf_alloc(g, S * (size_t)b->T2max * b->F2 * CH * fs);
    b->c2 = gpu_buf_alloc(g, S * (size_t)b->T2max * b->F2 * CH * fs);
    b->c3 = gpu_buf_alloc(g, S * (size_t)b->T3max * b->F3 * CH * fs);
    b->c4 = gpu_buf_alloc(g, S * (size_t)b->T3max * b->F3 * CH * fs);
    b->flat = gpu_buf_alloc(g, S * (size_t)b->T3max * b->F3 * CH * fs);
    b->pre_out = gpu_buf_alloc(g, S * (size_t)b->T3max * D * fs);
    /* the residual updates' partial rows (at most one part per 1024 of K, the feed-forward width)
     * live in the context's scratch: sized now, before any step is captured */
    {
        size_t parts = (size_t)c->d_ff / 1024;
        parts = parts < 2 ? 2 : parts > 8 ? 8 : parts;
        if (!gpu_scratch_ws(g, parts * Mm * D)) {
            snprintf(err, errlen, "batch: cannot allocate the residual-update scratch");
            nemoasr_batch_close(b);
            return NULL;
        }
    }
    b->h = gpu_buf_alloc(g, Mm * D * fs);
    b->tmp = gpu_buf_alloc(g, Mm * D * fs);
    b->lnb = gpu_buf_alloc(g, Mm * D * fs);
    b->ff = gpu_buf_alloc(g, Mm * (size_t)c->d_ff * fs);
    b->att = gpu_buf_alloc(g, Mm * D * fs);
    b->y = gpu_buf_alloc(g, Mm * D * fs);
    b->ph = gpu_buf_alloc(g, Mm * (size_t)c->prompt_hidden * fs);
    b->prompted = gpu_buf_alloc(g, Mm * D * fs);
    b->joint_enc = gpu_buf_alloc(g, Mm * (size_t)b->J * fs);
    b->kv_lstride = S * (size_t)b->cap_rows * 3 * D;
    b->din_lstride = S * (size_t)b->cap_rows * D;
    b->kv = gpu_buf_alloc(g, (size_t)c->n_layers * b->kv_lstride * fs);
    b->din = gpu_buf_alloc(g, (size_t)c->n_layers * b->din_lstride * fs);
    b->etab = gpu_buf_alloc(g, (6 * Mm + 4 * S) * sizeof(int));
    b->stage_win = gpu_host_alloc(g, S * (size_t)b->nwin_max * F * fs);
    b->stage_tab = gpu_host_alloc(g, (6 * Mm + 4 * S) * sizeof(int));
    b->wtmp = malloc((size_t)b->nwin_max * F * fs);
    const size_t P = (size_t)b->P, J = (size_t)b->J, R = S * DEC_WIN;
    b->hc = gpu_buf_alloc(g, S * 8 * P * fs);
    b->lin = gpu_buf_alloc(g, S * 2 * P * fs);
    b->gates = gpu_buf_alloc(g, S * 4 * P * fs);
    b->hout = gpu_buf_alloc(g, S * P * fs);
    b->hout2 = gpu_buf_alloc(g, S * P * fs);
    b->pred = gpu_buf_alloc(g, S * J * fs);
    b->jin = gpu_buf_alloc(g, R * J * fs);
    b->logits = gpu_buf_alloc(g, R * (size_t)b->Vp * fs);
    b->amax = gpu_buf_alloc(g, 2 * R * sizeof(int));
    b->dtab = gpu_buf_alloc(g, (10 * S + 2 * R) * sizeof(int));
    b->stage_dtab = gpu_host_alloc(g, (10 * S + 2 * R) * sizeof(int));
    b->stage_amax = gpu_host_alloc(g, 2 * R * sizeof(int));
    b->W = b->cmax;
    b->tok_ld = c->max_symbols * b->cmax + 16;
    b->bst = gpu_buf_alloc(g, S * sizeof(NkBDecStream));
    b->nkeys = 2 * (b->Vp / 64);
    b->keys = gpu_buf_alloc(g, S * (size_t)b->W * b->nkeys * sizeof(unsigned long long));
    b->bsetup = gpu_buf_alloc(g, 2 * S * sizeof(int));
    b->brows = gpu_buf_alloc(g, S * sizeof(NkBDecRow));
    b->bcnt = gpu_buf_alloc(g, 2 * sizeof(int));
    b->btok = gpu_buf_alloc(g, S * (size_t)b->tok_ld * sizeof(int));
    b->lin1 = gpu_buf_alloc(g, S * 2 * P * fs);
    b->pre0 = gpu_buf_alloc(g, S * 2 * 4 * P * fs); /* zero: the hidden half of layer 0 at h0 = 0 */
    b->stage_bst = gpu_host_alloc(g, S * sizeof(NkBDecStream));
    b->stage_bsetup = gpu_host_alloc(g, (2 * S + 2) * sizeof(int));
    b->stage_btok = gpu_host_alloc(g, S * (size_t)b->tok_ld * sizeof(int));
    if (!b->win || !b->kv || !b->din || !b->ff || !b->stage_win || !b->stage_dtab || !b->btok || !b->stage_btok) {
        snprintf(err, errlen, "batch: out of memory for %d streams", n_streams);
        nemoasr_batch_close(b);
        return NULL;
    }
    if (build_decoder_weights(b)) {
        snprintf(err, errlen, "batch: decoder weight setup failed: %s", gpu_last_error(g));
        nemoasr_batch_close(b);
        return NULL;
    }
    b->st = calloc(S, sizeof *b->st);
    b->order = malloc(S * sizeof(int));
    b->gid = malloc(S * sizeof(int));
    b->g_nwin = malloc(S * sizeof(int));
    b->g_cnt = malloc(S * sizeof(int));
    b->g_woff = malloc(S * sizeof(int));
    b->g_poff = malloc(S * sizeof(int));
    b->g_fill = malloc(S * sizeof(int));
    b->ord = malloc(S * sizeof(int));
    for (int s = 0; s < n_streams; ++s) stream_clear(b, s);
    for (int s = 0; s < n_streams; ++s)
        if (bdec_state_reset(b, s)) {
            snprintf(err, errlen, "batch: decoder state upload failed");
            nemoasr_batch_close(b);
            return NULL;
        }
    b->device_dec = device_dec_ok(b);
    if (b->device_dec) {
        /* the greedy loop's own GPU context and worker thread */
        b->gd = gpu_create(NULL, err, errlen);
        if (b->gd) gpu_set_many_rows(b->gd, 1);
        b->jdec[0] = gpu_buf_alloc(g, Mm * (size_t)b->J * fs);
        b->jdec[1] = gpu_buf_alloc(g, Mm * (size_t)b->J * fs);
        b->dorder = malloc(S * sizeof(int));
        b->dc = malloc(S * sizeof(int));
        b->drow0 = malloc(S * sizeof(int));
        if (!b->gd || !b->jdec[0] || !b->jdec[1] || !b->dorder || !b->dc || !b->drow0 || dec_start(b)) {
            if (!err[0]) snprintf(err, errlen, "batch: decoder context setup failed");
            nemoasr_batch_close(b);
            return NULL;
        }
    }
    if (mel_gpu_setup(b)) {
        snprintf(err, errlen, "batch: log-mel front end setup failed: %s", gpu_last_error(g));
        nemoasr_batch_close(b);
        return NULL;
    }
    b->fe_list = malloc(S * sizeof(int));
    pool_start(&b->pool, b);
    b->use_graphs = 1;
    /* whole-chunk attention when every window fits its LDS tables */
    b->chunk_attn = b->Lmax <= NK_ATTC_MAX_L && b->cmax <= NK_ATTC_MAX_C;
    return b;
}

void nemoasr_batch_close(nemoasr_batch_t *b) {
    if (!b) return;
    dec_stop(b);
    pool_stop(&b->pool);
    free(b->fe_list);
    drop_graphs(b);
    gpu_buf_t *bufs[] = { b->win, b->c1, b->c2, b->c3, b->c4, b->flat, b->pre_out, b->h, b->tmp, b->lnb,
                          b->ff, b->att, b->y, b->ph, b->prompted, b->joint_enc, b->kv, b->din, b->etab, b->wcat[0],
                          b->wcat[1], b->wout, b->bout, b->hc, b->lin, b->gates, b->hout, b->hout2, b->pred,
                          b->jin, b->logits, b->amax, b->dtab, b->bst, b->bsetup, b->btok, b->lin1, b->pre0, b->tx,
                          b->wcati[0], b->wcati[1], b->bi[0], b->bi[1], b->keys, b->ring, b->meltab, b->span_dev,
                          b->ftab_dev, b->wmap_dev, b->hrow_dev, b->hmap_dev, b->jdec[0], b->jdec[1], b->brows,
                          b->bcnt };
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs; ++i) gpu_buf_free(bufs[i]);
    gpu_host_free(b->stage_win);
    gpu_host_free(b->stage_tab);
    gpu_host_free(b->stage_span);
    gpu_host_free(b->stage_hrow);
    gpu_host_free(b->stage_ftab);
    gpu_host_free(b->stage_wmap);
    gpu_host_free(b->stage_hmap);
    gpu_host_free(b->stage_dtab);
    gpu_host_free(b->stage_amax);
    gpu_host_free(b->stage_bst);
    gpu_host_free(b->stage_bsetup);
    gpu_host_free(b->stage_btok);
    free(b->dorder);
    free(b->dc);
    free(b->drow0);
    for (int i = 0; i < 2; ++i)
        for (int k = 0; k < 6; ++k) gpu_graph_free(b->dgraph[i][k]);
    if (b->st)
        for (int s = 0; s < b->S; ++s) {
            melfe_destroy(b->st[s].mel);
            free(b->st[s].aq);
            free(b->st[s].pending);
            free(b->st[s].tok);
        }
    if (b->dj) {
        for (int s = 0; s < b->S; ++s) free(b->dj[s]);
        free(b->dj);
        free(b->dj_n);
        free(b->dj_cap);
    }
    free(b->st);
    free(b->order);
    free(b->gid);
    free(b->g_nwin);
    free(b->g_cnt);
    free(b->g_woff);
    free(b->g_poff);
    free(b->g_fill);
    free(b->ord);
    free(b->wtmp);
    free(b->step_ms);
    gpu_destroy(b->gd);
    model_free(b->m);
    free(b);
}

static int check_stream(const nemoasr_batch_t *b, int s, char *err, size_t errlen) {
    if (s < 0 || s >= b->S) { snprintf(err, errlen, "stream %d out of range (0..%d)", s, b->S - 1); return -1; }
    return 0;
}

static void queue_mel(bstream_t *x, const float *mel, size_t nframes) {
    if (!nframes) return;
    if (x->pending_n + nframes > x->pending_cap) {
        x->pending_cap = (x->pending_n + nframes) * 2;
        x->pending = realloc(x->pending, x->pending_cap * MEL_NMEL * sizeof(float));
    }
    memcpy(x->pending + x->pending_n * MEL_NMEL, mel, nframes * MEL_NMEL * sizeof(float));
    x->pending_n += nframes;
}

/* log-mel of the audio queued for one stream (src/nemoasr.c:134-160 without resampling: audio
 * is pushed at 16 kHz); a final push with no samples and an empty front end flushes nothing
 * (src/nemoasr.c:146) */
static void front_end(const nemoasr_batch_t *b, bstream_t *x) {
    if (!x->aq_n && !x->fe_final) return;
    if (!(x->fe_final && x->aq_n == 0 && melfe_samples(x->mel) == 0)) {
        if (b->gpu_fe) {
            /* samples only: the frames are computed on the GPU when a window takes them */
            x->pending_n = melfe_append(x->mel, x->aq, x->aq_n, x->fe_final);
        } else {
            const float *frames;
            size_t nf;
            melfe_push(x->mel, x->aq, x->aq_n, x->fe_final, &frames, &nf);
            queue_mel(x, frames, nf);
        }
    }
    x->aq_n = 0;
    if (x->fe_final) {
        x->fe_final = 0;
        x->final = 1;
    }
}

static void *pool_main(void *arg) {
    pool_t *p = arg;
    unsigned seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        while (!p->quit && p->gen == seen) pthread_cond_wait(&p->go, &p->mu);
        if (p->quit) {
            pthread_mutex_unlock(&p->mu);
            return NULL;
        }
        seen = p->gen;
        pthread_mutex_unlock(&p->mu);
        for (;;) {
            const int i = __atomic_fetch_add(&p->next, 1, __ATOMIC_RELAXED);
            if (i >= p->count) break;
            front_end(p->b, &p->b->st[p->list[i]]);
        }
        pthread_mutex_lock(&p->mu);
        if (--p->busy == 0) pthread_cond_signal(&p->done);
        pthread_mutex_unlock(&p->mu);
    }
}

static void pool_start(pool_t *p, struct nemoasr_batch *b) {
    long nc = sysconf(_SC_NPROCESSORS_ONLN);
    const char *env = getenv("NEMOASR_THREADS");
    if (env && atoi(env) > 0) nc = atoi(env);
    int n = (int)(nc < 1 ? 1 : nc) - 1; /* the calling thread works too */
    if (n > POOL_MAX) n = POOL_MAX;
    if (n > b->S - 1) n = b->S - 1;
    p->b = b;
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->go, NULL);
    pthread_cond_init(&p->done, NULL);
    p->started = 1;
    for (int i = 0; i < n; ++i) {
        if (pthread_create(&p->th[i], NULL, pool_main, p)) break;
        p->n++;
    }
}

static void pool_stop(pool_t *p) {
    if (!p->started) return;
    pthread_mutex_lock(&p->mu);
    p->quit = 1;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->n; ++i) pthread_join(p->th[i], NULL);
    pthread_mutex_destroy(&p->mu);
    pthread_cond_destroy(&p->go);
    pthread_cond_destroy(&p->done);
    p->started = 0;
}

/* front end of every stream with queued audio, spread over the pool */
static void front_end_all(nemoasr_batch_t *b) {
    int count = 0;
    for (int s = 0; s < b->S; ++s)
        if (b->st[s].aq_n || b->st[s].fe_final) b->fe_list[count++] = s;
    if (!count) return;
    pool_t *p = &b->pool;
    if (count == 1 || p->n == 0) {
        for (int i = 0; i < count; ++i) front_end(b, &b->st[b->fe_list[i]]);
        return;
    }
    pthread_mutex_lock(&p->mu);
    p->list = b->fe_list;
    p->count = count;
    p->next = 0;
    p->busy = p->n;
    p->gen++;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    for (;;) {
        const int i = __atomic_fetch_add(&p->next, 1, __ATOMIC_RELAXED);
        if (i >= count) break;
        front_end(b, &b->st[b->fe_list[i]]);
    }
    pthread_mutex_lock(&p->mu);
    while (p->busy > 0) pthread_cond_wait(&p->done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

int nemoasr_batch_push_mel(nemoasr_batch_t *b, int stream, const float *mel, size_t nframes, int final, char *err,
                           size_t errlen) {
    if (errlen) err[0] = 0;
    if (check_stream(b, stream, err, errlen)) return -1;
    bstream_t *x = &b->st[stream];
    if (x->ended) { snprintf(err, errlen, "stream %d already ended", stream); return -1; }
    if (b->gpu_fe && x->src == 1) {
        snprintf(err, errlen, "stream %d: audio and mel input cannot be mixed before a reset", stream);
        return -1;
    }
    front_end(b, x); /* audio queued before these frames goes first */
    queue_mel(x, mel, nframes);
    if (nframes || final) x->src = 2;
    if (final) x->ended = x->final = 1;
    return 0;
}

/* audio is only queued here; its log-mel is computed by the next step, for all streams at once */
int nemoasr_batch_push(nemoasr_batch_t *b, int stream, const float *samples, size_t n, int final, char *err,
                       size_t errlen) {
    if (errlen) err[0] = 0;
    if (check_stream(b, stream, err, errlen)) return -1;
    bstream_t *x = &b->st[stream];
    if (x->ended) { snprintf(err, errlen, "stream %d already ended", stream); return -1; }
    if (b->gpu_fe && x->src == 2) {
        snprintf(err, errlen, "stream %d: audio and mel input cannot be mixed before a reset", stream);
        return -1;
    }
    x->src = 1;
    if (n) {
        if (x->aq_n + n > x->aq_cap) {
            x->aq_cap = (x->aq_n + n) * 2;
            x->aq = realloc(x->aq, x->aq_cap * sizeof(float));
        }
        memcpy(x->aq + x->aq_n, samples, n * sizeof(float));
        x->aq_n += n;
    }
    if (final) x->ended = x->fe_final = 1;
    return 0;
}

/* Window of the planned chunk (mel cache ++ the rows taken); advance the stream's mel bookkeeping
 * exactly as a single-stream encoder step does.  Host front end: the window's rows go into dst.
 * GPU front end: the frames taken are staged (their sample spans for mel_frames, or the host's mel
 * rows for a scatter into the ring) and, when wrow >= 0, the window's ring rows go into the gather
 * map from row wrow on. */
static int take_window(nemoasr_batch_t *b, int s, float *dst, long wrow, char *err, size_t errlen) {
    bstream_t *x = &b->st[s];
    const enc_plan_t *p = &x->plan;
    const size_t rowb = MEL_NMEL * sizeof(float), take = (size_t)p->take;
    if (b->gpu_fe) {
        gpu_t *g = b->g;
        const size_t f0 = x->fr_taken - (size_t)x->cache_before;
        if (x->fr_taken + take - x->fr_lo > MEL_RING) {
            snprintf(err, errlen, "stream %d: more than %d log-mel frames in one step", s, MEL_RING);
            return -1;
        }
        if (wrow >= 0)
            for (int i = 0; i < p->nwin; ++i) b->stage_wmap[wrow + i] = s * MEL_RING + (int)((f0 + (size_t)i) % MEL_RING);
        if (take && x->src == 2) {
            const size_t hr = b->hrow_n / MEL_NMEL;
            if (grow_stage(g, (void **)&b->stage_hrow, &b->hrow_dev, &b->hrow_cap, b->hrow_n + take * MEL_NMEL, b->hrow_n,
                           sizeof(float)) ||
                grow_stage(g, (void **)&b->stage_hmap, &b->hmap_dev, &b->hmap_cap, hr + take, hr, sizeof(int))) {
                snprintf(err, errlen, "batch: out of memory for staged mel rows");
                return -1;
            }
            memcpy(b->stage_hrow + b->hrow_n, x->pending, take * rowb);
            for (size_t t = 0; t < take; ++t) b->stage_hmap[hr + t] = s * MEL_RING + (int)((x->fr_taken + t) % MEL_RING);
            b->hrow_n += take * MEL_NMEL;
            memmove(x->pending, x->pending + take * MEL_NMEL, (x->pending_n - take) * rowb);
        } else if (take) {
            const size_t len = melfe_span_len(take);
            if (grow_stage(g, (void **)&b->stage_span, &b->span_dev, &b->span_cap, b->span_n + len, b->span_n,
                           sizeof(float)) ||
                grow_stage(g, (void **)&b->stage_ftab, &b->ftab_dev, &b->ftab_cap, b->ftab_n + 2 * take, b->ftab_n,
                           sizeof(int))) {
                snprintf(err, errlen, "batch: out of memory for staged audio");
                return -1;
            }
            if (melfe_take(x->mel, b->stage_span + b->span_n, take) != take) {
                snprintf(err, errlen, "stream %d: front end has fewer frames than planned", s);
                return -1;
            }
            for (size_t t = 0; t < take; ++t) {
                b->stage_ftab[b->ftab_n + 2 * t] = (int)(b->span_n + t * MEL_HOP);
                b->stage_ftab[b->ftab_n + 2 * t + 1] = s * MEL_RING + (int)((x->fr_taken + t) % MEL_RING);
            }
            b->span_n += len;
            b->ftab_n += 2 * take;
        }
        x->fr_taken += take;
    } else {
        memcpy(dst, x->mel_cache, (size_t)x->cache_before * rowb);
        memcpy(dst + (size_t)x->cache_before * MEL_NMEL, x->pending, take * rowb);
        memcpy(x->mel_cache, dst + (size_t)(p->nwin - x->book.mel_cache_n) * MEL_NMEL, (size_t)x->book.mel_cache_n * rowb);
        memmove(x->pending, x->pending + take * MEL_NMEL, (x->pending_n - take) * rowb);
    }
    x->pending_n = x->book.pending_n;
    x->consumed = x->book.consumed;
    x->emitted = x->book.emitted;
    x->mel_cache_n = x->book.mel_cache_n;
    return 0;
}

/* The next chunk of one stream that yields rows (chunks that yield none are consumed on the way).
 * Returns 1 if the stream consumed input. */
static int plan_stream(nemoasr_batch_t *b, bstream_t *x, char *err, size_t errlen) {
    int ran = 0;
    x->c = 0;
    for (;;) {
        x->book = (enc_book_t){ x->pending_n, x->consumed, x->emitted, x->mel_cache_n, x->closed };
        x->cache_before = x->mel_cache_n;
        x->plan = enc_plan_step(&x->book, x->final, b->chunk_mel, b->m->cfg.subsampling, MEL_CACHE);
        x->closed = x->book.closed;
        if (!x->plan.ran) return ran;
        ran = 1;
        if (x->plan.c <= 0) {
            if (take_window(b, (int)(x - b->st), b->wtmp, -1, err, errlen)) return -1;
            continue;
        }
        x->c = x->plan.c;
        x->nwin = x->plan.nwin;
        x->lo = x->plan.lo;
        return 1;
    }
}

/* subsampling of `cnt` windows of nwin rows (back to back in win) into pre_out rows:
 * src/encoder.c:120-142 */
static void launch_pre_encode(nemoasr_batch_t *b, const float *win, int nwin, int cnt, float *pre_out) {
    model_t *m = b->m;
    gpu_t *g = b->g;
    const uint32_t CH = (uint32_t)m->cfg.sub_channels, F = (uint32_t)m->cfg.feat_in, n = (uint32_t)cnt;
    const uint32_t T1 = (uint32_t)sub_len(nwin), F1 = F / 2 + 1, T2 = T1 / 2 + 1, F2 = F1 / 2 + 1, T3 = T2 / 2 + 1,
                   F3 = F2 / 2 + 1;
    float *c1 = gpu_buf_dptr(b->c1), *c2 = gpu_buf_dptr(b->c2), *c3 = gpu_buf_dptr(b->c3);
    float *c4 = gpu_buf_dptr(b->c4), *flat = gpu_buf_dptr(b->flat);
    /* conv 0 + ReLU and the first depthwise conv in one launch (conv 0's output is not stored) */
    nk_conv2d_c1_dw_s2_b(g, win, m->conv0_w, m->conv0_b, m->conv2_w, m->conv2_b, c1, (uint32_t)nwin, F, T1, F1, T2,
                         F2, CH, n);
    nk_gemm(g, c1, CH, m->conv3_w, CH, m->conv3_b, c2, CH, n * T2 * F2, CH, CH, NK_ACT_RELU, 0, 1.0f);
    nk_dwconv2d_s2_b(g, c2, m->conv5_w, m->conv5_b, c3, T2, F2, T3, F3, CH, n);
    nk_gemm(g, c3, CH, m->conv6_w, CH, m->conv6_b, c4, CH, n * T3 * F3, CH, CH, NK_ACT_RELU, 0, 1.0f);
    nk_flatten_cf_b(g, c4, flat, T3, F3, CH, n);
    const uint32_t D = (uint32_t)m->cfg.d_model, K = CH * F3;
    nk_gemm(g, flat, K, m->pre_out_w, K, m->pre_out_b, pre_out, D, n * T3, D, K, NK_ACT_NONE, 0, 1.0f);
}

/* conformer blocks + prompt + joint projection on the M rows in h (src/encoder.c:144-197).
 * The order of operations and the LayerNorm placement are those of the single-stream encoder;
 * crow maps every row to its stream's cache row, rows is the attention/conv row table.
 * Activations that only feed a GEMM (LayerNorm outputs, the feed-forward hidden rows, attention
 * and conv module outputs, the prompt's hidden rows) are kept as split rows (nk_gemm_split): their
 * producers write bf16 hi / lo once, in the buffers that hold the f32 rows otherwise (a split row
 * of K values takes the bytes of K floats).  The residual stream, the caches and the rows that are
 * dumped stay f32.  Each residual update (FF down, out_proj, pw2) is left pending (nk_gemm_resid)
 * and applied by the LayerNorm that follows it, which reads the residual rows anyway. */
static void launch_blocks(nemoasr_batch_t *b, uint32_t M, const int *crow, const int *rows, const int *chunks,
                          uint32_t nchunks) {
    model_t *m = b->m;
    gpu_t *g = b->g;
    const model_cfg_t *cf = &m->cfg;
    const uint32_t D = (uint32_t)cf->d_model, FF = (uint32_t)cf->d_ff, H = (uint32_t)cf->n_heads,
                   dh = (uint32_t)cf->head_dim, nl = (uint32_t)cf->n_layers, taps = (uint32_t)cf->conv_kernel;
    const float eps = cf->ln_eps, scale = 1.0f / sqrtf((float)dh);
    float *R[2] = { gpu_buf_dptr(b->h), gpu_buf_dptr(b->tmp) };
    uint16_t *lns = gpu_buf_dptr(b->lnb), *ffs = gpu_buf_dptr(b->ff), *ys = gpu_buf_dptr(b->y);
    float *att = gpu_buf_dptr(b->att);
    uint16_t *atts = (uint16_t *)att;
    int cur = 0;
    nk_resid_t pend = { 0 }; /* the residual update the next LayerNorm applies */
    for (uint32_t l = 0; l < nl; ++l) {
        const layer_dev_t *W = &m->L[l];
        float *kv = (float *)gpu_buf_dptr(b->kv) + (size_t)l * b->kv_lstride;
        float *din = (float *)gpu_buf_dptr(b->din) + (size_t)l * b->din_lstride;
        /* FF1 half step: LN (paired with the previous block's output norm), up + SiLU, down */
        if (l == 0) {
            nk_layernorm2_split(g, R[0], NULL, W->ln_ff1_g, W->ln_ff1_b, NULL, NULL, NULL, lns, M, D, eps);
        } else {
            const layer_dev_t *Wp = &m->L[l - 1];
            const int prev = cur;
            cur ^= 1;
            nk_layernorm2_split(g, R[prev], &pend, Wp->ln_out_g, Wp->ln_out_b, W->ln_ff1_g, W->ln_ff1_b, R[cur], lns, M,
                                D, eps);
        }
        float *res = R[cur];
        nk_gemm_split(g, NULL, lns, 2 * D, W->ff1_w1, D, NULL, NULL, ffs, 2 * FF, NULL, M, FF, D, NK_ACT_SILU, 0, 1.0f);
        nk_gemm_resid(g, NULL, ffs, 2 * FF, W->ff1_w2, FF, res, D, M, D, FF, 0.5f, &pend);
        /* attention: LN, QKV into the cache rows, attention, out_proj into the residual */
        nk_layernorm2_split(g, res, &pend, W->ln_att_g, W->ln_att_b, NULL, NULL, NULL, lns, M, D, eps);
        nk_gemm_split(g, NULL, lns, 2 * D, W->wqkv, D, NULL, kv, NULL, 3 * D, crow, M, 3 * D, D, NK_ACT_NONE, 0, 1.0f);
        if (b->chunk_attn) {
            nk_attention_rel_chunks_split(g, kv, 3 * D, chunks, nchunks, W->ptab, W->bias_u, W->bias_v, atts,
                                          (uint32_t)b->Lmax, H, dh, D, scale);
            nk_gemm_resid(g, NULL, atts, 2 * D, W->wo, D, res, D, M, D, D, 1.0f, &pend);
        } else {
            nk_attention_rel_rows(g, kv, 3 * D, rows, M, W->ptab, W->bias_u, W->bias_v, att, (uint32_t)b->Lmax, H, dh, D,
                                  scale);
            nk_gemm_resid(g, att, NULL, D, W->wo, D, res, D, M, D, D, 1.0f, &pend);
        }
        /* conv module: LN, pw1 + GLU into the conv cache rows, depthwise conv + LN + SiLU, pw2 */
        nk_layernorm2_split(g, res, &pend, W->ln_conv_g, W->ln_conv_b, NULL, NULL, NULL, lns, M, D, eps);
        nk_gemm_split(g, NULL, lns, 2 * D, W->pw1, D, NULL, din, NULL, D, crow, M, 2 * D, D, NK_ACT_GLU, 0, 1.0f);
        nk_dwconv_ln_silu_rows_split(g, din, rows, M, W->dw_w, W->bn_g, W->bn_b, NULL, ys, D, taps, eps);
        nk_gemm_resid(g, NULL, ys, 2 * D, W->pw2, D, res, D, M, D, D, 1.0f, &pend);
        /* FF2 half step */
        nk_layernorm2_split(g, res, &pend, W->ln_ff2_g, W->ln_ff2_b, NULL, NULL, NULL, lns, M, D, eps);
        nk_gemm_split(g, NULL, lns, 2 * D, W->ff2_w1, D, NULL, NULL, ffs, 2 * FF, NULL, M, FF, D, NK_ACT_SILU, 0, 1.0f);
        nk_gemm_resid(g, NULL, ffs, 2 * FF, W->ff2_w2, FF, res, D, M, D, FF, 0.5f, &pend);
    }
    /* last output norm, prompt (W0 + ReLU, W2) and joint.enc (src/encoder.c:189-194) */
    const layer_dev_t *Wl = &m->L[nl - 1];
    const uint32_t PH = (uint32_t)cf->prompt_hidden, NP = (uint32_t)cf->num_prompts, JH = (uint32_t)b->J;
    uint16_t *phs = gpu_buf_dptr(b->ph);
    float *pr = gpu_buf_dptr(b->prompted);
    nk_layernorm2_split(g, R[cur], &pend, Wl->ln_out_g, Wl->ln_out_b, NULL, NULL, NULL, lns, M, D, eps);
    nk_gemm_split(g, NULL, lns, 2 * D, m->prompt_w0, D + NP, m->prompt_b0_eff, NULL, phs, 2 * PH, NULL, M, PH, D,
                  NK_ACT_RELU, 0, 1.0f);
    nk_gemm_split(g, NULL, phs, 2 * PH, m->prompt_w2, PH, m->prompt_b2, pr, NULL, D, NULL, M, D, PH, NK_ACT_NONE, 0, 1.0f);
    nk_gemm(g, pr, D, m->joint_enc_w, D, m->joint_enc_b, gpu_buf_dptr(b->joint_enc), JH, M, JH, D, NK_ACT_NONE, 0, 1.0f);
}

static void launch_encoder(nemoasr_batch_t *b, int M, int nact) {
    const size_t F = (size_t)b->m->cfg.feat_in, D = (size_t)b->m->cfg.d_model;
    const int *tab = gpu_buf_dptr(b->etab);
    for (int k = 0; k < b->ng; ++k)
        launch_pre_encode(b, (const float *)gpu_buf_dptr(b->win) + (size_t)b->g_woff[k] * F, b->g_nwin[k], b->g_cnt[k],
                          (float *)gpu_buf_dptr(b->pre_out) + (size_t)b->g_poff[k] * D);
    nk_gather_rows(b->g, gpu_buf_dptr(b->pre_out), (uint32_t)D, tab + 5 * M, gpu_buf_dptr(b->h), (uint32_t)D, (uint32_t)M,
                   (uint32_t)D);
    launch_blocks(b, (uint32_t)M, tab, tab + M, tab + 6 * M, (uint32_t)nact);
}

/* move a stream's live cache rows to the front of its region, every layer (src/encoder.c:199-211) */
static void compact_stream(nemoasr_batch_t *b, int s) {
    bstream_t *x = &b->st[s];
    const uint32_t D = (uint32_t)b->m->cfg.d_model, nl = (uint32_t)b->m->cfg.n_layers;
    float *kv = (float *)gpu_buf_dptr(b->kv) + (size_t)s * b->cap_rows * 3 * D;
    float *din = (float *)gpu_buf_dptr(b->din) + (size_t)s * b->cap_rows * D;
    if (x->cache_len > 0)
        nk_compact(b->g, kv, b->kv_lstride, nl, (uint32_t)x->cache_len, 3 * D, (uint32_t)(x->pos - x->cache_len), 0);
    nk_compact(b->g, din, b->din_lstride, nl, (uint32_t)b->conv_left, D, (uint32_t)(x->pos - b->conv_left),
               (uint32_t)(x->cache_len - b->conv_left));
    x->pos = x->cache_len;
}

/* One batched encoder step.  Returns the number of streams that consumed input; *M_out = rows. */
static int encoder_batch_step(nemoasr_batch_t *b, int *M_out, char *err, size_t errlen) {
    const size_t F = (size_t)b->m->cfg.feat_in;
    int consumed = 0, nact = 0;
    const double tf = now_ms();
    front_end_all(b);
    b->stats.frontend_ms += now_ms() - tf;
    b->span_n = b->ftab_n = b->hrow_n = 0;
    for (int s = 0; s < b->S; ++s) {
        bstream_t *x = &b->st[s];
        x->fr_lo = x->fr_taken - (size_t)x->mel_cache_n;
        const int r = plan_stream(b, x, err, errlen);
        if (r < 0) return -1;
        consumed += r;
        if (x->c > 0) b->order[nact++] = s;
    }
    *M_out = 0;
    if (!nact) return consumed;
    /* windows grouped by length, in order of first appearance; streams keep their order inside a
     * group and rows follow the group order */
    b->ng = 0;
    for (int i = 0; i < nact; ++i) {
        const bstream_t *x = &b->st[b->order[i]];
        int k = 0;
        while (k < b->ng && b->g_nwin[k] != x->nwin) ++k;
        if (k == b->ng) { b->g_nwin[k] = x->nwin; b->g_cnt[k] = 0; b->ng++; }
        b->gid[i] = k;
        b->g_cnt[k]++;
    }
    int woff = 0, poff = 0;
    for (int k = 0; k < b->ng; ++k) {
        b->g_woff[k] = woff;
        b->g_poff[k] = poff;
        woff += b->g_cnt[k] * b->g_nwin[k];
        poff += b->g_cnt[k] * sub_len(sub_len(sub_len(b->g_nwin[k])));
    }
    /* row order: group by group */
    int M = 0;
    int *fill = b->g_fill, *ord = b->ord;
    memset(fill, 0, (size_t)b->ng * sizeof(int));
    int n2 = 0;
    for (int k = 0; k < b->ng; ++k)
        for (int i = 0; i < nact; ++i)
            if (b->gid[i] == k) ord[n2++] = b->order[i];
    memcpy(b->order, ord, (size_t)nact * sizeof(int));
    gpu_t *g = b->g;
    gpu_begin(g);
    int *crow = b->stage_tab;
    for (int i = 0; i < nact; ++i) {
        const int s = b->order[i];
        bstream_t *x = &b->st[s];
        int k = 0;
        while (b->g_nwin[k] != x->nwin) ++k;
        const int j = fill[k]++;
        const int T3 = sub_len(sub_len(sub_len(x->nwin)));
        x->gk = k;
        x->gj = j;
        const size_t wr = (size_t)b->g_woff[k] + (size_t)j * x->nwin;
        if (take_window(b, s, b->stage_win + wr * F, (long)wr, err, errlen)) {
            gpu_end(g, NULL, 0);
            return -1;
        }
        if (x->pos + x->c > b->cap_rows) compact_stream(b, s);
        const int L = x->cache_len + x->c;
        if (L > b->Lmax || x->pos < x->cache_len || x->pos < b->conv_left || x->pos + x->c > b->cap_rows ||
            x->lo + x->c > T3) {
            snprintf(err, errlen, "stream %d: cache bookkeeping out of range (pos %d, cache %d, c %d)", s, x->pos,
                     x->cache_len, x->c);
            gpu_end(g, NULL, 0);
            return -1;
        }
        x->row0 = M;
        M += x->c;
    }
    if (M > b->Mmax) {
        snprintf(err, errlen, "batch: %d rows exceed %d", M, b->Mmax);
        gpu_end(g, NULL, 0);
        return -1;
    }
    /* tables: crow[M], rows[4M], gather map[M], chunks[4 nact] */
    int *rows = crow + M, *gmap = crow + 5 * M, *chunks = crow + 6 * M;
    for (int i = 0; i < nact; ++i) {
        const int s = b->order[i];
        const bstream_t *x = &b->st[s];
        const int k = x->gk, j = x->gj;
        const int T3 = sub_len(sub_len(sub_len(x->nwin)));
        for (int r = 0; r < x->c; ++r) {
            const int m = x->row0 + r;
            crow[m] = s * b->cap_rows + x->pos + r;
            rows[4 * m] = crow[m];
            rows[4 * m + 1] = r;
            rows[4 * m + 2] = x->c;
            rows[4 * m + 3] = x->cache_len;
            gmap[m] = b->g_poff[k] + j * T3 + x->lo + r;
        }
        chunks[4 * i] = s * b->cap_rows + x->pos;
        chunks[4 * i + 1] = x->row0;
        chunks[4 * i + 2] = x->c;
        chunks[4 * i + 3] = x->cache_len;
    }
    if (b->gpu_fe) {
        /* log-mel of the frames taken into the rings, the host's mel rows scattered into them, then
           every window gathered from its stream's ring */
        const char *t = gpu_buf_dptr(b->meltab);
        float *ring = gpu_buf_dptr(b->ring);
        const size_t nf = b->ftab_n / 2, nh = b->hrow_n / MEL_NMEL;
        if (nf) {
            gpu_upload_async(g, gpu_buf_dptr(b->span_dev), b->stage_span, b->span_n * sizeof(float));
            gpu_upload_async(g, gpu_buf_dptr(b->ftab_dev), b->stage_ftab, b->ftab_n * sizeof(int));
            nk_mel_frames(g, gpu_buf_dptr(b->span_dev), gpu_buf_dptr(b->ftab_dev), (uint32_t)nf,
                          (const float *)(t + MT_WIN), (const float *)(t + MT_FB), (const int *)(t + MT_LO),
                          (const int *)(t + MT_HI), (const double *)(t + MT_TWR), (const double *)(t + MT_TWI),
                          (const uint16_t *)(t + MT_REV), ring);
        }
        if (nh) {
            gpu_upload_async(g, gpu_buf_dptr(b->hrow_dev), b->stage_hrow, b->hrow_n * sizeof(float));
            gpu_upload_async(g, gpu_buf_dptr(b->hmap_dev), b->stage_hmap, nh * sizeof(int));
            nk_scatter_rows(g, gpu_buf_dptr(b->hrow_dev), MEL_NMEL, gpu_buf_dptr(b->hmap_dev), ring, MEL_NMEL,
                            (uint32_t)nh, MEL_NMEL);
        }
        gpu_upload_async(g, gpu_buf_dptr(b->wmap_dev), b->stage_wmap, (size_t)woff * sizeof(int));
        nk_gather_rows(g, ring, MEL_NMEL, gpu_buf_dptr(b->wmap_dev), gpu_buf_dptr(b->win), (uint32_t)F, (uint32_t)woff,
                       (uint32_t)F);
    } else {
        gpu_upload_async(g, gpu_buf_dptr(b->win), b->stage_win, (size_t)woff * F * sizeof(float));
    }
    gpu_upload_async(g, gpu_buf_dptr(b->etab), crow, (size_t)(6 * M + 4 * nact) * sizeof(int));
    bgraph_t *gs = b->use_graphs ? bgraph_slot(b, M) : NULL;
    if (gs) {
        gs->last_use = ++b->tick;
        if (!gs->graph && gs->seen >= 1 && !gpu_capture_begin(g)) {
            launch_encoder(b, M, nact);
            gs->graph = gpu_capture_end(g);
        }
        gs->seen++;
        if (gs->graph) gpu_graph_launch(g, gs->graph);
        else launch_encoder(b, M, nact);
    } else {
        launch_encoder(b, M, nact);
    }
    for (int i = 0; i < nact; ++i) {
        bstream_t *x = &b->st[b->order[i]];
        const int L = x->cache_len + x->c;
        x->pos += x->c;
        x->cache_len = L < b->left ? L : b->left;
    }
    /* the rows the greedy loop of this step reads (the loop of the previous step reads the other
       buffer while the next encoder step runs) */
    if (b->device_dec) nk_copy(g, gpu_buf_dptr(b->joint_enc), gpu_buf_dptr(b->jdec[b->jpar]), (uint32_t)(M * b->J));
    if (gpu_end(g, err, errlen)) return -1;
    b->stats.encoder_gpu_ms += gpu_last_ms(g);
    *M_out = M;
    return consumed;
}

/* ---- batched greedy RNNT --------------------------------------------------------------------- */

/* rows of the LSTM state buffer: stream s, slot set k: h0, c0, h1, c1 */
static int hc_row(int s, int k, int which) { return (s * 2 + k) * 4 + which; }

static void keep_token(bstream_t *x, int t) {
    if (x->n_tok == x->cap_tok) {
        x->cap_tok = x->cap_tok ? 2 * x->cap_tok : 256;
        x->tok = realloc(x->tok, x->cap_tok * sizeof(int));
    }
    x->tok[x->n_tok++] = t;
}

/* The greedy loop of src/decoder.c:92-127 for the chunks of the streams in order[0..nact). */
static int decoder_batch_run(nemoasr_batch_t *b, int nact, char *err, size_t errlen) {
    model_t *m = b->m;
    gpu_t *g = b->g;
    const int S = b->S, blank = m->cfg.blank_id, maxsym = m->cfg.max_symbols;
    const uint32_t P = (uint32_t)b->P, J = (uint32_t)b->J;
    int *T = b->stage_dtab;
    int *tok = T, *h0c = T + S, *c0c = T + 2 * S, *c0p = T + 3 * S, *h0p = T + 4 * S, *h1c = T + 5 * S, *c1c = T + 6 * S;
    int *c1p = T + 7 * S, *h1p = T + 8 * S, *pidx = T + 9 * S, *erow = T + 10 * S, *prow = erow + S * DEC_WIN;
    const int *D = gpu_buf_dptr(b->dtab);
    const int *dtok = D, *dh0c = D + S, *dc0c = D + 2 * S, *dc0p = D + 3 * S, *dh0p = D + 4 * S, *dh1c = D + 5 * S;
    const int *dc1c = D + 6 * S, *dc1p = D + 7 * S, *dh1p = D + 8 * S, *dpidx = D + 9 * S, *derow = D + 10 * S;
    const int *dprow = derow + S * DEC_WIN;
    float *hc = gpu_buf_dptr(b->hc), *lin = gpu_buf_dptr(b->lin), *gates = gpu_buf_dptr(b->gates);
    float *hout = gpu_buf_dptr(b->hout), *hout2 = gpu_buf_dptr(b->hout2), *pred = gpu_buf_dptr(b->pred);
    int *rcount = malloc((size_t)nact * sizeof(int));
    for (int it = 0;; ++it) {
        if (it > 1 << 20) { free(rcount); snprintf(err, errlen, "decoder: no progress"); return -1; }
        int n = 0, R = 0;
        for (int i = 0; i < nact; ++i) {
            const int s = b->order[i];
            bstream_t *x = &b->st[s];
            rcount[i] = 0;
            if (x->t >= x->frames) continue;
            if (!x->pred_valid) {
                const int kc = x->cur, kp = x->cur ^ 1;
                tok[n] = x->last_token;
                h0c[n] = hc_row(s, kc, 0); c0c[n] = hc_row(s, kc, 1); h1c[n] = hc_row(s, kc, 2); c1c[n] = hc_row(s, kc, 3);
                h0p[n] = hc_row(s, kp, 0); c0p[n] = hc_row(s, kp, 1); h1p[n] = hc_row(s, kp, 2); c1p[n] = hc_row(s, kp, 3);
                pidx[n] = s;
                n++;
            }
            int r = x->frames - x->t;
            if (r > DEC_WIN) r = DEC_WIN;
            for (int k = 0; k < r; ++k) {
                erow[R + k] = x->erow0 + x->t + k;
                prow[R + k] = s;
            }
            rcount[i] = r;
            R += r;
        }
        if (!R) break;
        gpu_begin(g);
        gpu_upload_async(g, gpu_buf_dptr(b->dtab), T, (size_t)(10 * S + 2 * S * DEC_WIN) * sizeof(int));
        if (n) {
            /* prediction network from the committed state, input embed(last token) (zeros for blank) */
            const uint32_t un = (uint32_t)n;
            nk_lstm_input_rows(g, m->embed_dev, dtok, NULL, hc, dh0c, lin, un, P, (uint32_t)blank);
            nk_gemm(g, lin, 2 * P, gpu_buf_dptr(b->wcat[0]), 2 * P, m->lstm_b[0], gates, 4 * P, un, 4 * P, 2 * P,
                    NK_ACT_NONE, 0, 1.0f);
            nk_lstm_cell_rows(g, gates, hc, dc0c, dc0p, dh0p, hout, un, P);
            nk_lstm_input_rows(g, NULL, NULL, hout, hc, dh1c, lin, un, P, (uint32_t)blank);
            nk_gemm(g, lin, 2 * P, gpu_buf_dptr(b->wcat[1]), 2 * P, m->lstm_b[1], gates, 4 * P, un, 4 * P, 2 * P,
                    NK_ACT_NONE, 0, 1.0f);
            nk_lstm_cell_rows(g, gates, hc, dc1c, dc1p, dh1p, hout2, un, P);
            nk_gemm_rows(g, hout2, P, m->joint_pred_w, P, m->joint_pred_b, pred, J, dpidx, un, J, P, NK_ACT_NONE, 0,
                         1.0f);
        }
        /* joint + argmax for every stream's pending frames (speculating blank) */
        const uint32_t uR = (uint32_t)R, Vp = (uint32_t)b->Vp;
        nk_joint_in_rows(g, gpu_buf_dptr(b->joint_enc), pred, derow, dprow, gpu_buf_dptr(b->jin), uR, J);
        nk_gemm(g, gpu_buf_dptr(b->jin), J, gpu_buf_dptr(b->wout), J, gpu_buf_dptr(b->bout), gpu_buf_dptr(b->logits),
                Vp, uR, Vp, J, NK_ACT_NONE, 0, 1.0f);
        nk_argmax_rows(g, gpu_buf_dptr(b->logits), Vp, uR, (uint32_t)b->V, gpu_buf_dptr(b->amax));
        gpu_download_async(g, b->stage_amax, gpu_buf_dptr(b->amax), (size_t)2 * R * sizeof(int));
        if (gpu_end(g, err, errlen)) { free(rcount); return -1; }
        b->stats.joint_steps++;
        const int *res = b->stage_amax;
        int r0 = 0;
        for (int i = 0; i < nact; ++i) {
            bstream_t *x = &b->st[b->order[i]];
            const int rows = rcount[i];
            if (!rows) continue;
            x->pred_valid = 1;
            int k = 0;
            for (; k < rows; ++k) {
                const int pr = res[2 * (r0 + k)];
                if (pr == blank) { x->symbols = 0; continue; }
                keep_token(x, pr);
                b->stats.tokens++;
                x->last_token = pr;
                x->cur ^= 1; /* commit the provisional state */
                x->pred_valid = 0;
                x->symbols++;
                if (x->symbols >= maxsym) { x->symbols = 0; k++; }
                break;
            }
            x->t += k;
            r0 += rows;
        }
    }
    free(rcount);
    return 0;
}

/* ---- device-resident batched greedy loop (kernels/nk_bdec.hip) --------------------------------- */
/* Steps per graph run (even: step parities repeat; the host reads the state back once per run):
 * the first run of a batch step, then runs sized from an estimate of the steps still to go (each
 * stream's decisions per finished frame times its frames left), so that a step whose streams all
 * emit max_symbols per frame takes two runs instead of seven; steps past a stream's end return at
 * once. */
static const int k_brun_steps[6] = { 10, 2, 6, 14, 30, 62 };

static NkBDecArgs bdec_args(nemoasr_batch_t *b) {
    model_t *m = b->m;
    NkBDecArgs a;
    memset(&a, 0, sizeof a);
    a.st = gpu_buf_dptr(b->bst);
    a.keys = gpu_buf_dptr(b->keys);
    a.nkeys = (uint32_t)b->nkeys;
    a.setup = gpu_buf_dptr(b->bsetup);
    a.tokens = gpu_buf_dptr(b->btok);
    a.enc = gpu_buf_dptr(b->jdec[b->dbuf]);
    a.tx = gpu_buf_dptr(b->tx);
    a.hc = gpu_buf_dptr(b->hc);
    a.pre0 = gpu_buf_dptr(b->pre0);
    a.wh0 = (const uint16_t *)gpu_buf_dptr(b->wcati[0]) + b->P; /* the Wh0 half of [Wx0 | Wh0] */
    a.wh0_ld = (uint32_t)(2 * b->P);
    a.A1 = gpu_buf_dptr(b->lin1);
    a.hout = gpu_buf_dptr(b->hout);
    a.pred = gpu_buf_dptr(b->pred);
    a.jin = gpu_buf_dptr(b->jin);
    a.rows = gpu_buf_dptr(b->brows);
    a.cnt = gpu_buf_dptr(b->bcnt);
    a.S = (uint32_t)b->S;
    a.W = (uint32_t)b->W;
    a.P = (uint32_t)b->P;
    a.J = (uint32_t)b->J;
    a.blank = (uint32_t)m->cfg.blank_id;
    a.max_symbols = (uint32_t)m->cfg.max_symbols;
    a.tok_ld = (uint32_t)b->tok_ld;
    return a;
}

/* `steps` decoder steps over all streams (fixed shapes: one graph serves every run) */
typedef NkBDecGemmArgs bdec_launch_t;

/* grid: N / 16 column workgroups (plus gx_more) by row blocks of 64 */
static int launch_bdec_gemm(nemoasr_batch_t *b, uint32_t par, const char *kernel, const float *A, uint32_t lda,
                            const uint16_t *W, uint32_t ldw, const float *bias, uint32_t N, uint32_t K, uint32_t waves,
                            uint32_t gx_more) {
    bdec_launch_t x;
    memset(&x, 0, sizeof x);
    x.g.A = A;
    x.g.lda = lda;
    x.g.W = W;
    x.g.ldw = ldw;
    x.g.bias = bias;
    x.g.M = (uint32_t)b->S;
    x.g.N = N;
    x.g.K = K;
    x.d = bdec_args(b);
    x.d.par = par;
    return gpu_launch(b->gd, kernel, &x, sizeof x, N / 16 + gx_more, ((uint32_t)b->S + 63) / 64, 1, 64 * waves, 1, 1);
}

static void launch_bdec_steps(nemoasr_batch_t *b, int steps) {
    gpu_t *g = b->gd;
    NkBDecArgs a = bdec_args(b);
    const uint32_t S = a.S, P = a.P, J = a.J, Vp = (uint32_t)b->Vp, R = a.S * a.W;
    for (int k = 0; k < steps; ++k) {
        /* step parity: the rows come from counter par ^ 1, the decisions append to counter par */
        const uint32_t par = (uint32_t)k & 1u;
        a.par = par;
        launch_bdec_gemm(b, par, "bdec_lstm1_w8s5", a.A1, 2 * P, gpu_buf_dptr(b->wcati[1]), 2 * P,
                         gpu_buf_dptr(b->bi[1]), 4 * P, 2 * P, 8, 0);
        /* joint.pred, and the hidden half of the next step's layer 0 (4P/16 more workgroups) */
        launch_bdec_gemm(b, par, "bdec_pred_w4s5", a.hout, P, b->m->joint_pred_w, P, b->m->joint_pred_b, J, P, 4,
                         4 * P / 16);
        /* more than one row block: only the step's rows are scored */
        nk_gemm_argmax_rows(g, a.jin, J, gpu_buf_dptr(b->wout), J, gpu_buf_dptr(b->bout), gpu_buf_dptr(b->keys),
                            (uint32_t)b->nkeys, R, Vp, J, (uint32_t)b->V, S > 64 ? a.cnt + (par ^ 1u) : NULL, a.W);
        gpu_launch(g, "bdec_decide", &a, sizeof a, S, 1, 1, 256, 1, 1);
    }
}

/* the chunks of order[0..nact) through the device loop: one setup launch, then graph runs of
 * k_brun_steps steps until every chunk is done */
static int decoder_batch_device(nemoasr_batch_t *b, char *err, size_t errlen) {
    gpu_t *g = b->gd;
    const int S = b->S, nact = b->dnact;
    int *su = b->stage_bsetup;
    memset(su, 0, (size_t)(2 * S + 2) * sizeof(int));
    int maxc = 0;
    for (int i = 0; i < nact; ++i) {
        su[2 * b->dorder[i]] = b->dc[i];
        su[2 * b->dorder[i] + 1] = b->drow0[i];
        if (b->dc[i] > maxc) maxc = b->dc[i];
    }
    if (maxc > b->W) { snprintf(err, errlen, "decoder: chunk of %d frames exceeds %d", maxc, b->W); return -1; }
    const NkBDecArgs a = bdec_args(b);
    const int max_runs = (maxc * b->m->cfg.max_symbols + maxc) / k_brun_steps[1] + 3;
    for (int run = 0;; ++run) {
        if (run >= max_runs) { snprintf(err, errlen, "decoder: no progress"); return -1; }
        int which = 0;
        if (run) {
            int est = 0;
            for (int i = 0; i < nact; ++i) {
                const NkBDecStream *x = &b->stage_bst[b->dorder[i]];
                const int left = x->frames - x->t;
                if (left <= 0) continue;
                const int e = x->t > 0 ? (x->joints * left + x->t - 1) / x->t + 1 : (x->joints + 1) * left;
                if (e > est) est = e;
            }
            which = 5;
            for (int k = 1; k < 6; ++k)
                if (k_brun_steps[k] >= est) { which = k; break; }
        }
        gpu_begin(g);
        if (run == 0) {
            gpu_upload_async(g, gpu_buf_dptr(b->bsetup), su, (size_t)2 * S * sizeof(int));
            gpu_upload_async(g, gpu_buf_dptr(b->bcnt), su + 2 * S, 2 * sizeof(int)); /* zero row counters */
            gpu_launch(g, "bdec_setup", &a, sizeof a, (uint32_t)S, 1, 1, 64, 1, 1);
        }
        gpu_graph_t **gslot = &b->dgraph[b->dbuf][which];
        if (b->use_graphs && !*gslot) {
            if (b->dstarted) pthread_mutex_lock(&b->cmu);
            if (!gpu_capture_begin(g)) {
                launch_bdec_steps(b, k_brun_steps[which]);
                *gslot = gpu_capture_end(g);
            }
            if (b->dstarted) pthread_mutex_unlock(&b->cmu);
        }
        if (*gslot) gpu_graph_launch(g, *gslot);
        else launch_bdec_steps(b, k_brun_steps[which]);
        gpu_download_async(g, b->stage_bst, gpu_buf_dptr(b->bst), (size_t)S * sizeof(NkBDecStream));
        gpu_download_async(g, b->stage_btok, gpu_buf_dptr(b->btok), (size_t)S * b->tok_ld * sizeof(int));
        if (gpu_end(g, err, errlen)) return -1;
        int done = 1;
        for (int i = 0; i < nact && done; ++i) {
            const NkBDecStream *x = &b->stage_bst[b->dorder[i]];
            done = x->t >= x->frames;
        }
        if (done) break;
    }
    /* the batched joint evaluations: the steps in which some stream was still inside its chunk */
    int live = 0;
    for (int i = 0; i < nact; ++i)
        if (b->stage_bst[b->dorder[i]].joints > live) live = b->stage_bst[b->dorder[i]].joints;
    b->stats.joint_steps += (size_t)live;
    for (int i = 0; i < nact; ++i) {
        const int s = b->dorder[i];
        const int n = b->stage_bst[s].n_out;
        if (n > b->tok_ld) { snprintf(err, errlen, "decoder: stream %d emitted %d tokens in a chunk", s, n); return -1; }
        for (int k = 0; k < n; ++k) keep_token(&b->st[s], b->stage_btok[(size_t)s * b->tok_ld + k]);
        b->stats.tokens += (size_t)n;
    }
    return 0;
}

static void record_step(nemoasr_batch_t *b, double ms) {
    if (b->n_step == b->cap_step) {
        b->cap_step = b->cap_step ? 2 * b->cap_step : 256;
        b->step_ms = realloc(b->step_ms, b->cap_step * sizeof(double));
    }
    b->step_ms[b->n_step++] = ms;
}

static void *dec_main(void *arg) {
    nemoasr_batch_t *b = arg;
    pthread_mutex_lock(&b->dmu);
    for (;;) {
        while (!b->dquit && b->dstate != 1) pthread_cond_wait(&b->dcv, &b->dmu);
        if (b->dquit) break;
        b->dstate = 2;
        pthread_mutex_unlock(&b->dmu);
        char err[256] = "";
        const double t1 = now_ms();
        const int rc = decoder_batch_device(b, err, sizeof err);
        const double t2 = now_ms();
        b->stats.decoder_ms += t2 - t1;
        record_step(b, t2 - b->dt0);
        pthread_mutex_lock(&b->dmu);
        if (rc && !b->drc) {
            b->drc = -1;
            snprintf(b->derr, sizeof b->derr, "%s", err);
        }
        b->dstate = 0;
        pthread_cond_broadcast(&b->dcv);
    }
    pthread_mutex_unlock(&b->dmu);
    return NULL;
}

/* wait until the worker is idle; report an error of the loop it ran */
static int dec_drain(const nemoasr_batch_t *cb, char *err, size_t errlen) {
    nemoasr_batch_t *b = (nemoasr_batch_t *)cb;
    if (!b->dstarted) return 0;
    pthread_mutex_lock(&b->dmu);
    while (b->dstate) pthread_cond_wait(&b->dcv, &b->dmu);
    const int rc = b->drc;
    if (rc && errlen) snprintf(err, errlen, "%s", b->derr);
    b->drc = 0;
    pthread_mutex_unlock(&b->dmu);
    return rc;
}

static int dec_start(nemoasr_batch_t *b) {
    pthread_mutex_init(&b->dmu, NULL);
    pthread_mutex_init(&b->cmu, NULL);
    pthread_cond_init(&b->dcv, NULL);
    if (pthread_create(&b->dth, NULL, dec_main, b)) {
        pthread_mutex_destroy(&b->dmu);
        pthread_mutex_destroy(&b->cmu);
        pthread_cond_destroy(&b->dcv);
        return -1;
    }
    b->dstarted = 1;
    return 0;
}

static void dec_stop(nemoasr_batch_t *b) {
    if (!b->dstarted) return;
    pthread_mutex_lock(&b->dmu);
    while (b->dstate) pthread_cond_wait(&b->dcv, &b->dmu);
    b->dquit = 1;
    pthread_cond_broadcast(&b->dcv);
    pthread_mutex_unlock(&b->dmu);
    pthread_join(b->dth, NULL);
    pthread_mutex_destroy(&b->dmu);
    pthread_mutex_destroy(&b->cmu);
    pthread_cond_destroy(&b->dcv);
    b->dstarted = 0;
}

/* debug dumps: the step's joint.enc rows, appended per stream */
static int step_dump(nemoasr_batch_t *b, int M, char *err, size_t errlen) {
    if (!b->dump) return 0;
    const size_t J = (size_t)b->J;
    float *all = malloc((size_t)M * J * sizeof(float));
    if (gpu_download(b->g, all, gpu_buf_dptr(b->joint_enc), (size_t)M * J * sizeof(float))) {
        free(all);
        snprintf(err, errlen, "batch: dump download failed");
        return -1;
    }
    for (int s = 0; s < b->S; ++s) {
        const bstream_t *x = &b->st[s];
        if (x->c <= 0) continue;
        if (b->dj_n[s] + (size_t)x->c > b->dj_cap[s]) {
            b->dj_cap[s] = (b->dj_n[s] + (size_t)x->c) * 2 + 64;
            b->dj[s] = realloc(b->dj[s], b->dj_cap[s] * J * sizeof(float));
        }
        memcpy(b->dj[s] + b->dj_n[s] * J, all + (size_t)x->row0 * J, (size_t)x->c * J * sizeof(float));
        b->dj_n[s] += (size_t)x->c;
    }
    free(all);
    return 0;
}

int nemoasr_batch_step(nemoasr_batch_t *b, char *err, size_t errlen) {
    if (errlen) err[0] = 0;
    const double t0 = now_ms();
    int M = 0;
    if (b->dstarted) pthread_mutex_lock(&b->cmu);
    const int consumed = encoder_batch_step(b, &M, err, errlen);
    const int rc = consumed < 0 || !M ? 0 : step_dump(b, M, err, errlen);
    if (b->dstarted) pthread_mutex_unlock(&b->cmu);
    if (consumed < 0 || rc) return -1;
    if (!M) return consumed;
    const double t1 = now_ms();
    int nact = 0;
    for (int s = 0; s < b->S; ++s) {
        bstream_t *x = &b->st[s];
        if (x->c <= 0) continue;
        nact++;
    }
    /* order[] holds the streams of this step in row order */
    for (int i = 0; i < nact; ++i) {
        bstream_t *x = &b->st[b->order[i]];
        x->frames = x->c;
        x->t = 0;
        x->symbols = 0;
        x->erow0 = x->row0;
    }
    b->stats.steps++;
    b->stats.chunks += (size_t)nact;
    b->stats.rows += (size_t)M;
    b->stats.encoder_ms += t1 - t0;
    if (b->device_dec) {
        /* hand the step's greedy loop to the worker once it has finished the previous one; this
           step's joint.enc rows are already in jdec[jpar] (copied by the encoder step) */
        if (dec_drain(b, err, errlen)) return -1;
        for (int i = 0; i < nact; ++i) {
            const bstream_t *x = &b->st[b->order[i]];
            b->dorder[i] = b->order[i];
            b->dc[i] = x->c;
            b->drow0[i] = x->row0;
        }
        b->dnact = nact;
        b->dbuf = b->jpar;
        b->dt0 = t0;
        b->jpar ^= 1;
        pthread_mutex_lock(&b->dmu);
        b->dstate = 1;
        pthread_cond_broadcast(&b->dcv);
        pthread_mutex_unlock(&b->dmu);
        return consumed;
    }
    if (decoder_batch_run(b, nact, err, errlen)) return -1;
    const double t2 = now_ms();
    b->stats.decoder_ms += t2 - t1;
    record_step(b, t2 - t0);
    return consumed;
}

int nemoasr_batch_run(nemoasr_batch_t *b, char *err, size_t errlen) {
    int steps = 0;
    for (;;) {
        const int rc = nemoasr_batch_step(b, err, errlen);
        if (rc < 0) return -1;
        if (rc == 0) return dec_drain(b, err, errlen) ? -1 : steps;
        steps++;
    }
}

const int *nemoasr_batch_tokens(const nemoasr_batch_t *b, int stream, size_t *n) {
    dec_drain(b, NULL, 0);
    if (stream < 0 || stream >= b->S) { *n = 0; return NULL; }
    *n = b->st[stream].n_tok;
    return b->st[stream].tok;
}

/* token pieces as text, leading spaces of the first printed piece dropped (src/nemoasr.c:123-129) */
char *nemoasr_batch_text(nemoasr_batch_t *b, int stream) {
    dec_drain(b, NULL, 0);
    if (stream < 0 || stream >= b->S) return NULL;
    bstream_t *x = &b->st[stream];
    char *out = NULL;
    size_t len = 0, cap = 0;
    for (; x->n_text < x->n_tok; ++x->n_text) {
        char *txt = piece_text(&b->m->vocab, x->tok[x->n_text]);
        const char *p = txt;
        if (!x->printed_any) while (*p == ' ') p++;
        const size_t k = strlen(p);
        if (k) {
            if (len + k + 1 > cap) {
                cap = (len + k + 1) * 2;
                out = realloc(out, cap);
            }
            memcpy(out + len, p, k + 1);
            len += k;
            x->printed_any = 1;
        }
        free(txt);
    }
    return out;
}

int nemoasr_batch_reset_stream(nemoasr_batch_t *b, int stream, char *err, size_t errlen) {
    if (errlen) err[0] = 0;
    if (check_stream(b, stream, err, errlen)) return -1;
    if (dec_drain(b, err, errlen)) return -1;
    stream_clear(b, stream);
    b->st[stream].n_tok = 0;
    if (stream_zero_device(b, stream)) { snprintf(err, errlen, "batch: reset upload failed"); return -1; }
    return 0;
}

void nemoasr_batch_stats(const nemoasr_batch_t *b, nemoasr_batch_stats_t *out) {
    dec_drain(b, NULL, 0);
    *out = b->stats;
}

const double *nemoasr_batch_step_ms(const nemoasr_batch_t *b, size_t *n) {
    dec_drain(b, NULL, 0);
    *n = b->n_step;
    return b->step_ms;
}

/* ---- test hooks ---------------------------------------------------------------------------- */
void nemoasr_batch_debug_use_graphs(nemoasr_batch_t *b, int on) {
    dec_drain(b, NULL, 0);
    b->use_graphs = on;
    if (!on) {
        drop_graphs(b);
        for (int i = 0; i < 2; ++i)
            for (int k = 0; k < 6; ++k) {
                gpu_graph_free(b->dgraph[i][k]);
                b->dgraph[i][k] = NULL;
            }
    }
}

int nemoasr_batch_debug_gpu_frontend(nemoasr_batch_t *b, int on) {
    for (int s = 0; s < b->S; ++s) {
        const bstream_t *x = &b->st[s];
        if (x->src || x->pending_n || x->aq_n || x->consumed) return -1;
    }
    b->gpu_fe = on != 0;
    return 0;
}

int nemoasr_batch_debug_device_decoder(nemoasr_batch_t *b, int on) {
    /* the two loops keep their greedy state apart (the device loop's stream records, its stored
     * hidden halves of layer 0): the choice is made before any input */
    for (int s = 0; s < b->S; ++s) {
        const bstream_t *x = &b->st[s];
        if (x->src || x->pending_n || x->aq_n || x->consumed) return -1;
    }
    dec_drain(b, NULL, 0);
    b->device_dec = on && b->gd && device_dec_ok(b);
    return 0;
}

void nemoasr_batch_debug_set_dump(nemoasr_batch_t *b, int on) {
    b->dump = on;
    if (on && !b->dj) {
        b->dj = calloc((size_t)b->S, sizeof(float *));
        b->dj_n = calloc((size_t)b->S, sizeof(size_t));
        b->dj_cap = calloc((size_t)b->S, sizeof(size_t));
    }
}

const float *nemoasr_batch_debug_joint_enc(const nemoasr_batch_t *b, int stream, size_t *frames) {
    if (!b->dj || stream < 0 || stream >= b->S) { *frames = 0; return NULL; }
    *frames = b->dj_n[stream];
    return b->dj[stream];
}

int nemoasr_batch_debug_time_kernel(nemoasr_batch_t *b, const char *kernel, int max_launches) {
    return gpu_timing_set(b->g, kernel, max_launches);
}

int nemoasr_batch_debug_kernel_ms(nemoasr_batch_t *b, double *mean_ms, int *count, double *bytes, double *flops) {
    const int rc = gpu_timing_collect(b->g, mean_ms, count, bytes);
    if (flops) *flops = gpu_timing_last_flops(b->g);
    return rc;
}
