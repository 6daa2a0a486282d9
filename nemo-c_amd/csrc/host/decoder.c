/* Greedy RNN-T decoder (see decoder.h).
 *
 * The loop is the reference's (src/decoder.c:92-127): committed and provisional LSTM states, the
 * joint evaluated for up to 16 remaining frames per step with the current prediction (speculating
 * blank), and on the first non-blank: emit, commit the provisional state, redo the later frames.
 * It runs on the device (kernels/nk_dec.hip): one step is three launches, a graph holds a run of
 * steps, and the host replays graphs until the device state says the chunk is done.  The host
 * reads back the state and the emitted tokens once per graph, not once per joint evaluation. */
#include "decoder.h"
#include "nemo_kernels.h"
#include "../kernel_params.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* Steps per graph run (odd: see launch_steps): the first run of a chunk, then runs sized from an
 * estimate of the steps still to go, so that a long chunk (560 ms with every frame emitting
 * max_symbols: ~70 steps) takes two or three runs instead of five; an overestimate costs steps
 * whose kernels return at once, an underestimate one more host round trip. */
static const int k_run_steps[] = { 11, 3, 7, 15, 31, 63 };
#define N_RUN_SIZES (int)(sizeof k_run_steps / sizeof k_run_steps[0])
#define MAX_GRAPHS_PER_CHUNK 64
/* graph sets kept, one per joint.enc buffer (a session keeps one encoder per prepared latency) */
#define DEC_GRAPH_SETS 5

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec / 1e6;
}

typedef struct {
    const float *enc;
    gpu_graph_t *g[N_RUN_SIZES]; /* by k_run_steps index */
} dgraph_t;

struct decoder {
    model_t *m;
    gpu_t *g;
    gpu_buf_t *st, *part, *tokens, *hc, *pre0, *pred, *tx;
    NkDecState *host_st; /* pinned: chunk fields in, final state out */
    int *host_tok;       /* pinned: tokens of the chunk               */
    dgraph_t gr[DEC_GRAPH_SETS];
    int ngr, last_steps, use_graphs;
    double last_ms;
};

static NkDecArgs dec_args(decoder_t *d, const float *enc, uint32_t parity, uint32_t decide_only);

decoder_t *decoder_create(model_t *m) {
    decoder_t *d = calloc(1, sizeof *d);
    d->m = m;
    d->g = m->gpu;
    const size_t P = (size_t)m->cfg.pred_hidden, J = (size_t)m->cfg.joint_hidden;
    d->st = gpu_buf_alloc(d->g, 2 * sizeof(NkDecState));
    d->part = gpu_buf_alloc(d->g, 2 * NK_DEC_MAX_BATCH * NK_DEC_GROUPS * sizeof(unsigned long long));
    d->tokens = gpu_buf_alloc(d->g, NK_DEC_MAX_TOKENS * sizeof(int));
    d->hc = gpu_buf_alloc(d->g, 2 * 4 * P * sizeof(float));
    d->pre0 = gpu_buf_alloc(d->g, 2 * 4 * P * sizeof(float));
    d->pred = gpu_buf_alloc(d->g, J * sizeof(float));
    d->host_st = gpu_host_alloc(d->g, sizeof(NkDecState));
    d->host_tok = gpu_host_alloc(d->g, NK_DEC_MAX_TOKENS * sizeof(int));
    /* the layer-0 input table, one row per token and the blank's (zero input) row */
    const uint32_t nv = (uint32_t)m->cfg.blank_id + 1;
    d->tx = gpu_buf_alloc(d->g, (size_t)nv * 4 * P * sizeof(float));
    const NkDecArgs a = dec_args(d, NULL, 0, 0);
    gpu_begin(d->g);
    gpu_launch(d->g, "dec_tx_build", &a, sizeof a, (uint32_t)(P + 3) / 4, nv, 1, 256, 1, 1);
    if (gpu_end(d->g, NULL, 0)) {
        decoder_destroy(d);
        return NULL;
    }
    d->use_graphs = 1;
    decoder_reset(d);
    return d;
}

static void free_graphs(decoder_t *d) {
    for (int i = 0; i < d->ngr; ++i)
        for (int k = 0; k < N_RUN_SIZES; ++k) gpu_graph_free(d->gr[i].g[k]);
    memset(d->gr, 0, sizeof d->gr);
    d->ngr = 0;
}

void decoder_destroy(decoder_t *d) {
    if (!d) return;
    free_graphs(d);
    gpu_buf_t *bufs[] = { d->st, d->part, d->tokens, d->hc, d->pre0, d->pred, d->tx };
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs; ++i) gpu_buf_free(bufs[i]);
    gpu_host_free(d->host_st);
    gpu_host_free(d->host_tok);
    free(d);
}

/* src/decoder.c:48-53: zero LSTM state (so Wh0 . h0 is zero too), last token blank, no valid
 * prediction */
void decoder_reset(decoder_t *d) {
    const size_t P = (size_t)d->m->cfg.pred_hidden;
    float *z = calloc(2 * 4 * P, sizeof(float));
    gpu_upload(d->g, gpu_buf_dptr(d->hc), z, 2 * 4 * P * sizeof(float));
    gpu_upload(d->g, gpu_buf_dptr(d->pre0), z, 2 * 4 * P * sizeof(float));
    free(z);
    NkDecState s[2];
    memset(s, 0, sizeof s);
    s[0].last_token = d->m->cfg.blank_id;
    gpu_upload(d->g, gpu_buf_dptr(d->st), s, sizeof s);
}
double decoder_last_ms(const decoder_t *d) { return d->last_ms; }
void decoder_use_graphs(decoder_t *d, int on) {
    d->use_graphs = on;
    if (!on) free_graphs(d);
}
int decoder_last_steps(const decoder_t *d) { return d->last_steps; }



static NkDecArgs dec_args(decoder_t *d, const float *enc, uint32_t parity, uint32_t decide_only) {
    const model_t *m = d->m;
    NkDecArgs a;
    memset(&a, 0, sizeof a);
    a.st = gpu_buf_dptr(d->st);
    a.part = gpu_buf_dptr(d->part);
    a.tokens = gpu_buf_dptr(d->tokens);
    a.enc = enc;
    a.embed = m->embed_dev;
    a.wx0 = m->lstm_wx[0]; a.wh0 = m->lstm_wh[0]; a.wx1 = m->lstm_wx[1]; a.wh1 = m->lstm_wh[1];
    a.b0 = m->lstm_b[0]; a.b1 = m->lstm_b[1];
    a.hc = gpu_buf_dptr(d->hc);
    a.pre0 = gpu_buf_dptr(d->pre0);
    a.wjp = m->joint_pred_w; a.bjp = m->joint_pred_b;
    a.pred = gpu_buf_dptr(d->pred);
    a.wout = m->joint_out_w; a.bout = m->joint_out_b;
    a.tx = gpu_buf_dptr(d->tx);
    a.P = (uint32_t)m->cfg.pred_hidden;
    a.J = (uint32_t)m->cfg.joint_hidden;
    a.V = (uint32_t)m->cfg.num_classes;
    a.blank = (uint32_t)m->cfg.blank_id;
    a.max_symbols = (uint32_t)m->cfg.max_symbols;
    a.parity = parity;
    a.enc_ld = a.J;
    a.decide_only = decide_only;
    return a;
}

/* `steps` steps (odd) then the decision of the last joint: step j reads state copy j%2, so the run
 * ends with the state back in copy 0, where the next run starts. */
static int launch_steps(decoder_t *d, const float *enc, int steps) {
    gpu_t *g = d->g;
    const uint32_t P = (uint32_t)d->m->cfg.pred_hidden, J = (uint32_t)d->m->cfg.joint_hidden;
    for (int j = 0; j <= steps; ++j) {
        const NkDecArgs a = dec_args(d, enc, (uint32_t)j & 1u, j == steps);
        if (gpu_launch(g, "dec_step", &a, sizeof a, (P + 3) / 4, 1, 1, 256, 1, 1)) return -1;
        if (j == steps) break;
        if (gpu_launch(g, "dec_pred", &a, sizeof a, (J + 3) / 4, 1, 1, 256, 1, 1)) return -1;
        if (gpu_launch(g, "dec_joint", &a, sizeof a, NK_DEC_GROUPS, NK_DEC_MAX_BATCH, 1, 256, 1, 1)) return -1;
    }
    return 0;
}

static dgraph_t *graphs_for(decoder_t *d, const float *enc) {
    for (int i = 0; i < d->ngr; ++i)
        if (d->gr[i].enc == enc) return &d->gr[i];
    if (d->ngr == DEC_GRAPH_SETS) free_graphs(d);
    dgraph_t *x = &d->gr[d->ngr++];
    x->enc = enc;
    return x;
}

int decoder_run(decoder_t *d, const float *joint_enc, int frames, int *out, int max_out, char *err, size_t errlen) {
    model_t *m = d->m;
    gpu_t *g = d->g;
    const double t0 = now_ms();
    d->last_steps = 0;
    if (frames <= 0) { d->last_ms = now_ms() - t0; return 0; }
    const uint32_t P = (uint32_t)m->cfg.pred_hidden, J = (uint32_t)m->cfg.joint_hidden;
    if (frames > NK_DEC_MAX_BATCH || P % 8 || P > 1024 || J % 8 || J > 1024 || m->cfg.num_classes > 32 * NK_DEC_GROUPS ||
        (long)frames * m->cfg.max_symbols > NK_DEC_MAX_TOKENS) {
        snprintf(err, errlen, "decoder: unsupported sizes (frames %d, pred %u, joint %u)", frames, P, J);
        return -1;
    }
    dgraph_t *gr = graphs_for(d, joint_enc);
    /* chunk fields of state copy 0: frames, t, symbols, n_out, pending, joints */
    NkDecState *h = d->host_st;
    memset(h, 0, sizeof *h);
    h->frames = frames;
    int n = 0;
    for (int run = 0;; ++run) {
        if (run >= MAX_GRAPHS_PER_CHUNK) { snprintf(err, errlen, "decoder: no progress"); return -1; }
        int which = 0;
        if (run) {
            /* steps still to go, from the chunk's pace so far (decisions per finished frame) */
            const int left = h->frames - h->t;
            const int est = h->t > 0 ? (h->joints * left + h->t - 1) / h->t + 1 : (h->joints + 1) * left;
            which = N_RUN_SIZES - 1;
            for (int k = 1; k < N_RUN_SIZES; ++k)
                if (k_run_steps[k] >= est) { which = k; break; }
        }
        gpu_begin(g);
        if (!run) gpu_upload_async(g, gpu_buf_dptr(d->st), h, 6 * sizeof(int));
        if (d->use_graphs && !gr->g[which]) {
            if (!gpu_capture_begin(g)) {
                launch_steps(d, joint_enc, k_run_steps[which]);
                gr->g[which] = gpu_capture_end(g);
            }
        }
        if (gr->g[which]) gpu_graph_launch(g, gr->g[which]);
        else launch_steps(d, joint_enc, k_run_steps[which]);
        gpu_download_async(g, h, gpu_buf_dptr(d->st), sizeof *h);
        gpu_download_async(g, d->host_tok, gpu_buf_dptr(d->tokens), NK_DEC_MAX_TOKENS * sizeof(int));
        if (gpu_end(g, err, errlen)) return -1;
        if (h->done) break;
    }
    const int nt = h->n_out < NK_DEC_MAX_TOKENS ? h->n_out : NK_DEC_MAX_TOKENS;
    for (int i = 0; i < nt; ++i)
        if (n < max_out) out[n++] = d->host_tok[i];
    d->last_steps = h->joints;
    d->last_ms = now_ms() - t0;
    return n;
}

/* Capture the graph of every run size for chunks whose joint.enc rows live at joint_enc, without
 * running them (warm-up: the first chunks of a session then replay graphs from their first step).
 * Returns the number of graphs held for that buffer. */
int decoder_prepare_graphs(decoder_t *d, const float *joint_enc) {
    if (!d->use_graphs) return 0;
    dgraph_t *gr = graphs_for(d, joint_enc);
    int n = 0;
    for (int k = 0; k < N_RUN_SIZES; ++k) {
        if (!gr->g[k]) {
            gpu_begin(d->g);
            if (!gpu_capture_begin(d->g)) {
                launch_steps(d, joint_enc, k_run_steps[k]);
                gr->g[k] = gpu_capture_end(d->g);
            }
            if (gpu_end(d->g, NULL, 0)) break;
        }
        n += gr->g[k] != NULL;
    }
    return n;
}
