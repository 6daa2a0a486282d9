/* Greedy RNN-T decoder (see decoder.h).
 *
 * The loop is the reference's (src/decoder.c:92-127): committed and provisional LSTM states, the
 * joint evaluated for up to 16 remaining frames per round trip with the current prediction
 * (speculating blank), and on the first non-blank: emit, commit the provisional state, redo the
 * later frames.  A round trip is one ordered batch on the stream: [embedding row upload,
 * 2 x (Wx GEMV + bias, Wh GEMV accumulate, LSTM cell), joint.pred GEMV], joint scoring + argmax,
 * and a download of 2 ints per frame into pinned memory. */
#include "decoder.h"
#include "nemo_kernels.h"
#include "../kernel_params.h"
#include "safetensors.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec / 1e6;
}

struct decoder {
    model_t *m;
    gpu_t *g;
    gpu_buf_t *x, *gates, *pred_out, *argmax, *part_v, *part_i, *state;
    float *h[2], *c[2], *hp[2], *cp[2]; /* device: committed and provisional LSTM state */
    float *x_host;                        /* pinned: embedding row */
    int *res_host;                        /* pinned: argmax results */
    int last_token, pred_valid, last_steps;
    double last_ms;
};

decoder_t *decoder_create(model_t *m) {
    decoder_t *d = calloc(1, sizeof *d);
    d->m = m;
    d->g = m->gpu;
    const size_t P = (size_t)m->cfg.pred_hidden, fs = sizeof(float);
    d->x = gpu_buf_alloc(d->g, P * fs);
    d->gates = gpu_buf_alloc(d->g, 4 * P * fs);
    d->pred_out = gpu_buf_alloc(d->g, (size_t)m->cfg.joint_hidden * fs);
    d->argmax = gpu_buf_alloc(d->g, NK_DEC_MAX_BATCH * 2 * sizeof(int));
    d->part_v = gpu_buf_alloc(d->g, NK_DEC_MAX_BATCH * NK_JOINT_GROUPS * NK_JOINT_WAVES * fs);
    d->part_i = gpu_buf_alloc(d->g, NK_DEC_MAX_BATCH * NK_JOINT_GROUPS * NK_JOINT_WAVES * sizeof(int));
    d->state = gpu_buf_alloc(d->g, 8 * P * fs);
    float *s = gpu_buf_dptr(d->state);
    for (int l = 0; l < 2; ++l) {
        d->h[l] = s + (0 + l) * P;
        d->c[l] = s + (2 + l) * P;
        d->hp[l] = s + (4 + l) * P;
        d->cp[l] = s + (6 + l) * P;
    }
    d->x_host = gpu_host_alloc(d->g, P * fs);
    d->res_host = gpu_host_alloc(d->g, NK_DEC_MAX_BATCH * 2 * sizeof(int));
    decoder_reset(d);
    return d;
}

void decoder_destroy(decoder_t *d) {
    if (!d) return;
    gpu_buf_t *bufs[] = { d->x, d->gates, d->pred_out, d->argmax, d->part_v, d->part_i, d->state };
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs; ++i) gpu_buf_free(bufs[i]);
    gpu_host_free(d->x_host);
    gpu_host_free(d->res_host);
    free(d);
}

/* src/decoder.c:48-53 */
void decoder_reset(decoder_t *d) {
    const size_t P = (size_t)d->m->cfg.pred_hidden;
    float *z = calloc(4 * P, sizeof(float));
    gpu_upload(d->g, gpu_buf_dptr(d->state), z, 4 * P * sizeof(float)); /* h[0], h[1], c[0], c[1] */
    free(z);
    float *s = gpu_buf_dptr(d->state);
    for (int l = 0; l < 2; ++l) {
        d->h[l] = s + (0 + l) * P;
        d->c[l] = s + (2 + l) * P;
        d->hp[l] = s + (4 + l) * P;
        d->cp[l] = s + (6 + l) * P;
    }
    d->last_token = d->m->cfg.blank_id;
    d->pred_valid = 0;
}
double decoder_last_ms(const decoder_t *d) { return d->last_ms; }
int decoder_last_steps(const decoder_t *d) { return d->last_steps; }

/* prediction network from the committed state, input embed(last_token) or zeros for blank:
 * src/decoder.c:57-77 */
static void encode_pred(decoder_t *d) {
    model_t *m = d->m;
    gpu_t *g = d->g;
    const uint32_t P = (uint32_t)m->cfg.pred_hidden, J = (uint32_t)m->cfg.joint_hidden;
    if (d->last_token == m->cfg.blank_id) memset(d->x_host, 0, P * sizeof(float));
    else {
        const uint16_t *row = m->embed_host + (size_t)d->last_token * P;
        for (uint32_t i = 0; i < P; ++i) d->x_host[i] = st_bf16(row[i]);
    }
    gpu_upload_async(g, gpu_buf_dptr(d->x), d->x_host, P * sizeof(float));
    const float *in = gpu_buf_dptr(d->x);
    float *gates = gpu_buf_dptr(d->gates);
    for (int l = 0; l < 2; ++l) {
        nk_gemm(g, in, P, m->lstm_wx[l], P, m->lstm_b[l], gates, 4 * P, 1, 4 * P, P, NK_ACT_NONE, 0, 1.0f);
        nk_gemm(g, d->h[l], P, m->lstm_wh[l], P, NULL, gates, 4 * P, 1, 4 * P, P, NK_ACT_NONE, 1, 1.0f);
        nk_lstm_cell(g, gates, d->c[l], d->cp[l], d->hp[l], P);
        in = d->hp[l];
    }
    nk_gemm(g, d->hp[1], P, m->joint_pred_w, P, m->joint_pred_b, gpu_buf_dptr(d->pred_out), J, 1, J, P, NK_ACT_NONE, 0, 1.0f);
}

int decoder_run(decoder_t *d, const float *joint_enc, int frames, int *out, int max_out, char *err, size_t errlen) {
    model_t *m = d->m;
    gpu_t *g = d->g;
    const double t0 = now_ms();
    const uint32_t J = (uint32_t)m->cfg.joint_hidden, V = (uint32_t)m->cfg.num_classes;
    int n = 0, steps = 0, t = 0, symbols = 0;
    while (t < frames) {
        int rows = frames - t;
        if (rows > NK_DEC_MAX_BATCH) rows = NK_DEC_MAX_BATCH;
        gpu_begin(g);
        if (!d->pred_valid) encode_pred(d);
        nk_joint_argmax(g, joint_enc, (uint32_t)t, J, (uint32_t)rows, gpu_buf_dptr(d->pred_out), m->joint_out_w,
                        m->joint_out_b, V, J, gpu_buf_dptr(d->part_v), gpu_buf_dptr(d->part_i), gpu_buf_dptr(d->argmax));
        gpu_download_async(g, d->res_host, gpu_buf_dptr(d->argmax), (size_t)rows * 2 * sizeof(int));
        if (gpu_end(g, err, errlen)) return -1;
        steps++;
        d->pred_valid = 1;
        int i = 0;
        for (; i < rows; ++i) {
            const int pred = d->res_host[2 * i];
            if (pred == m->cfg.blank_id) { symbols = 0; continue; } /* blank: frame done, keep the prediction */
            if (n < max_out) out[n++] = pred;
            d->last_token = pred;
            for (int l = 0; l < 2; ++l) { /* commit the provisional state */
                float *s = d->h[l]; d->h[l] = d->hp[l]; d->hp[l] = s;
                s = d->c[l]; d->c[l] = d->cp[l]; d->cp[l] = s;
            }
            d->pred_valid = 0;
            symbols++;
            if (symbols >= m->cfg.max_symbols) { symbols = 0; i++; } /* frame exhausted: move on */
            break; /* later frames were scored with the old prediction: redo them */
        }
        t += i;
    }
    d->last_ms = now_ms() - t0;
    d->last_steps = steps;
    return n;
}
