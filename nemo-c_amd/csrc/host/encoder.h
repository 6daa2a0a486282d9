/* Cache-aware streaming FastConformer encoder + language prompt + joint encoder projection.
 * Same interface and bookkeeping as the reference (src/encoder.h:1-29, src/encoder.c). */
#ifndef NEMO_ENCODER_H
#define NEMO_ENCODER_H
#include "model.h"

typedef struct encoder encoder_t;

typedef struct {
    int frames;              /* encoder frames produced by this step (may be 0) */
    const float *prompted;   /* device [frames][d_model] post-prompt encoder output */
    const float *joint_enc;  /* device [frames][joint_hidden] joint.enc projection */
    double gpu_ms, wall_ms;
} enc_out_t;

encoder_t *encoder_create(model_t *m, int right_context);
void encoder_destroy(encoder_t *e);
void encoder_reset(encoder_t *e);
int encoder_right(const encoder_t *e);
int encoder_chunk_frames(const encoder_t *e);
int encoder_chunk_mel(const encoder_t *e);
void encoder_push(encoder_t *e, const float *mel, size_t nframes);
/* 1: a piece was consumed (out->frames may be 0); 0: nothing to do; -1: error in err.
 * Unless dumps are on, the step's GPU work is queued without waiting for it (the decoder's work
 * queues behind it on the same stream): out->gpu_ms is then 0 and encoder_take_gpu_ms returns the
 * step's GPU time, waiting for it. */
int encoder_step(encoder_t *e, int final, enc_out_t *out, char *err, size_t errlen);
double encoder_take_gpu_ms(encoder_t *e);

/* Replay each chunk shape as a captured hipGraph (default on). */
void encoder_use_graphs(encoder_t *e, int on);
/* 1: capture a chunk shape's graph on its first chunk (warm-up); 0 (default): on its second, so a
 * shape seen once (a stream's last, boundary chunk) costs no capture. */
void encoder_capture_first(encoder_t *e, int on);
/* Chunk shapes with a captured graph. */
int encoder_graphs(const encoder_t *e);
/* 1 (default): fused attention + out_proj and dwconv + pw2 launches for chunks of few rows. */
void encoder_fuse(encoder_t *e, int on);
/* 1 (default where usable): one-row chunks run all conformer blocks as one persistent launch;
 * 0: the per-kernel sequence.  Usable for the d_model 1024 / d_ff 4096 / 8-head shape on a device
 * with at least 256 compute units. */
void encoder_chain(encoder_t *e, int on);
int encoder_chain_usable(const encoder_t *e);
/* Polls a chain hand-off may spend before it gives up (0: the default, 2^20, about half a second). */
void encoder_chain_spin(encoder_t *e, uint32_t spin_max);
/* -1 with err set when a chain launch reported a time-out (checked after the stream has synced). */
int encoder_check(encoder_t *e, char *err, size_t errlen);
/* Keep per-layer block outputs of every chunk (test hook). */
void encoder_set_dump(encoder_t *e, int on);
size_t encoder_dump_frames(const encoder_t *e);
const float *encoder_dump_layers(const encoder_t *e);   /* frames x n_layers x d_model */
const float *encoder_dump_prompted(const encoder_t *e); /* frames x d_model */
const float *encoder_dump_joint(const encoder_t *e);    /* frames x joint_hidden */

/* Bookkeeping of one step (src/encoder.c:213-251), exposed for host-side tests. */
typedef struct {
    size_t pending_n, consumed, emitted;
    int mel_cache_n, closed;
} enc_book_t;
typedef struct {
    int ran, take, nwin, lo, hi, c, include_boundary, T3;
} enc_plan_t;
enc_plan_t enc_plan_step(enc_book_t *b, int final, int chunk_mel, int subsampling, int mel_cache);

#endif
