/* Greedy RNN-T decoding (2-layer LSTM prediction network + joint), one encoder chunk at a time.
 * Same interface and loop as the reference (src/decoder.h:1-16, src/decoder.c:92-127). */
#ifndef NEMO_DECODER_H
#define NEMO_DECODER_H
#include "model.h"

typedef struct decoder decoder_t;

decoder_t *decoder_create(model_t *m);
void decoder_destroy(decoder_t *d);
void decoder_reset(decoder_t *d);
/* Decode `frames` rows of joint_enc (device [frames][joint_hidden]); appends token ids to out.
 * Returns the count, or -1 on error. */
int decoder_run(decoder_t *d, const float *joint_enc, int frames, int *out, int max_out, char *err, size_t errlen);
double decoder_last_ms(const decoder_t *d);
/* 1 (default): replay each run of steps from a captured hipGraph; 0: launch every kernel directly */
void decoder_use_graphs(decoder_t *d, int on);
int decoder_last_steps(const decoder_t *d); /* joint evaluations (round trips) in the last run */
/* Capture (without running) the graphs of every run size for joint.enc rows at joint_enc; returns
 * the number of graphs held for it. */
int decoder_prepare_graphs(decoder_t *d, const float *joint_enc);

#endif
