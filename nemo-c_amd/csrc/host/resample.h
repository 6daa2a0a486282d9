/* Streaming windowed-sinc resampler to 16 kHz (host side, before the hot path).
 * Same filter family as the reference (src/resample.c): Blackman-windowed sinc with 16 zero
 * crossings at the lower of the two Nyquist rates, each output normalised by the kernel sum;
 * equal rates pass samples through unchanged. */
#ifndef NEMO_RESAMPLE_H
#define NEMO_RESAMPLE_H
#include <stddef.h>

typedef struct rsmp rsmp_t;
rsmp_t *rsmp_create(int in_rate, int out_rate);
void rsmp_destroy(rsmp_t *r);
size_t rsmp_process(rsmp_t *r, const float *in, size_t n, float *out, size_t out_max);
size_t rsmp_flush(rsmp_t *r, float *out, size_t out_max);

#endif
