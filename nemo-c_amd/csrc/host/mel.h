/* Streaming 128-bin log-mel front end on the host CPU (before the hot path).
 * Same signal chain as the reference (src/mel.h:1-13, src/mel.c): 16 kHz, pre-emphasis 0.97,
 * symmetric Hann(400) centred in a 512-point FFT, 10 ms hop, centred frames with reflect
 * padding, power spectrum, Slaney mel filterbank (128 bins), log(x + 2^-24). */
#ifndef NEMO_MEL_H
#define NEMO_MEL_H
#include <stddef.h>

#define MEL_SR 16000
#define MEL_NFFT 512
#define MEL_WIN 400
#define MEL_HOP 160
#define MEL_NMEL 128
#define MEL_NBIN (MEL_NFFT / 2 + 1)

typedef struct melfe melfe_t;

melfe_t *melfe_create(void);
void melfe_destroy(melfe_t *m);
/* Append n samples (n may be 0; final flushes the tail).  *frames points at the newly complete
 * frames (MEL_NMEL floats each), valid until the next call. */
void melfe_push(melfe_t *m, const float *x, size_t n, int final, const float **frames, size_t *nframes);
size_t melfe_samples(const melfe_t *m);
size_t melfe_frames(const melfe_t *m);

#endif
