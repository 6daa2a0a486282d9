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

/* melfe_push in three parts, for front ends that compute the frames elsewhere (the batched GPU
 * front end):
 *   melfe_append  appends n samples (final flushes the tail) and returns how many complete frames
 *                 are waiting to be taken;
 *   melfe_take    writes the pre-emphasised samples the first cnt = min(kmax, waiting) frames read
 *                 (melfe_span_len(cnt) floats: frame t reads span[t*MEL_HOP .. t*MEL_HOP + MEL_NFFT),
 *                 reflection at both ends applied), marks them taken and returns cnt;
 *   melfe_compute turns cnt frames of a span into log-mel rows (the host computation). */
size_t melfe_append(melfe_t *m, const float *x, size_t n, int final);
size_t melfe_span_len(size_t cnt);
size_t melfe_take(melfe_t *m, float *span, size_t kmax);
void melfe_compute(const melfe_t *m, const float *span, size_t cnt, float *out);

/* The front end's constant tables (identical for every instance): window [MEL_NFFT], filterbank
 * [MEL_NMEL][MEL_NBIN] with each filter's nonzero bin range [fb_lo, fb_hi), FFT twiddles
 * e^{-2 pi i k / MEL_NFFT} for k < MEL_NFFT/2 (double), bit-reversal permutation [MEL_NFFT]. */
typedef struct {
    const float *win, *fb;
    const int *fb_lo, *fb_hi;
    const double *tw_re, *tw_im;
    const unsigned short *rev;
} melfe_tables_t;
void melfe_tables(const melfe_t *m, melfe_tables_t *t);

#endif
