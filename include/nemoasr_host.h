/* Host-side pieces of the streaming path exported for CPU tests (no GPU needed):
 *   melfe_*        streaming log-mel front end       (reference src/mel.h:17-23)
 *   rsmp_*         streaming resampler               (reference src/resample.h:9-11)
 *   nemo_enc_plan  encoder step bookkeeping          (reference src/encoder.c:213-251)
 *   nemo_piece_text  token piece -> text             (reference src/tokenizer.c:34-50) */
#ifndef NEMOASR_HOST_H
#define NEMOASR_HOST_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct melfe melfe_t;
melfe_t *melfe_create(void);
void melfe_destroy(melfe_t *m);
void melfe_push(melfe_t *m, const float *x, size_t n, int final, const float **frames, size_t *nframes);
size_t melfe_samples(const melfe_t *m);
size_t melfe_frames(const melfe_t *m);

typedef struct rsmp rsmp_t;
rsmp_t *rsmp_create(int in_rate, int out_rate);
void rsmp_destroy(rsmp_t *r);
size_t rsmp_process(rsmp_t *r, const float *in, size_t n, float *out, size_t out_max);
size_t rsmp_flush(rsmp_t *r, float *out, size_t out_max);

/* state: [pending_n, consumed, emitted] in/out; flags: [mel_cache_n, closed] in/out.
 * plan receives {ran, take, nwin, lo, hi, c, include_boundary, T3}; returns ran. */
int nemo_enc_plan(int *plan, size_t pending_n, size_t consumed, size_t emitted, int mel_cache_n, int closed, int final,
                  int chunk_mel, int subsampling, int mel_cache, int *state_out);
/* Text of one vocabulary piece: 0 and the text in out, or -1 if out is too small. */
int nemo_piece_text(const char *piece, size_t unused, char *out, size_t outlen);

#ifdef __cplusplus
}
#endif
#endif
