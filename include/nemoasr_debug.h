/* Test and benchmark hooks of the nemoasr library.  No counterpart in the reference (whose
 * parity dumps come from CLI flags, src/main.c:209-211 and :99, :112, :128); they expose the
 * same artefacts per session: mel input injection, per-layer encoder outputs, post-prompt rows,
 * joint.enc rows and token ids, plus per-kernel timing. */
#ifndef NEMOASR_DEBUG_H
#define NEMOASR_DEBUG_H
#include "nemoasr.h"
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Queue log-mel frames (128 floats each) directly, bypassing resampler and front end; runs every
   ready chunk (all of them when final).  Returns new token count, -1 on error. */
int nemoasr_debug_feed_mel(nemoasr_t *s, const float *mel, size_t nframes, int final, char *err, size_t errlen);
/* All token ids emitted since open/reset. */
const int *nemoasr_debug_tokens(const nemoasr_t *s, size_t *n);
/* Keep per-chunk dumps: block outputs (frames x n_layers x d_model), prompted rows
   (frames x d_model), joint.enc rows (frames x joint_hidden).  Dumps disable graph replay. */
void nemoasr_debug_set_dump(nemoasr_t *s, int on);
size_t nemoasr_debug_frames(const nemoasr_t *s);
const float *nemoasr_debug_dump_layers(const nemoasr_t *s);
const float *nemoasr_debug_dump_prompted(const nemoasr_t *s);
const float *nemoasr_debug_dump_joint_enc(const nemoasr_t *s);
/* Log-mel frames (128 floats each) the front end produced from fed audio since open/reset while
   dumps were on (the reference CLI's --dump-mel, src/main.c:128). */
const float *nemoasr_debug_dump_mel(const nemoasr_t *s, size_t *nframes);
/* 0: launch every kernel directly; 1: replay chunks as hipGraphs (default). */
void nemoasr_debug_use_graphs(nemoasr_t *s, int on);
/* The graph setting of sessions opened from now on, their warm-up included (1 by default): 0 makes
 * every launch of the session a direct launch from its first (profilers that cannot follow graph
 * launches). */
void nemoasr_debug_default_graphs(int on);
/* 1 (default): chunks of at most two rows run attention + output projection and depthwise conv +
 * pointwise conv as one launch each; 0: the separate launches. */
void nemoasr_debug_fuse(nemoasr_t *s, int on);
/* 1 (default): one-row chunks run every conformer block in one persistent launch, where the
 * model shape and device allow it (nemoasr_debug_chain_usable); 0: the per-kernel sequence. */
void nemoasr_debug_chain(nemoasr_t *s, int on);
int nemoasr_debug_chain_usable(const nemoasr_t *s);
/* Polls a hand-off of the chain may spend before the launch gives up (0: the default, 2^20, about
 * half a second).  A launch that gives up ends every workgroup at its next barrier or wait and
 * leaves the session in error ("encoder chain: hand-off N timed out"); a tiny bound forces that
 * path (the failure-handling test).  Applies to the session's current latency. */
void nemoasr_debug_chain_spin(nemoasr_t *s, unsigned spin_max);
/* Round trips of the decoder since open/reset, and GPU time of the encoder chunks (ms). */
size_t nemoasr_debug_joint_steps(const nemoasr_t *s);
double nemoasr_debug_encoder_gpu_ms(const nemoasr_t *s);
/* Wall ms of every chunk (encoder step + its decoder round trips) since open/reset. */
const double *nemoasr_debug_chunk_ms(const nemoasr_t *s, size_t *n);
/* Time every launch of `kernel` on the stream with hipEvents (direct launches only);
   collect returns the mean duration (ms) and the launch count since the last collect. */
int nemoasr_debug_time_kernel(nemoasr_t *s, const char *kernel, int max_launches);
int nemoasr_debug_kernel_ms(nemoasr_t *s, double *mean_ms, int *count, double *bytes);
/* Bytes of bf16 weights resident in HBM (the per-chunk streamed set plus decoder weights). */
size_t nemoasr_debug_weight_bytes(const nemoasr_t *s);
uint64_t nemoasr_debug_launches(const nemoasr_t *s);

#ifdef __cplusplus
}
#endif
#endif
