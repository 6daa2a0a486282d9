/* nemoasr multi-stream batching on one MI355X.  No counterpart in the reference, which decodes
 * one stream per session (src/nemoasr.h:15-54); these symbols are additive and the single-stream
 * API is unchanged.
 *
 * A batch holds n_streams independent streams on one loaded model (same language prompt and
 * latency for all).  Audio (or log-mel frames) is pushed per stream; nemoasr_batch_step() then
 * runs every encoder chunk that is ready across the streams as ONE batched encoder step (the
 * streams' rows stacked into each GEMM; attention, depthwise conv and the caches indexed per
 * stream) followed by the RNNT greedy loop of all those chunks together (one batched LSTM and
 * joint evaluation per step of the loop).  Each stream follows the reference's streaming rules
 * (src/encoder.c:213-251, src/decoder.c:92-127) exactly: its tokens equal what a single-stream
 * session would emit for the same audio.
 * Not thread-safe: call all functions of one batch on one thread. */
#ifndef NEMOASR_BATCH_H
#define NEMOASR_BATCH_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nemoasr_batch nemoasr_batch_t;

typedef struct {
    size_t steps;          /* batched encoder steps run               */
    size_t chunks;         /* stream chunks encoded (sum over steps)   */
    size_t rows;           /* encoder rows (frames) over all chunks    */
    size_t joint_steps;    /* batched joint evaluations                */
    size_t tokens;
    double frontend_ms;    /* wall time of the host log-mel front end  */
    double encoder_ms, decoder_ms; /* wall time of the two phases     */
    double encoder_gpu_ms; /* GPU time of the encoder steps (hipEvents) */
} nemoasr_batch_stats_t;

/* Load the model and allocate n_streams streams (caches for all of them live in HBM).
   latency_ms: 80, 160, 320, 560 or 1120; audio is pushed at 16 kHz. */
nemoasr_batch_t *nemoasr_batch_open(const char *model_dir, const char *language, int latency_ms, int n_streams,
                                    char *err, size_t errlen);
void nemoasr_batch_close(nemoasr_batch_t *b);
int nemoasr_batch_streams(const nemoasr_batch_t *b);

/* Queue 16 kHz mono audio for one stream (log-mel computed on the host).  final = 1 ends it. */
int nemoasr_batch_push(nemoasr_batch_t *b, int stream, const float *samples, size_t n, int final, char *err,
                       size_t errlen);
/* Queue log-mel frames (128 floats each) for one stream directly. */
int nemoasr_batch_push_mel(nemoasr_batch_t *b, int stream, const float *mel, size_t nframes, int final, char *err,
                           size_t errlen);
/* One batched step over every stream with a ready chunk.  Returns the number of streams that
   consumed input (0: nothing ready), -1 on error. */
int nemoasr_batch_step(nemoasr_batch_t *b, char *err, size_t errlen);
/* Steps until no stream has a ready chunk; returns the number of steps run, -1 on error. */
int nemoasr_batch_run(nemoasr_batch_t *b, char *err, size_t errlen);

/* Token ids emitted so far by one stream. */
const int *nemoasr_batch_tokens(const nemoasr_batch_t *b, int stream, size_t *n);
/* Text of the tokens not yet returned for one stream (malloc'd, free with nemoasr_free) or NULL. */
char *nemoasr_batch_text(nemoasr_batch_t *b, int stream);
/* Start a fresh stream in slot `stream` (caches, decoder state, queued input and tokens cleared). */
int nemoasr_batch_reset_stream(nemoasr_batch_t *b, int stream, char *err, size_t errlen);
void nemoasr_batch_stats(const nemoasr_batch_t *b, nemoasr_batch_stats_t *out);
/* Wall ms of every batched step (encoder step + its decoder loop) since open. */
const double *nemoasr_batch_step_ms(const nemoasr_batch_t *b, size_t *n);

/* Test hooks: 0 launches every encoder step directly instead of replaying captured hipGraphs;
   set_dump(1) keeps every stream's joint.enc rows (the joint's encoder input) on the host. */
void nemoasr_batch_debug_use_graphs(nemoasr_batch_t *b, int on);
void nemoasr_batch_debug_set_dump(nemoasr_batch_t *b, int on);
/* 1 (default): the greedy loop runs on the device, graph-replayed runs of steps; 0: one host round
   trip per joint evaluation.  The two keep their greedy state apart, so only before any input;
   returns -1 afterwards. */
int nemoasr_batch_debug_device_decoder(nemoasr_batch_t *b, int on);
/* 1 (default): log-mel on the GPU (frames computed when a window takes them, kept in per-stream
   device rings; within one stream audio and mel input cannot be mixed); 0: on the host's threads.
   Only before any input; returns -1 afterwards. */
int nemoasr_batch_debug_gpu_frontend(nemoasr_batch_t *b, int on);
const float *nemoasr_batch_debug_joint_enc(const nemoasr_batch_t *b, int stream, size_t *frames);
/* Per-kernel timing of direct launches (kernel: exact name or a prefix ending in '*'): mean ms per
   launch, launches, and the summed algorithmic bytes and flops of those launches. */
int nemoasr_batch_debug_time_kernel(nemoasr_batch_t *b, const char *kernel, int max_launches);
int nemoasr_batch_debug_kernel_ms(nemoasr_batch_t *b, double *mean_ms, int *count, double *bytes, double *flops);

#ifdef __cplusplus
}
#endif
#endif
