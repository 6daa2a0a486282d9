/* Public session API (include/nemoasr.h) on the HIP backend, plus the test hooks of
 * include/nemoasr_debug.h.
 *
 * A session moves audio through three stages:
 *   input   the caller's samples, resampled to 16 kHz when the caller's rate differs (rsmp_*);
 *   frames  streaming log-mel rows (melfe_*), queued as the encoder's pending rows;
 *   chunks  every encoder step that is ready, whose joint.enc rows the greedy loop decodes.
 * Token text collects in an output buffer whose ownership passes to the caller on each feed.
 * The observable behaviour is the reference's (src/nemoasr.c:58-196): the latency -> right context
 * table, language prompt, warm-up at open, feed / final flush, reset, leading spaces dropped from
 * the stream's first text. */
#include "nemoasr.h"
#include "nemoasr_debug.h"
#include "decoder.h"
#include "encoder.h"
#include "mel.h"
#include "model.h"
#include "resample.h"
#include <glob.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* graph replay for sessions opened from now on (warm-up included); nemoasr_debug_default_graphs */
static int g_default_graphs = 1;

#define TOKENS_PER_CHUNK_MAX 4096

static double clock_ms(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return 1e3 * (double)t.tv_sec + 1e-6 * (double)t.tv_nsec;
}

/* Grow *buf (element size esz) to hold at least `need` elements; 0 on success. */
static int reserve(void **buf, size_t *cap, size_t need, size_t esz) {
    if (need <= *cap) return 0;
    size_t n = *cap ? *cap : 64;
    while (n < need) n *= 2;
    void *p = realloc(*buf, n * esz);
    if (!p) return -1;
    *buf = p;
    *cap = n;
    return 0;
}

static void set_err(char *err, size_t errlen, const char *fmt, ...) {
    if (!errlen) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

/* chunk latency -> attention right context, the checkpoint's trained settings */
static const struct { int ms, right; } k_latency[] = { { 80, 0 }, { 160, 1 }, { 320, 3 }, { 560, 6 }, { 1120, 13 } };

static int latency_right(int ms) {
    for (size_t i = 0; i < sizeof k_latency / sizeof k_latency[0]; ++i)
        if (k_latency[i].ms == ms) return k_latency[i].right;
    return -1;
}

/* A latency the session can run: a known setting that the checkpoint was trained for. */
static int check_latency(const model_t *m, int ms, char *err, size_t errlen) {
    const int r = latency_right(ms);
    if (r < 0) {
        set_err(err, errlen, "unsupported latency %d ms (one of 80, 160, 320, 560, 1120)", ms);
        return -1;
    }
    if (m && !model_right_context_trained(m, r)) {
        set_err(err, errlen, "the checkpoint has no trained context for %d ms chunks", ms);
        return -1;
    }
    return r;
}

#define N_LATENCIES (int)(sizeof k_latency / sizeof k_latency[0])

struct nemoasr {
    model_t *m;
    encoder_t *enc;               /* the current latency's, one of encs  */
    encoder_t *encs[N_LATENCIES]; /* by latency index: prepared encoders */
    decoder_t *dec;
    struct { /* input stage */
        int rate;
        rsmp_t *rs;  /* NULL at 16 kHz */
        float *buf;  /* resampled samples of one feed */
        size_t cap;
        melfe_t *mel;
    } in;
    struct { /* text handed out by the next feed */
        char *p;
        size_t len, cap;
        int started; /* a non-space character has been emitted since open / reset */
    } out;
    struct { /* records since open / reset (stats and test hooks) */
        int *ids;
        size_t nids, capids;
        double *chunk_ms;
        size_t nchunk, capchunk;
        size_t joint_steps;
        double enc_gpu_ms;
        float *mel;
        size_t nmel, capmel;
    } rec;
    nemoasr_stats_t stats;
    int latency_ms, done, dump, graphs, fuse, chain;
    unsigned warm; /* bit r: chunk shapes of right context r have run once */
    double open_ms;
    int ids[TOKENS_PER_CHUNK_MAX];
};

/* The mlx-community/nemotron-3.5-asr-streaming-0.6b snapshot in the Hugging Face cache: the first
 * snapshot directory (in name order) that holds model.safetensors. */
int nemoasr_default_model_dir(char *out, size_t n) {
    const char *home = getenv("HOME");
    char pat[1200];
    snprintf(pat, sizeof pat,
             "%s/.cache/huggingface/hub/models--mlx-community--nemotron-3.5-asr-streaming-0.6b/snapshots/*/model.safetensors",
             home ? home : ".");
    glob_t g;
    if (glob(pat, 0, NULL, &g) != 0 || g.gl_pathc == 0) {
        globfree(&g);
        return -1;
    }
    const char *hit = g.gl_pathv[0];
    const size_t dirlen = strlen(hit) - strlen("/model.safetensors");
    const int ok = dirlen < n;
    if (ok) snprintf(out, n, "%.*s", (int)dirlen, hit);
    globfree(&g);
    return ok ? 0 : -1;
}

static int latency_index(int right) {
    for (int i = 0; i < N_LATENCIES; ++i)
        if (k_latency[i].right == right) return i;
    return -1;
}

/* The session's encoder for a right context (created on first use), with the session's settings. */
static encoder_t *encoder_for(nemoasr_t *s, int right) {
    const int i = latency_index(right);
    if (i < 0) return NULL;
    if (!s->encs[i]) s->encs[i] = encoder_create(s->m, right);
    encoder_t *e = s->encs[i];
    if (e) {
        encoder_set_dump(e, s->dump);
        encoder_use_graphs(e, s->graphs);
        encoder_fuse(e, s->fuse);
        encoder_chain(e, s->chain && encoder_chain_usable(e));
    }
    return e;
}

/* Warm-up, as the reference's (src/warmup.c:23-42): silence through an encoder of this right
 * context and a throwaway decoder, so that every kernel is loaded and the scratch sized.  Here the
 * encoder is the session's own for that right context (kept for later resets to it), which
 * captures each chunk shape's hipGraph on first sight (the first chunk's window and the steady
 * window: at least 1.5 s and three chunks of zeros), and the session's decoder captures, without
 * running them, its graphs of every run size for that encoder's joint.enc rows.  The encoder then
 * returns to its start state; the session's decoder state is not touched (a stream in progress at
 * another latency goes on undisturbed).  Errors are not fatal. */
static void warm_up(nemoasr_t *s, int right) {
    encoder_t *e = encoder_for(s, right);
    decoder_t *d = decoder_create(s->m);
    melfe_t *fe = melfe_create();
    if (e && d && fe) {
        const size_t need = (size_t)(3 * encoder_chunk_mel(e) + 32) * 160, n = need > 24000 ? need : 24000;
        float *silence = calloc(n, sizeof(float));
        const float *rows, *joint_enc = NULL;
        size_t nrows;
        char scratch[256];
        int ids[256];
        if (silence) {
            encoder_capture_first(e, 1);
            melfe_push(fe, silence, n, 1, &rows, &nrows);
            encoder_push(e, rows, nrows);
            enc_out_t o;
            while (encoder_step(e, 1, &o, scratch, sizeof scratch) == 1) {
                if (o.frames > 0) {
                    joint_enc = o.joint_enc;
                    if (decoder_run(d, o.joint_enc, o.frames, ids, 256, scratch, sizeof scratch) < 0) break;
                }
                encoder_take_gpu_ms(e);
            }
            encoder_capture_first(e, 0);
            if (joint_enc && s->dec) decoder_prepare_graphs(s->dec, joint_enc);
        }
        free(silence);
    }
    melfe_destroy(fe);
    decoder_destroy(d);
    if (e) encoder_reset(e);
}

/* Fresh front end and empty records (open and reset). */
static int begin_stream(nemoasr_t *s) {
    melfe_destroy(s->in.mel);
    rsmp_destroy(s->in.rs);
    s->in.mel = melfe_create();
    s->in.rs = s->in.rate != MEL_SR ? rsmp_create(s->in.rate, MEL_SR) : NULL;
    free(s->out.p);
    s->out.p = NULL;
    s->out.len = s->out.cap = 0;
    s->out.started = 0;
    s->rec.nids = s->rec.nchunk = s->rec.nmel = 0;
    s->rec.joint_steps = 0;
    s->rec.enc_gpu_ms = 0.0;
    memset(&s->stats, 0, sizeof s->stats);
    s->done = 0;
    return s->in.mel && (s->in.rate == MEL_SR || s->in.rs) ? 0 : -1;
}

nemoasr_t *nemoasr_open(const char *model_dir, const char *language, int latency_ms, int input_rate, char *err,
                        size_t errlen) {
    set_err(err, errlen, "%s", "");
    const double t0 = clock_ms();
    if (check_latency(NULL, latency_ms, err, errlen) < 0) return NULL;
    if (input_rate <= 0) {
        set_err(err, errlen, "input_rate must be > 0 (got %d)", input_rate);
        return NULL;
    }
    nemoasr_t *s = calloc(1, sizeof *s);
    if (!s) {
        set_err(err, errlen, "out of memory");
        return NULL;
    }
    s->in.rate = input_rate;
    s->latency_ms = latency_ms;
    if (!(s->m = model_load(model_dir, err, errlen))) {
        free(s);
        return NULL;
    }
    const int right = check_latency(s->m, latency_ms, err, errlen);
    if (right < 0 || model_set_language(s->m, language ? language : "auto", err, errlen)) {
        nemoasr_close(s);
        return NULL;
    }
    s->graphs = g_default_graphs;
    s->fuse = 1;
    s->chain = 1; /* one-row chunks run the persistent chain where the device and model allow it */
    s->dec = decoder_create(s->m);
    if (s->dec) decoder_use_graphs(s->dec, s->graphs);
    if (s->dec) warm_up(s, right);
    s->warm = 1u << right;
    s->enc = encoder_for(s, right);
    if (!s->enc || !s->dec || begin_stream(s)) {
        set_err(err, errlen, "session setup on the GPU failed: %s", gpu_last_error(s->m->gpu));
        nemoasr_close(s);
        return NULL;
    }
    set_err(err, errlen, "%s", "");
    s->open_ms = clock_ms() - t0;
    return s;
}

void nemoasr_close(nemoasr_t *s) {
    if (!s) return;
    for (int i = 0; i < N_LATENCIES; ++i) encoder_destroy(s->encs[i]);
    decoder_destroy(s->dec);
    melfe_destroy(s->in.mel);
    rsmp_destroy(s->in.rs);
    model_free(s->m);
    free(s->in.buf);
    free(s->out.p);
    free(s->rec.ids);
    free(s->rec.chunk_ms);
    free(s->rec.mel);
    free(s);
}

/* Token text into the output buffer; the stream's first text loses its leading spaces. */
static int emit_text(nemoasr_t *s, int id) {
    char *piece = piece_text(&s->m->vocab, id);
    if (!piece) return -1;
    const char *t = piece;
    if (!s->out.started) t += strspn(t, " ");
    const size_t n = strlen(t);
    int rc = 0;
    if (n) {
        if (reserve((void **)&s->out.p, &s->out.cap, s->out.len + n + 1, 1)) rc = -1;
        else {
            memcpy(s->out.p + s->out.len, t, n + 1);
            s->out.len += n;
            s->out.started = 1;
        }
    }
    free(piece);
    return rc;
}

/* Run every encoder step that is ready (all remaining ones when final) and decode each chunk's
 * frames.  Returns the number of new tokens, or -1 with err set. */
static int drain_chunks(nemoasr_t *s, int final, char *err, size_t errlen) {
    int fresh = 0;
    for (;;) {
        enc_out_t o;
        const int rc = encoder_step(s->enc, final, &o, err, errlen);
        if (rc < 0) return -1;
        if (rc == 0) return fresh;
        if (o.frames <= 0) {
            o.gpu_ms += encoder_take_gpu_ms(s->enc);
            continue;
        }
        /* the decoder's work queues behind the encoder's on the stream; its wall time includes
         * the wait for the encoder, whose GPU time is moved to the encoder's account */
        const double t0 = clock_ms();
        const int n = decoder_run(s->dec, o.joint_enc, o.frames, s->ids, TOKENS_PER_CHUNK_MAX, err, errlen);
        const double enc_gpu = encoder_take_gpu_ms(s->enc);
        o.gpu_ms += enc_gpu;
        if (n < 0) return -1;
        if (encoder_check(s->enc, err, errlen)) return -1;
        if (reserve((void **)&s->rec.ids, &s->rec.capids, s->rec.nids + (size_t)n, sizeof(int)) ||
            reserve((void **)&s->rec.chunk_ms, &s->rec.capchunk, s->rec.nchunk + 1, sizeof(double))) {
            set_err(err, errlen, "out of memory");
            return -1;
        }
        for (int i = 0; i < n; ++i)
            if (emit_text(s, s->ids[i])) {
                set_err(err, errlen, "out of memory");
                return -1;
            }
        memcpy(s->rec.ids + s->rec.nids, s->ids, (size_t)n * sizeof(int));
        s->rec.nids += (size_t)n;
        s->rec.chunk_ms[s->rec.nchunk++] = o.wall_ms + (clock_ms() - t0);
        s->rec.joint_steps += (size_t)decoder_last_steps(s->dec);
        s->rec.enc_gpu_ms += o.gpu_ms;
        s->stats.chunks += 1;
        s->stats.tokens += (size_t)n;
        const double dec_ms = decoder_last_ms(s->dec);
        s->stats.encoder_ms += o.wall_ms + (enc_gpu < dec_ms ? enc_gpu : dec_ms);
        s->stats.decoder_ms += dec_ms > enc_gpu ? dec_ms - enc_gpu : 0.0;
        fresh += n;
    }
}

char *nemoasr_feed(nemoasr_t *s, const float *samples, size_t n, int final, char *err, size_t errlen) {
    set_err(err, errlen, "%s", "");
    if (s->done) return NULL;
    const float *x = samples;
    size_t cnt = n;
    if (s->in.rs) { /* to 16 kHz, plus the filter's tail when the stream ends */
        const size_t most = (size_t)((double)n * MEL_SR / s->in.rate) + 4096;
        if (reserve((void **)&s->in.buf, &s->in.cap, most, sizeof(float))) {
            set_err(err, errlen, "out of memory");
            return NULL;
        }
        cnt = n ? rsmp_process(s->in.rs, samples, n, s->in.buf, s->in.cap) : 0;
        if (final) cnt += rsmp_flush(s->in.rs, s->in.buf + cnt, s->in.cap - cnt);
        x = s->in.buf;
    }
    s->stats.audio_seconds += (double)cnt / MEL_SR;
    /* a final call on a stream that never received a sample has nothing to flush */
    const int nothing = final && cnt == 0 && melfe_samples(s->in.mel) == 0;
    if (!nothing) {
        const float *rows;
        size_t nrows;
        melfe_push(s->in.mel, x, cnt, final, &rows, &nrows);
        if (nrows && s->dump) {
            if (reserve((void **)&s->rec.mel, &s->rec.capmel, (s->rec.nmel + nrows) * MEL_NMEL, sizeof(float))) {
                set_err(err, errlen, "out of memory");
                return NULL;
            }
            memcpy(s->rec.mel + s->rec.nmel * MEL_NMEL, rows, nrows * MEL_NMEL * sizeof(float));
            s->rec.nmel += nrows;
        }
        if (nrows) encoder_push(s->enc, rows, nrows);
        if (drain_chunks(s, final, err, errlen) < 0) return NULL;
    }
    if (final) s->done = 1;
    if (!s->out.len) return NULL;
    char *text = s->out.p; /* ownership moves to the caller */
    s->out.p = NULL;
    s->out.len = s->out.cap = 0;
    return text;
}

void nemoasr_free(char *text) { free(text); }

int nemoasr_prepare_latency(nemoasr_t *s, int latency_ms, char *err, size_t errlen) {
    set_err(err, errlen, "%s", "");
    const int right = check_latency(s->m, latency_ms, err, errlen);
    if (right < 0) return -1;
    if (!(s->warm & (1u << right))) {
        warm_up(s, right);
        s->warm |= 1u << right;
        if (!s->encs[latency_index(right)]) {
            set_err(err, errlen, "encoder setup on the GPU failed: %s", gpu_last_error(s->m->gpu));
            return -1;
        }
    }
    return 0;
}

int nemoasr_reset(nemoasr_t *s, const char *language, int latency_ms, char *err, size_t errlen) {
    if (nemoasr_prepare_latency(s, latency_ms, err, errlen)) return -1;
    if (language && model_set_language(s->m, language, err, errlen)) return -1;
    const int right = latency_right(latency_ms);
    if (!(s->enc = encoder_for(s, right))) { /* the prepared encoder of this chunk shape */
        set_err(err, errlen, "encoder setup on the GPU failed: %s", gpu_last_error(s->m->gpu));
        s->done = 1;
        return -1;
    }
    encoder_reset(s->enc);
    decoder_reset(s->dec);
    s->latency_ms = latency_ms;
    if (begin_stream(s)) {
        set_err(err, errlen, "out of memory");
        s->done = 1;
        return -1;
    }
    return 0;
}

double nemoasr_load_ms(const nemoasr_t *s) { return s->open_ms; }
const char *nemoasr_gpu_name(const nemoasr_t *s) { return gpu_device_name(s->m->gpu); }
int nemoasr_latency_ms(const nemoasr_t *s) { return s->latency_ms; }
void nemoasr_stats(const nemoasr_t *s, nemoasr_stats_t *out) { *out = s->stats; }

/* ---- test hooks ---------------------------------------------------------------------------- */
int nemoasr_debug_feed_mel(nemoasr_t *s, const float *mel, size_t nframes, int final, char *err, size_t errlen) {
    set_err(err, errlen, "%s", "");
    if (nframes) encoder_push(s->enc, mel, nframes);
    return drain_chunks(s, final, err, errlen);
}
const int *nemoasr_debug_tokens(const nemoasr_t *s, size_t *n) {
    *n = s->rec.nids;
    return s->rec.ids;
}
void nemoasr_debug_set_dump(nemoasr_t *s, int on) {
    s->dump = on;
    encoder_set_dump(s->enc, on);
}
const float *nemoasr_debug_dump_mel(const nemoasr_t *s, size_t *nframes) {
    *nframes = s->rec.nmel;
    return s->rec.mel;
}
size_t nemoasr_debug_frames(const nemoasr_t *s) { return encoder_dump_frames(s->enc); }
const float *nemoasr_debug_dump_layers(const nemoasr_t *s) { return encoder_dump_layers(s->enc); }
const float *nemoasr_debug_dump_prompted(const nemoasr_t *s) { return encoder_dump_prompted(s->enc); }
const float *nemoasr_debug_dump_joint_enc(const nemoasr_t *s) { return encoder_dump_joint(s->enc); }
void nemoasr_debug_default_graphs(int on) { g_default_graphs = on != 0; }
void nemoasr_debug_use_graphs(nemoasr_t *s, int on) {
    s->graphs = on != 0;
    encoder_use_graphs(s->enc, on);
    decoder_use_graphs(s->dec, on);
}
void nemoasr_debug_fuse(nemoasr_t *s, int on) {
    s->fuse = on != 0;
    encoder_fuse(s->enc, on);
}
void nemoasr_debug_chain(nemoasr_t *s, int on) {
    s->chain = on != 0;
    encoder_chain(s->enc, s->chain && encoder_chain_usable(s->enc));
}
int nemoasr_debug_chain_usable(const nemoasr_t *s) { return encoder_chain_usable(s->enc); }
void nemoasr_debug_chain_spin(nemoasr_t *s, unsigned spin_max) { encoder_chain_spin(s->enc, spin_max); }
size_t nemoasr_debug_joint_steps(const nemoasr_t *s) { return s->rec.joint_steps; }
double nemoasr_debug_encoder_gpu_ms(const nemoasr_t *s) { return s->rec.enc_gpu_ms; }
const double *nemoasr_debug_chunk_ms(const nemoasr_t *s, size_t *n) {
    *n = s->rec.nchunk;
    return s->rec.chunk_ms;
}
int nemoasr_debug_time_kernel(nemoasr_t *s, const char *kernel, int max_launches) {
    return gpu_timing_set(s->m->gpu, kernel, max_launches);
}
int nemoasr_debug_kernel_ms(nemoasr_t *s, double *mean_ms, int *count, double *bytes) {
    return gpu_timing_collect(s->m->gpu, mean_ms, count, bytes);
}
size_t nemoasr_debug_weight_bytes(const nemoasr_t *s) { return s->m->warena_bytes; }
uint64_t nemoasr_debug_launches(const nemoasr_t *s) { return gpu_launch_count(s->m->gpu); }
