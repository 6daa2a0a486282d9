/* Library API (include/nemoasr.h): the reference's src/nemoasr.c:1-202 behaviour on the HIP
 * backend, plus the test hooks of include/nemoasr_debug.h. */
#include "nemoasr.h"
#include "nemoasr_debug.h"
#include "decoder.h"
#include "encoder.h"
#include "mel.h"
#include "model.h"
#include "resample.h"
#include <dirent.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec / 1e6;
}

struct nemoasr {
    model_t *m;
    encoder_t *enc;
    decoder_t *dec;
    melfe_t *mel;
    rsmp_t *rs;
    int input_rate, latency_ms, finished, printed_any;
    unsigned warmed;
    float *tmp;
    size_t tmp_cap;
    char *text;
    size_t text_len, text_cap;
    int tokbuf[4096];
    int *all_tok;
    size_t n_tok, cap_tok;
    double *chunk_ms;
    size_t n_chunk, cap_chunk;
    size_t joint_steps;
    double enc_gpu_ms;
    double load_ms;
    nemoasr_stats_t stats;
    /* test hook: the front end's log-mel frames since open/reset, kept while dumps are on */
    int dump;
    float *mel_dump;
    size_t n_mel_dump, cap_mel_dump;
};

int nemoasr_default_model_dir(char *out, size_t n) {
    const char *home = getenv("HOME");
    char snaps[1024];
    snprintf(snaps, sizeof snaps, "%s/.cache/huggingface/hub/models--mlx-community--nemotron-3.5-asr-streaming-0.6b/snapshots",
             home ? home : ".");
    DIR *d = opendir(snaps);
    if (!d) return -1;
    struct dirent *ent;
    int found = 0;
    while (!found && (ent = readdir(d))) {
        if (ent->d_name[0] == '.') continue;
        snprintf(out, n, "%s/%s", snaps, ent->d_name);
        char probe[1400];
        snprintf(probe, sizeof probe, "%s/model.safetensors", out);
        struct stat sb;
        found = stat(probe, &sb) == 0;
    }
    closedir(d);
    return found ? 0 : -1;
}

/* latency -> right context (src/nemoasr.c:58-64) */
static int right_for(int latency_ms) {
    static const int ms[] = { 80, 160, 320, 560, 1120 }, r[] = { 0, 1, 3, 6, 13 };
    for (size_t i = 0; i < sizeof ms / sizeof *ms; ++i)
        if (ms[i] == latency_ms) return r[i];
    return -1;
}

/* Run zeros through a throwaway encoder/decoder so the first real chunk finds every kernel
 * loaded and the split-K scratch allocated (the reference's asr_warmup, src/warmup.c:23-42). */
static void warmup(model_t *m, int right, char *err, size_t errlen) {
    encoder_t *e = encoder_create(m, right);
    decoder_t *d = decoder_create(m);
    if (!e || !d) {
        decoder_destroy(d);
        encoder_destroy(e);
        return;
    }
    melfe_t *ms = melfe_create();
    static const float zeros[1600];
    int tok[64];
    for (int i = 0; i < 15; ++i) {
        const float *fr;
        size_t nf;
        melfe_push(ms, zeros, 1600, i == 14, &fr, &nf);
        encoder_push(e, fr, nf);
        enc_out_t out;
        while (encoder_step(e, i == 14, &out, err, errlen) == 1)
            if (out.frames > 0) decoder_run(d, out.joint_enc, out.frames, tok, 64, err, errlen);
    }
    melfe_destroy(ms);
    decoder_destroy(d);
    encoder_destroy(e);
}

nemoasr_t *nemoasr_open(const char *model_dir, const char *language, int latency_ms, int input_rate, char *err, size_t errlen) {
    if (errlen) err[0] = 0;
    const int right = right_for(latency_ms);
    if (right < 0) { snprintf(err, errlen, "latency must be one of 80, 160, 320, 560, 1120 ms"); return NULL; }
    if (input_rate <= 0) { snprintf(err, errlen, "input_rate must be positive"); return NULL; }
    const double t0 = now_ms();
    nemoasr_t *s = calloc(1, sizeof *s);
    s->m = model_load(model_dir, err, errlen);
    if (!s->m) { free(s); return NULL; }
    if (!model_right_context_trained(s->m, right)) {
        snprintf(err, errlen, "latency %d ms not trained for this checkpoint", latency_ms);
        nemoasr_close(s);
        return NULL;
    }
    if (model_set_language(s->m, language ? language : "auto", err, errlen)) { nemoasr_close(s); return NULL; }
    warmup(s->m, right, err, errlen);
    if (errlen) err[0] = 0;
    s->warmed = 1u << right;
    s->enc = encoder_create(s->m, right);
    s->dec = decoder_create(s->m);
    s->mel = melfe_create();
    if (!s->enc || !s->dec) {
        snprintf(err, errlen, "nemoasr_open: GPU setup failed: %s", gpu_last_error(s->m->gpu));
        nemoasr_close(s);
        return NULL;
    }
    s->input_rate = input_rate;
    s->latency_ms = latency_ms;
    if (input_rate != MEL_SR) s->rs = rsmp_create(input_rate, MEL_SR);
    s->load_ms = now_ms() - t0;
    return s;
}

void nemoasr_close(nemoasr_t *s) {
    if (!s) return;
    melfe_destroy(s->mel);
    decoder_destroy(s->dec);
    encoder_destroy(s->enc);
    rsmp_destroy(s->rs);
    model_free(s->m);
    free(s->tmp);
    free(s->text);
    free(s->all_tok);
    free(s->chunk_ms);
    free(s->mel_dump);
    free(s);
}

static void append_text(nemoasr_t *s, const char *t) {
    const size_t n = strlen(t);
    if (!n) return;
    if (s->text_len + n + 1 > s->text_cap) {
        s->text_cap = (s->text_len + n + 1) * 2;
        s->text = realloc(s->text, s->text_cap);
    }
    memcpy(s->text + s->text_len, t, n + 1);
    s->text_len += n;
}

static void keep_tokens(nemoasr_t *s, const int *t, int n) {
    if (s->n_tok + (size_t)n > s->cap_tok) {
        s->cap_tok = (s->n_tok + (size_t)n) * 2 + 256;
        s->all_tok = realloc(s->all_tok, s->cap_tok * sizeof(int));
    }
    memcpy(s->all_tok + s->n_tok, t, (size_t)n * sizeof(int));
    s->n_tok += (size_t)n;
}

/* every ready chunk: encoder step, then the decoder over its frames (src/nemoasr.c:112-132) */
static int run_pending(nemoasr_t *s, int final, int *new_tokens, char *err, size_t errlen) {
    enc_out_t out;
    int rc, total = 0;
    while ((rc = encoder_step(s->enc, final, &out, err, errlen)) == 1) {
        if (out.frames <= 0) continue;
        const double t0 = now_ms();
        s->stats.chunks++;
        s->stats.encoder_ms += out.wall_ms;
        s->enc_gpu_ms += out.gpu_ms;
        const int n = decoder_run(s->dec, out.joint_enc, out.frames, s->tokbuf, 4096, err, errlen);
        if (n < 0) return -1;
        s->stats.decoder_ms += decoder_last_ms(s->dec);
        s->joint_steps += (size_t)decoder_last_steps(s->dec);
        s->stats.tokens += (size_t)n;
        keep_tokens(s, s->tokbuf, n);
        total += n;
        for (int i = 0; i < n; ++i) {
            char *txt = piece_text(&s->m->vocab, s->tokbuf[i]);
            const char *p = txt;
            if (!s->printed_any) while (*p == ' ') p++;
            if (*p) { append_text(s, p); s->printed_any = 1; }
            free(txt);
        }
        if (s->n_chunk == s->cap_chunk) {
            s->cap_chunk = s->cap_chunk ? 2 * s->cap_chunk : 256;
            s->chunk_ms = realloc(s->chunk_ms, s->cap_chunk * sizeof(double));
        }
        s->chunk_ms[s->n_chunk++] = out.wall_ms + (now_ms() - t0);
    }
    if (new_tokens) *new_tokens = total;
    return rc;
}

char *nemoasr_feed(nemoasr_t *s, const float *samples, size_t n, int final, char *err, size_t errlen) {
    if (errlen) err[0] = 0;
    if (s->finished) return NULL;
    const float *in = samples;
    size_t count = n;
    if (s->rs) {
        const size_t need = (size_t)((double)n * MEL_SR / s->input_rate) + 4096;
        if (need > s->tmp_cap) {
            s->tmp_cap = need * 2;
            s->tmp = realloc(s->tmp, s->tmp_cap * sizeof(float));
        }
        count = n ? rsmp_process(s->rs, samples, n, s->tmp, s->tmp_cap) : 0;
        if (final) count += rsmp_flush(s->rs, s->tmp + count, s->tmp_cap - count);
        in = s->tmp;
    }
    s->stats.audio_seconds += (double)count / MEL_SR;
    if (!(final && count == 0 && melfe_samples(s->mel) == 0)) {
        const float *frames;
        size_t nf;
        melfe_push(s->mel, in, count, final, &frames, &nf);
        if (nf && s->dump) {
            if (s->n_mel_dump + nf > s->cap_mel_dump) {
                s->cap_mel_dump = (s->n_mel_dump + nf) * 2;
                s->mel_dump = realloc(s->mel_dump, s->cap_mel_dump * MEL_NMEL * sizeof(float));
            }
            memcpy(s->mel_dump + s->n_mel_dump * MEL_NMEL, frames, nf * MEL_NMEL * sizeof(float));
            s->n_mel_dump += nf;
        }
        if (nf) encoder_push(s->enc, frames, nf);
        if (run_pending(s, final, NULL, err, errlen) < 0) return NULL;
    }
    if (final) s->finished = 1;
    if (!s->text_len) return NULL;
    char *out = s->text;
    s->text = NULL;
    s->text_len = s->text_cap = 0;
    return out;
}

int nemoasr_prepare_latency(nemoasr_t *s, int latency_ms, char *err, size_t errlen) {
    if (errlen) err[0] = 0;
    const int right = right_for(latency_ms);
    if (right < 0) { snprintf(err, errlen, "latency must be one of 80, 160, 320, 560, 1120 ms"); return -1; }
    if (!model_right_context_trained(s->m, right)) {
        snprintf(err, errlen, "latency %d ms not trained for this checkpoint", latency_ms);
        return -1;
    }
    if (!(s->warmed & (1u << right))) {
        warmup(s->m, right, err, errlen);
        if (errlen) err[0] = 0;
        s->warmed |= 1u << right;
    }
    return 0;
}

int nemoasr_reset(nemoasr_t *s, const char *language, int latency_ms, char *err, size_t errlen) {
    if (errlen) err[0] = 0;
    if (nemoasr_prepare_latency(s, latency_ms, err, errlen)) return -1;
    if (language && model_set_language(s->m, language, err, errlen)) return -1;
    const int right = right_for(latency_ms);
    if (encoder_right(s->enc) == right) {
        encoder_reset(s->enc);
    } else {
        encoder_destroy(s->enc);
        s->enc = encoder_create(s->m, right);
        if (!s->enc) {
            snprintf(err, errlen, "nemoasr_reset: GPU setup failed: %s", gpu_last_error(s->m->gpu));
            s->finished = 1;
            return -1;
        }
        encoder_set_dump(s->enc, s->dump);
    }
    melfe_destroy(s->mel);
    s->mel = melfe_create();
    decoder_reset(s->dec);
    if (s->rs) { rsmp_destroy(s->rs); s->rs = rsmp_create(s->input_rate, MEL_SR); }
    free(s->text);
    s->text = NULL;
    s->text_len = s->text_cap = 0;
    s->finished = 0;
    s->printed_any = 0;
    s->latency_ms = latency_ms;
    s->n_tok = 0;
    s->n_chunk = 0;
    s->n_mel_dump = 0;
    s->joint_steps = 0;
    s->enc_gpu_ms = 0;
    memset(&s->stats, 0, sizeof s->stats);
    return 0;
}

void nemoasr_free(char *text) { free(text); }
double nemoasr_load_ms(const nemoasr_t *s) { return s->load_ms; }
const char *nemoasr_gpu_name(const nemoasr_t *s) { return gpu_device_name(s->m->gpu); }
int nemoasr_latency_ms(const nemoasr_t *s) { return s->latency_ms; }
void nemoasr_stats(const nemoasr_t *s, nemoasr_stats_t *out) { *out = s->stats; }

/* ---- test hooks ---------------------------------------------------------------------------- */
int nemoasr_debug_feed_mel(nemoasr_t *s, const float *mel, size_t nframes, int final, char *err, size_t errlen) {
    if (errlen) err[0] = 0;
    if (nframes) encoder_push(s->enc, mel, nframes);
    int n = 0;
    if (run_pending(s, final, &n, err, errlen) < 0) return -1;
    return n;
}
const int *nemoasr_debug_tokens(const nemoasr_t *s, size_t *n) {
    *n = s->n_tok;
    return s->all_tok;
}
void nemoasr_debug_set_dump(nemoasr_t *s, int on) {
    s->dump = on;
    encoder_set_dump(s->enc, on);
}
const float *nemoasr_debug_dump_mel(const nemoasr_t *s, size_t *nframes) {
    *nframes = s->n_mel_dump;
    return s->mel_dump;
}
size_t nemoasr_debug_frames(const nemoasr_t *s) { return encoder_dump_frames(s->enc); }
const float *nemoasr_debug_dump_layers(const nemoasr_t *s) { return encoder_dump_layers(s->enc); }
const float *nemoasr_debug_dump_prompted(const nemoasr_t *s) { return encoder_dump_prompted(s->enc); }
const float *nemoasr_debug_dump_joint_enc(const nemoasr_t *s) { return encoder_dump_joint(s->enc); }
void nemoasr_debug_use_graphs(nemoasr_t *s, int on) {
    encoder_use_graphs(s->enc, on);
    decoder_use_graphs(s->dec, on);
}
void nemoasr_debug_fuse(nemoasr_t *s, int on) { encoder_fuse(s->enc, on); }
size_t nemoasr_debug_joint_steps(const nemoasr_t *s) { return s->joint_steps; }
double nemoasr_debug_encoder_gpu_ms(const nemoasr_t *s) { return s->enc_gpu_ms; }
const double *nemoasr_debug_chunk_ms(const nemoasr_t *s, size_t *n) {
    *n = s->n_chunk;
    return s->chunk_ms;
}
int nemoasr_debug_time_kernel(nemoasr_t *s, const char *kernel, int max_launches) {
    return gpu_timing_set(s->m->gpu, kernel, max_launches);
}
int nemoasr_debug_kernel_ms(nemoasr_t *s, double *mean_ms, int *count, double *bytes) {
    return gpu_timing_collect(s->m->gpu, mean_ms, count, bytes);
}
size_t nemoasr_debug_weight_bytes(const nemoasr_t *s) { return s->m->warena_bytes; }
uint64_t nemoasr_debug_launches(const nemoasr_t *s) { return gpu_launch_count(s->m->gpu); }
