#include "mel.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define PRE_EMPH 0.97f
#define LOG_FLOOR 5.9604644775390625e-08f /* 2^-24 */
#define HALF (MEL_NFFT / 2)

struct melfe {
    float *y;               /* pre-emphasised samples; y[i] is global sample y0 + i */
    size_t ny, cap, y0;
    float prev;
    int started, closed;
    size_t total, next;     /* samples received; next frame index to emit */
    size_t end;             /* frames complete so far (next .. end-1 not yet taken) */
    float *span;            /* melfe_push's span buffer */
    size_t span_cap;
    float win[MEL_NFFT];
    float fb[MEL_NMEL][MEL_NBIN];
    int fb_lo[MEL_NMEL], fb_hi[MEL_NMEL]; /* nonzero bin range per filter */
    double tw_re[MEL_NFFT / 2], tw_im[MEL_NFFT / 2];
    unsigned short rev[MEL_NFFT];
    float *out;
    size_t out_cap;
};

/* Slaney mel scale: linear below 1 kHz (200/3 Hz per mel), logarithmic above. */
static double slaney_mel(double hz) {
    const double sp = 200.0 / 3.0, brk = 1000.0, step = log(6.4) / 27.0;
    return hz < brk ? hz / sp : brk / sp + log(hz / brk) / step;
}
static double slaney_hz(double mel) {
    const double sp = 200.0 / 3.0, brk = 1000.0, step = log(6.4) / 27.0;
    return mel < brk / sp ? mel * sp : brk * exp(step * (mel - brk / sp));
}

melfe_t *melfe_create(void) {
    melfe_t *m = calloc(1, sizeof *m);
    m->cap = 1 << 16;
    m->y = malloc(m->cap * sizeof(float));
    const int off = (MEL_NFFT - MEL_WIN) / 2;
    for (int i = 0; i < MEL_WIN; ++i) m->win[off + i] = (float)(0.5 - 0.5 * cos(2.0 * M_PI * i / (MEL_WIN - 1)));
    /* triangular filters between consecutive points equally spaced in mel, area-normalised */
    double pts[MEL_NMEL + 2];
    const double mlo = slaney_mel(0.0), mhi = slaney_mel(MEL_SR / 2.0);
    for (int i = 0; i < MEL_NMEL + 2; ++i) pts[i] = slaney_hz(mlo + (mhi - mlo) * i / (MEL_NMEL + 1));
    for (int b = 0; b < MEL_NMEL; ++b) {
        const double norm = 2.0 / (pts[b + 2] - pts[b]);
        m->fb_lo[b] = MEL_NBIN;
        m->fb_hi[b] = 0;
        for (int k = 0; k < MEL_NBIN; ++k) {
            const double f = (MEL_SR / 2.0) * k / (MEL_NBIN - 1);
            const double rise = (f - pts[b]) / (pts[b + 1] - pts[b]);
            const double fall = (pts[b + 2] - f) / (pts[b + 2] - pts[b + 1]);
            double w = rise < fall ? rise : fall;
            if (w < 0) w = 0;
            m->fb[b][k] = (float)(w * norm);
            if (m->fb[b][k] != 0.0f) {
                if (k < m->fb_lo[b]) m->fb_lo[b] = k;
                m->fb_hi[b] = k + 1;
            }
        }
    }
    for (int i = 0; i < MEL_NFFT / 2; ++i) {
        m->tw_re[i] = cos(-2.0 * M_PI * i / MEL_NFFT);
        m->tw_im[i] = sin(-2.0 * M_PI * i / MEL_NFFT);
    }
    int bits = 0;
    while ((1 << bits) < MEL_NFFT) bits++;
    for (int i = 0; i < MEL_NFFT; ++i) {
        int r = 0;
        for (int b = 0; b < bits; ++b) r |= ((i >> b) & 1) << (bits - 1 - b);
        m->rev[i] = (unsigned short)r;
    }
    return m;
}

void melfe_destroy(melfe_t *m) {
    if (!m) return;
    free(m->y);
    free(m->out);
    free(m->span);
    free(m);
}
size_t melfe_samples(const melfe_t *m) { return m->total; }
size_t melfe_frames(const melfe_t *m) { return m->next; }

/* iterative radix-2 decimation-in-time FFT of MEL_NFFT points, double precision */
static void fft(const melfe_t *m, double *re, double *im) {
    for (int i = 0; i < MEL_NFFT; ++i) {
        const int j = m->rev[i];
        if (j > i) {
            double t = re[i]; re[i] = re[j]; re[j] = t;
            t = im[i]; im[i] = im[j]; im[j] = t;
        }
    }
    for (int len = 2; len <= MEL_NFFT; len <<= 1) {
        const int h = len >> 1, stride = MEL_NFFT / len;
        for (int s = 0; s < MEL_NFFT; s += len)
            for (int k = 0; k < h; ++k) {
                const double wr = m->tw_re[k * stride], wi = m->tw_im[k * stride];
                const int a = s + k, b = a + h;
                const double xr = re[b] * wr - im[b] * wi, xi = re[b] * wi + im[b] * wr;
                re[b] = re[a] - xr; im[b] = im[a] - xi;
                re[a] += xr; im[a] += xi;
            }
    }
}

/* pre-emphasised sample at global index g with reflection (no edge repeat) at both ends */
static float at(const melfe_t *m, long g) {
    const long n = (long)m->total;
    if (g < 0) g = -g;
    if (g >= n) g = 2 * n - 2 - g;
    if (g < 0 || g >= n) return 0.0f;
    const long i = g - (long)m->y0;
    return (i >= 0 && i < (long)m->ny) ? m->y[i] : 0.0f;
}

size_t melfe_append(melfe_t *m, const float *x, size_t n, int final) {
    if (m->closed) return m->end > m->next ? m->end - m->next : 0;
    if (m->ny + n > m->cap) {
        while (m->ny + n > m->cap) m->cap *= 2;
        m->y = realloc(m->y, m->cap * sizeof(float));
    }
    if (n) {
        /* y[i] = x[i] - 0.97 x[i-1] (the first sample of the stream passes unchanged) */
        float *y = m->y + m->ny;
        y[0] = m->started ? x[0] - PRE_EMPH * m->prev : x[0];
        for (size_t i = 1; i < n; ++i) y[i] = x[i] - PRE_EMPH * x[i - 1];
        m->ny += n;
        m->prev = x[n - 1];
        m->started = 1;
    }
    m->total += n;
    size_t end;
    if (final) end = m->total / MEL_HOP + 1;
    else end = m->total >= HALF ? (m->total - HALF) / MEL_HOP + 1 : 0; /* every sample of the frame is in */
    if (final) m->closed = 1;
    if (end > m->end) m->end = end;
    return m->end > m->next ? m->end - m->next : 0;
}

size_t melfe_span_len(size_t cnt) { return cnt ? (cnt - 1) * MEL_HOP + MEL_NFFT : 0; }

size_t melfe_take(melfe_t *m, float *span, size_t kmax) {
    size_t cnt = m->end > m->next ? m->end - m->next : 0;
    if (cnt > kmax) cnt = kmax;
    if (!cnt) return 0;
    const long base = (long)m->next * MEL_HOP - HALF, len = (long)melfe_span_len(cnt), n = (long)m->total;
    /* samples inside the stream come straight from the buffer; reflected ones through at() */
    long lo = base < 0 ? -base : 0, hi = n - base < len ? n - base : len;
    if (hi < lo || base + lo < (long)m->y0 || base + hi > (long)(m->y0 + m->ny)) lo = hi = 0;
    for (long i = 0; i < lo; ++i) span[i] = at(m, base + i);
    if (hi > lo) memcpy(span + lo, m->y + (base + lo - (long)m->y0), (size_t)(hi - lo) * sizeof(float));
    for (long i = hi > lo ? hi : lo; i < len; ++i) span[i] = at(m, base + i);
    m->next += cnt;
    /* drop samples no future frame reads */
    const long keep = (long)m->next * MEL_HOP - HALF - 4;
    if (keep > (long)m->y0) {
        size_t drop = (size_t)(keep - (long)m->y0);
        if (drop > m->ny) drop = m->ny;
        memmove(m->y, m->y + drop, (m->ny - drop) * sizeof(float));
        m->ny -= drop;
        m->y0 += drop;
    }
    return cnt;
}

void melfe_compute(const melfe_t *m, const float *span, size_t cnt, float *out) {
    double re[MEL_NFFT], im[MEL_NFFT];
    float pw[MEL_NBIN];
    for (size_t t = 0; t < cnt; ++t) {
        const float *fr = span + t * MEL_HOP;
        for (int k = 0; k < MEL_NFFT; ++k) {
            re[k] = (double)(fr[k] * m->win[k]);
            im[k] = 0.0;
        }
        fft(m, re, im);
        for (int k = 0; k < MEL_NBIN; ++k) pw[k] = (float)(re[k] * re[k] + im[k] * im[k]);
        float *row = out + t * MEL_NMEL;
        for (int b = 0; b < MEL_NMEL; ++b) {
            float acc = 0.0f;
            for (int k = m->fb_lo[b]; k < m->fb_hi[b]; ++k) acc += m->fb[b][k] * pw[k];
            row[b] = logf(acc + LOG_FLOOR);
        }
    }
}

void melfe_push(melfe_t *m, const float *x, size_t n, int final, const float **frames, size_t *nframes) {
    *frames = NULL;
    *nframes = 0;
    const size_t cnt = melfe_append(m, x, n, final);
    if (!cnt) return;
    const size_t len = melfe_span_len(cnt);
    if (len > m->span_cap) {
        m->span_cap = len;
        m->span = realloc(m->span, m->span_cap * sizeof(float));
    }
    if (cnt * MEL_NMEL > m->out_cap) {
        m->out_cap = cnt * MEL_NMEL;
        m->out = realloc(m->out, m->out_cap * sizeof(float));
    }
    melfe_take(m, m->span, cnt);
    melfe_compute(m, m->span, cnt, m->out);
    *frames = m->out;
    *nframes = cnt;
}

void melfe_tables(const melfe_t *m, melfe_tables_t *t) {
    t->win = m->win;
    t->fb = &m->fb[0][0];
    t->fb_lo = m->fb_lo;
    t->fb_hi = m->fb_hi;
    t->tw_re = m->tw_re;
    t->tw_im = m->tw_im;
    t->rev = m->rev;
}
