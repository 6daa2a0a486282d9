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

void melfe_push(melfe_t *m, const float *x, size_t n, int final, const float **frames, size_t *nframes) {
    *frames = NULL;
    *nframes = 0;
    if (m->closed) return;
    if (m->ny + n > m->cap) {
        while (m->ny + n > m->cap) m->cap *= 2;
        m->y = realloc(m->y, m->cap * sizeof(float));
    }
    for (size_t i = 0; i < n; ++i) {
        m->y[m->ny++] = m->started ? x[i] - PRE_EMPH * m->prev : x[i];
        m->prev = x[i];
        m->started = 1;
    }
    m->total += n;
    size_t end;
    if (final) end = m->total / MEL_HOP + 1;
    else end = m->total >= HALF ? (m->total - HALF) / MEL_HOP + 1 : 0; /* every sample of the frame is in */
    if (final) m->closed = 1;
    if (end <= m->next) return;
    const size_t cnt = end - m->next;
    if (cnt * MEL_NMEL > m->out_cap) {
        m->out_cap = cnt * MEL_NMEL;
        m->out = realloc(m->out, m->out_cap * sizeof(float));
    }
    double re[MEL_NFFT], im[MEL_NFFT];
    float pw[MEL_NBIN];
    for (size_t t = m->next; t < end; ++t) {
        const long base = (long)t * MEL_HOP - HALF;
        for (int k = 0; k < MEL_NFFT; ++k) {
            re[k] = (double)(at(m, base + k) * m->win[k]);
            im[k] = 0.0;
        }
        fft(m, re, im);
        for (int k = 0; k < MEL_NBIN; ++k) pw[k] = (float)(re[k] * re[k] + im[k] * im[k]);
        float *row = m->out + (t - m->next) * MEL_NMEL;
        for (int b = 0; b < MEL_NMEL; ++b) {
            float acc = 0.0f;
            for (int k = m->fb_lo[b]; k < m->fb_hi[b]; ++k) acc += m->fb[b][k] * pw[k];
            row[b] = logf(acc + LOG_FLOOR);
        }
    }
    *frames = m->out;
    *nframes = cnt;
    m->next = end;
    /* drop samples no future frame reads */
    const long keep = (long)m->next * MEL_HOP - HALF - 4;
    if (keep > (long)m->y0) {
        size_t drop = (size_t)(keep - (long)m->y0);
        if (drop > m->ny) drop = m->ny;
        memmove(m->y, m->y + drop, (m->ny - drop) * sizeof(float));
        m->ny -= drop;
        m->y0 += drop;
    }
}
