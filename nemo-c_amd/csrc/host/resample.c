#include "resample.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define CROSSINGS 16

struct rsmp {
    int same;
    double step;   /* input samples per output sample */
    double reach;  /* kernel half width in input samples */
    double band;   /* cutoff as a fraction of the input rate, times 2 */
    float *buf;    /* buffered input; buf[i] is input sample base + i */
    size_t len, cap;
    unsigned long long base, seen, made;
};

rsmp_t *rsmp_create(int in_rate, int out_rate) {
    rsmp_t *r = calloc(1, sizeof *r);
    r->same = in_rate == out_rate;
    r->step = (double)in_rate / out_rate;
    r->reach = CROSSINGS * (r->step > 1.0 ? r->step : 1.0);
    r->band = r->step > 1.0 ? 1.0 / r->step : 1.0;
    r->cap = 1 << 14;
    r->buf = malloc(r->cap * sizeof(float));
    return r;
}

void rsmp_destroy(rsmp_t *r) {
    if (!r) return;
    free(r->buf);
    free(r);
}

/* band * sinc(band * u) * Blackman(u / reach), zero outside |u| < reach */
static double tap(const rsmp_t *r, double u) {
    const double x = u / r->reach;
    if (fabs(x) >= 1.0) return 0.0;
    const double w = 0.42 + 0.5 * cos(M_PI * x) + 0.08 * cos(2.0 * M_PI * x);
    const double a = M_PI * r->band * u;
    return r->band * (fabs(a) < 1e-9 ? 1.0 : sin(a) / a) * w;
}

static size_t run(rsmp_t *r, float *out, size_t out_max, int final) {
    size_t k = 0;
    while (k < out_max) {
        const double c = (double)r->made * r->step;
        const long lo = (long)ceil(c - r->reach), hi = (long)floor(c + r->reach);
        if (!final && (unsigned long long)(hi + 1) > r->seen) break;
        if (final && lo >= 0 && (unsigned long long)lo >= r->seen) break;
        double acc = 0.0, norm = 0.0;
        for (long i = lo; i <= hi; ++i) {
            const double h = tap(r, (double)i - c);
            norm += h;
            if (i < 0 || (unsigned long long)i >= r->seen) continue;
            const long j = i - (long)r->base;
            if (j >= 0 && (size_t)j < r->len) acc += h * r->buf[j];
        }
        out[k++] = (float)(norm > 0.0 ? acc / norm : 0.0);
        r->made++;
    }
    const long keep = (long)floor((double)r->made * r->step - r->reach) - 2;
    if (keep > (long)r->base) {
        size_t d = (size_t)(keep - (long)r->base);
        if (d > r->len) d = r->len;
        memmove(r->buf, r->buf + d, (r->len - d) * sizeof(float));
        r->len -= d;
        r->base += d;
    }
    return k;
}

size_t rsmp_process(rsmp_t *r, const float *in, size_t n, float *out, size_t out_max) {
    if (r->same) {
        const size_t m = n < out_max ? n : out_max;
        memcpy(out, in, m * sizeof(float));
        return m;
    }
    if (r->len + n > r->cap) {
        while (r->len + n > r->cap) r->cap *= 2;
        r->buf = realloc(r->buf, r->cap * sizeof(float));
    }
    memcpy(r->buf + r->len, in, n * sizeof(float));
    r->len += n;
    r->seen += n;
    return run(r, out, out_max, 0);
}

size_t rsmp_flush(rsmp_t *r, float *out, size_t out_max) { return r->same ? 0 : run(r, out, out_max, 1); }
