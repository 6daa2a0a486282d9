/* Safetensors checkpoint index over pread (see ckpt.h). */
#include "ckpt.h"
#include "json.h"
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

struct ckpt {
    int fd;
    uint64_t size;
    ck_tensor_t *t; /* sorted by name */
    size_t n;
    char *names;    /* every name, NUL-terminated, back to back */
};

static const struct { const char *tag; ck_dtype_t dt; unsigned esz; } k_dtypes[] = {
    { "BF16", CK_BF16, 2 }, { "F16", CK_F16, 2 }, { "F32", CK_F32, 4 },
};

/* the whole range or an error (short reads and EINTR retried) */
static int pread_all(int fd, void *dst, size_t len, uint64_t at) {
    char *p = dst;
    while (len) {
        const ssize_t r = pread(fd, p, len, (off_t)at);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return -1;
        p += r;
        len -= (size_t)r;
        at += (uint64_t)r;
    }
    return 0;
}

static int by_name(const void *a, const void *b) {
    return strcmp(((const ck_tensor_t *)a)->name, ((const ck_tensor_t *)b)->name);
}

/* a JSON number that is a non-negative integer below 2^53 */
static int as_index(const jn_t *v, uint64_t *out) {
    if (!v || v->type != JN_NUM || v->num < 0 || v->num > 9007199254740992.0 || v->num != (double)(uint64_t)v->num)
        return -1;
    *out = (uint64_t)v->num;
    return 0;
}

/* One header entry -> t; the name pointer is filled in by the caller.  0 or an error text. */
static const char *describe(const jn_t *d, uint64_t data0, uint64_t fsize, ck_tensor_t *t) {
    const char *tag = jn_str(jn_get(d, "dtype"), "");
    unsigned esz = 0;
    t->dtype = CK_OTHER;
    for (size_t k = 0; k < sizeof k_dtypes / sizeof k_dtypes[0]; ++k)
        if (!strcmp(tag, k_dtypes[k].tag)) {
            t->dtype = k_dtypes[k].dt;
            esz = k_dtypes[k].esz;
        }
    const jn_t *shape = jn_get(d, "shape"), *range = jn_get(d, "data_offsets");
    if (!shape || shape->type != JN_ARR) return "no shape";
    uint64_t numel = 1, dim;
    for (size_t k = 0; k < jn_len(shape); ++k) {
        if (as_index(jn_at(shape, k), &dim)) return "bad shape";
        numel *= dim;
    }
    uint64_t lo, hi;
    if (jn_len(range) != 2 || as_index(jn_at(range, 0), &lo) || as_index(jn_at(range, 1), &hi) || hi < lo)
        return "bad data_offsets";
    if (data0 + hi > fsize) return "data past the end of the file";
    if (esz && hi - lo != numel * esz) return "byte length does not match the shape";
    t->numel = (size_t)numel;
    t->at = data0 + lo;
    t->bytes = hi - lo;
    return NULL;
}

ckpt_t *ckpt_open(const char *path, char *err, size_t errlen) {
    ckpt_t *c = calloc(1, sizeof *c);
    if (!c) { snprintf(err, errlen, "out of memory"); return NULL; }
    c->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (c->fd < 0) {
        snprintf(err, errlen, "%s: %s", path, strerror(errno));
        free(c);
        return NULL;
    }
    struct stat sb;
    unsigned char len8[8];
    jn_t *h = NULL;
    char *text = NULL;
    const char *why = NULL;
    if (fstat(c->fd, &sb) || pread_all(c->fd, len8, 8, 0)) { why = "unreadable"; goto bad; }
    c->size = (uint64_t)sb.st_size;
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | len8[i]; /* little-endian */
    if (hlen == 0 || hlen > c->size - 8) { why = "header length out of range"; goto bad; }
    if (!(text = malloc((size_t)hlen)) || pread_all(c->fd, text, (size_t)hlen, 8)) { why = "header unreadable"; goto bad; }
    char jerr[128];
    if (!(h = jn_parse(text, (size_t)hlen, jerr, sizeof jerr)) || h->type != JN_OBJ) {
        snprintf(err, errlen, "%s: header is not a JSON object (%s)", path, h ? "wrong type" : jerr);
        goto fail;
    }
    size_t namebytes = 0;
    for (size_t i = 0; i < h->n; ++i) namebytes += strlen(h->keys[i]) + 1;
    c->t = calloc(h->n ? h->n : 1, sizeof *c->t);
    c->names = malloc(namebytes ? namebytes : 1);
    if (!c->t || !c->names) { why = "out of memory"; goto bad; }
    char *np = c->names;
    for (size_t i = 0; i < h->n; ++i) {
        if (!strcmp(h->keys[i], "__metadata__")) continue;
        ck_tensor_t *t = &c->t[c->n];
        const char *e = describe(h->kids[i], 8 + hlen, c->size, t);
        if (e) {
            snprintf(err, errlen, "%s: tensor %s: %s", path, h->keys[i], e);
            goto fail;
        }
        const size_t l = strlen(h->keys[i]) + 1;
        memcpy(np, h->keys[i], l);
        t->name = np;
        np += l;
        c->n++;
    }
    qsort(c->t, c->n, sizeof *c->t, by_name);
    for (size_t i = 1; i < c->n; ++i)
        if (!strcmp(c->t[i - 1].name, c->t[i].name)) {
            snprintf(err, errlen, "%s: tensor %s listed twice", path, c->t[i].name);
            goto fail;
        }
    jn_free(h);
    free(text);
    return c;
bad:
    snprintf(err, errlen, "%s: not a readable safetensors file (%s)", path, why);
fail:
    jn_free(h);
    free(text);
    ckpt_close(c);
    return NULL;
}

void ckpt_close(ckpt_t *c) {
    if (!c) return;
    if (c->fd >= 0) close(c->fd);
    free(c->t);
    free(c->names);
    free(c);
}

int ckpt_fd(const ckpt_t *c) { return c->fd; }
size_t ckpt_count(const ckpt_t *c) { return c->n; }

const ck_tensor_t *ckpt_find(const ckpt_t *c, const char *name) {
    const ck_tensor_t key = { .name = name };
    return bsearch(&key, c->t, c->n, sizeof *c->t, by_name);
}

int ckpt_read(const ckpt_t *c, const ck_tensor_t *t, void *dst) { return pread_all(c->fd, dst, (size_t)t->bytes, t->at); }
