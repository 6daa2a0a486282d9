#include "safetensors.h"
#include "json.h"
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

int st_map(const char *path, st_map_t *out, char *err, size_t errlen) {
    memset(out, 0, sizeof *out);
    int fd = open(path, O_RDONLY);
    if (fd < 0) { snprintf(err, errlen, "cannot open %s", path); return -1; }
    struct stat sb;
    if (fstat(fd, &sb) || sb.st_size < 8) { close(fd); snprintf(err, errlen, "%s: not a safetensors file", path); return -1; }
    void *m = mmap(NULL, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) { snprintf(err, errlen, "mmap %s failed", path); return -1; }
    out->map = m;
    out->size = (size_t)sb.st_size;
    uint64_t hlen = 0;
    memcpy(&hlen, m, 8);
    if (hlen > out->size - 8) { snprintf(err, errlen, "%s: bad header length", path); st_unmap(out); return -1; }
    char jerr[128];
    jn_t *h = jn_parse((const char *)m + 8, (size_t)hlen, jerr, sizeof jerr);
    if (!h || h->type != JN_OBJ) {
        snprintf(err, errlen, "%s: header: %s", path, h ? "not an object" : jerr);
        jn_free(h);
        st_unmap(out);
        return -1;
    }
    const size_t data0 = 8 + (size_t)hlen;
    out->t = calloc(h->n ? h->n : 1, sizeof *out->t);
    for (size_t i = 0; i < h->n; ++i) {
        if (!strcmp(h->keys[i], "__metadata__")) continue;
        const jn_t *d = h->kids[i];
        st_entry_t *e = &out->t[out->n];
        const char *dt = jn_str(jn_get(d, "dtype"), "");
        e->dtype = !strcmp(dt, "BF16") ? STD_BF16 : !strcmp(dt, "F16") ? STD_F16 : !strcmp(dt, "F32") ? STD_F32 : STD_OTHER;
        const jn_t *shape = jn_get(d, "shape"), *offs = jn_get(d, "data_offsets");
        e->numel = 1;
        for (size_t k = 0; k < jn_len(shape); ++k) e->numel *= (size_t)jn_num(jn_at(shape, k), 0);
        const double a = jn_num(jn_at(offs, 0), -1), b = jn_num(jn_at(offs, 1), -1);
        if (a < 0 || b < a || data0 + (size_t)b > out->size) {
            snprintf(err, errlen, "%s: tensor %s outside the file", path, h->keys[i]);
            jn_free(h);
            st_unmap(out);
            return -1;
        }
        e->offset = data0 + (size_t)a;
        e->nbytes = (size_t)(b - a);
        e->name = strdup(h->keys[i]);
        out->n++;
    }
    jn_free(h);
    return 0;
}

void st_unmap(st_map_t *f) {
    if (f->map) munmap(f->map, f->size);
    for (size_t i = 0; i < f->n; ++i) free(f->t[i].name);
    free(f->t);
    memset(f, 0, sizeof *f);
}

const st_entry_t *st_lookup(const st_map_t *f, const char *name) {
    for (size_t i = 0; i < f->n; ++i)
        if (!strcmp(f->t[i].name, name)) return &f->t[i];
    return NULL;
}
