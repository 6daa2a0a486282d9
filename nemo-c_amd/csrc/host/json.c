#include "json.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    const char *p, *end, *start;
    char *err;
    size_t errlen;
    int depth;
} jp_t;

static void ws(jp_t *s) {
    while (s->p < s->end && (*s->p == ' ' || *s->p == '\t' || *s->p == '\n' || *s->p == '\r')) s->p++;
}

static jn_t *mk(jn_type t) {
    jn_t *v = calloc(1, sizeof *v);
    v->type = t;
    return v;
}

static int perr(jp_t *s, const char *what) {
    if (s->errlen && !s->err[0]) snprintf(s->err, s->errlen, "json: %s at offset %ld", what, (long)(s->p - s->start));
    return -1;
}

static void put_utf8(char **o, unsigned cp) {
    char *q = *o;
    if (cp < 0x80) *q++ = (char)cp;
    else if (cp < 0x800) { *q++ = (char)(0xC0 | (cp >> 6)); *q++ = (char)(0x80 | (cp & 0x3F)); }
    else if (cp < 0x10000) { *q++ = (char)(0xE0 | (cp >> 12)); *q++ = (char)(0x80 | ((cp >> 6) & 0x3F)); *q++ = (char)(0x80 | (cp & 0x3F)); }
    else { *q++ = (char)(0xF0 | (cp >> 18)); *q++ = (char)(0x80 | ((cp >> 12) & 0x3F)); *q++ = (char)(0x80 | ((cp >> 6) & 0x3F)); *q++ = (char)(0x80 | (cp & 0x3F)); }
    *o = q;
}

static int hex4(const char *p, unsigned *out) {
    unsigned v = 0;
    for (int i = 0; i < 4; ++i) {
        char c = p[i];
        v <<= 4;
        if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
        else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
        else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
        else return -1;
    }
    *out = v;
    return 0;
}

static char *pstring(jp_t *s) {
    if (s->p >= s->end || *s->p != '"') { perr(s, "expected string"); return NULL; }
    s->p++;
    const char *b = s->p;
    size_t cap = 16;
    while (s->p < s->end && *s->p != '"') { if (*s->p == '\\') s->p++; s->p++; cap++; }
    if (s->p >= s->end) { perr(s, "unterminated string"); return NULL; }
    char *out = malloc(cap * 2 + 8), *o = out;
    for (const char *q = b; q < s->p; ++q) {
        if (*q != '\\') { *o++ = *q; continue; }
        ++q;
        switch (*q) {
        case 'n': *o++ = '\n'; break;
        case 't': *o++ = '\t'; break;
        case 'r': *o++ = '\r'; break;
        case 'b': *o++ = '\b'; break;
        case 'f': *o++ = '\f'; break;
        case 'u': {
            unsigned cp;
            if (q + 4 >= s->p + 1 || hex4(q + 1, &cp)) { free(out); perr(s, "bad \\u escape"); return NULL; }
            q += 4;
            if (cp >= 0xD800 && cp < 0xDC00 && q + 6 < s->p && q[1] == '\\' && q[2] == 'u') {
                unsigned lo;
                if (!hex4(q + 3, &lo) && lo >= 0xDC00 && lo < 0xE000) { cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00); q += 6; }
            }
            put_utf8(&o, cp);
            break;
        }
        default: *o++ = *q; break;
        }
    }
    *o = 0;
    s->p++;
    return out;
}

static jn_t *pvalue(jp_t *s);

static jn_t *pcontainer(jp_t *s, int obj) {
    jn_t *v = mk(obj ? JN_OBJ : JN_ARR);
    size_t cap = 0;
    s->p++;
    ws(s);
    if (s->p < s->end && *s->p == (obj ? '}' : ']')) { s->p++; return v; }
    for (;;) {
        char *key = NULL;
        if (obj) {
            ws(s);
            if (!(key = pstring(s))) { jn_free(v); return NULL; }
            ws(s);
            if (s->p >= s->end || *s->p != ':') { free(key); jn_free(v); perr(s, "expected ':'"); return NULL; }
            s->p++;
        }
        jn_t *k = pvalue(s);
        if (!k) { free(key); jn_free(v); return NULL; }
        if (v->n == cap) {
            cap = cap ? cap * 2 : 8;
            v->kids = realloc(v->kids, cap * sizeof *v->kids);
            if (obj) v->keys = realloc(v->keys, cap * sizeof *v->keys);
        }
        v->kids[v->n] = k;
        if (obj) v->keys[v->n] = key;
        v->n++;
        ws(s);
        if (s->p < s->end && *s->p == ',') { s->p++; continue; }
        if (s->p < s->end && *s->p == (obj ? '}' : ']')) { s->p++; return v; }
        jn_free(v);
        perr(s, obj ? "expected ',' or '}'" : "expected ',' or ']'");
        return NULL;
    }
}

static jn_t *pvalue(jp_t *s) {
    ws(s);
    if (s->p >= s->end) { perr(s, "unexpected end"); return NULL; }
    if (++s->depth > 256) { perr(s, "nesting too deep"); return NULL; }
    jn_t *v = NULL;
    const char c = *s->p;
    if (c == '{' || c == '[') v = pcontainer(s, c == '{');
    else if (c == '"') {
        char *str = pstring(s);
        if (str) { v = mk(JN_STR); v->str = str; }
    } else if (!strncmp(s->p, "true", 4) && s->end - s->p >= 4) { v = mk(JN_BOOL); v->num = 1; s->p += 4; }
    else if (!strncmp(s->p, "false", 5) && s->end - s->p >= 5) { v = mk(JN_BOOL); s->p += 5; }
    else if (!strncmp(s->p, "null", 4) && s->end - s->p >= 4) { v = mk(JN_NULL); s->p += 4; }
    else {
        char buf[64];
        size_t n = 0;
        while (s->p + n < s->end && n < sizeof buf - 1 && strchr("+-0123456789.eE", s->p[n])) { buf[n] = s->p[n]; n++; }
        buf[n] = 0;
        char *e;
        double d = strtod(buf, &e);
        if (!n || *e) perr(s, "bad token");
        else { v = mk(JN_NUM); v->num = d; s->p += n; }
    }
    s->depth--;
    return v;
}

jn_t *jn_parse(const char *text, size_t len, char *err, size_t errlen) {
    jp_t s = { text, text + len, text, err, errlen, 0 };
    if (errlen) err[0] = 0;
    jn_t *v = pvalue(&s);
    if (!v) return NULL;
    ws(&s);
    if (s.p != s.end && *s.p != 0) {
        jn_free(v);
        if (errlen) snprintf(err, errlen, "json: trailing characters");
        return NULL;
    }
    return v;
}

void jn_free(jn_t *v) {
    if (!v) return;
    for (size_t i = 0; i < v->n; ++i) {
        jn_free(v->kids[i]);
        if (v->keys) free(v->keys[i]);
    }
    free(v->kids);
    free(v->keys);
    free(v->str);
    free(v);
}

const jn_t *jn_get(const jn_t *o, const char *key) {
    if (!o || o->type != JN_OBJ) return NULL;
    for (size_t i = 0; i < o->n; ++i)
        if (!strcmp(o->keys[i], key)) return o->kids[i];
    return NULL;
}
const jn_t *jn_at(const jn_t *a, size_t i) {
    if (!a || (a->type != JN_ARR && a->type != JN_OBJ) || i >= a->n) return NULL;
    return a->kids[i];
}
size_t jn_len(const jn_t *v) { return v && (v->type == JN_ARR || v->type == JN_OBJ) ? v->n : 0; }
double jn_num(const jn_t *v, double d) { return v && (v->type == JN_NUM || v->type == JN_BOOL) ? v->num : d; }
const char *jn_str(const jn_t *v, const char *d) { return v && v->type == JN_STR ? v->str : d; }
