#include "tokenizer.h"
#include <stdlib.h>
#include <string.h>

int vocab_load(const jn_t *arr, vocab_t *v) {
    memset(v, 0, sizeof *v);
    if (!arr || arr->type != JN_ARR) return -1;
    v->n = (int)arr->n;
    v->piece = calloc((size_t)v->n + 1, sizeof *v->piece);
    for (int i = 0; i < v->n; ++i) v->piece[i] = strdup(jn_str(arr->kids[i], ""));
    return 0;
}

void vocab_release(vocab_t *v) {
    for (int i = 0; i < v->n; ++i) free(v->piece[i]);
    free(v->piece);
    memset(v, 0, sizeof *v);
}

static int is_lower(char c) { return c >= 'a' && c <= 'z'; }
static int is_alpha(char c) { return is_lower(c) || (c >= 'A' && c <= 'Z'); }

/* "<" + 2..3 lowercase letters + "-" + 2..4 letters + ">" */
int piece_is_lang_tag(const char *p) {
    const size_t n = strlen(p);
    if (n < 7 || p[0] != '<' || p[n - 1] != '>') return 0;
    size_t i = 1, a = 0, b = 0;
    while (i < n - 1 && p[i] != '-') { if (!is_lower(p[i])) return 0; a++; i++; }
    if (i >= n - 1 || p[i] != '-') return 0;
    for (i++; i < n - 1; ++i) { if (!is_alpha(p[i])) return 0; b++; }
    return a >= 2 && a <= 3 && b >= 2 && b <= 4;
}

int piece_is_special(const char *p) {
    static const char *sp[] = { "<unk>", "<pad>", "<s>", "</s>" };
    for (size_t i = 0; i < sizeof sp / sizeof *sp; ++i)
        if (!strcmp(p, sp[i])) return 1;
    return piece_is_lang_tag(p);
}

char *piece_text(const vocab_t *v, int id) {
    if (id < 0 || id >= v->n || piece_is_special(v->piece[id])) return strdup("");
    const unsigned char *p = (const unsigned char *)v->piece[id];
    const size_t n = strlen((const char *)p);
    char *out = malloc(n + 1), *o = out;
    for (size_t i = 0; i < n;) {
        if (i + 2 < n && p[i] == 0xE2 && p[i + 1] == 0x96 && p[i + 2] == 0x81) { *o++ = ' '; i += 3; }
        else *o++ = (char)p[i++];
    }
    *o = 0;
    return out;
}
