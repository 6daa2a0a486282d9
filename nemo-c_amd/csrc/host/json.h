/* Minimal read-only JSON tree for config.json and safetensors headers (load time only).
 * Same role as the reference's src/json.h; independent implementation. */
#ifndef NEMO_JSON_H
#define NEMO_JSON_H
#include <stddef.h>

typedef enum { JN_NULL, JN_BOOL, JN_NUM, JN_STR, JN_ARR, JN_OBJ } jn_type;

typedef struct jn {
    jn_type type;
    double num;          /* JN_NUM, JN_BOOL (0/1) */
    char *str;           /* JN_STR */
    size_t n;            /* JN_ARR / JN_OBJ: element count */
    struct jn **kids;    /* elements / values */
    char **keys;         /* JN_OBJ keys */
} jn_t;

jn_t *jn_parse(const char *text, size_t len, char *err, size_t errlen);
void jn_free(jn_t *v);
const jn_t *jn_get(const jn_t *obj, const char *key); /* NULL if absent or not an object */
const jn_t *jn_at(const jn_t *arr, size_t i);
size_t jn_len(const jn_t *v);
double jn_num(const jn_t *v, double dflt);
const char *jn_str(const jn_t *v, const char *dflt);

#endif
