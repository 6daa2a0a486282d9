/* Read-only safetensors access (memory-mapped), load time only.  The file format and the tensor
 * names are the checkpoint contract of the reference (src/safetensors.h, src/model.c:215-282). */
#ifndef NEMO_SAFETENSORS_H
#define NEMO_SAFETENSORS_H
#include <stddef.h>
#include <stdint.h>

typedef enum { STD_BF16, STD_F16, STD_F32, STD_OTHER } st_dtype_t;

typedef struct {
    char *name;
    st_dtype_t dtype;
    size_t numel, nbytes, offset; /* offset: absolute byte offset in the file */
} st_entry_t;

typedef struct {
    void *map;
    size_t size;
    st_entry_t *t;
    size_t n;
} st_map_t;

int st_map(const char *path, st_map_t *out, char *err, size_t errlen);
void st_unmap(st_map_t *f);
const st_entry_t *st_lookup(const st_map_t *f, const char *name);
static inline const void *st_ptr(const st_map_t *f, const st_entry_t *e) { return (const char *)f->map + e->offset; }

/* bf16 bit pattern -> f32: the pattern is the upper half of the f32 (src/safetensors.h:32-36). */
static inline float st_bf16(uint16_t v) {
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)v << 16;
    return c.f;
}

#endif
