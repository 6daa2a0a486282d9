/* Read-only index of a safetensors checkpoint, load time only.
 *
 * The file format is the reference's checkpoint contract (src/safetensors.h): an 8-byte
 * little-endian header length, a JSON header giving every tensor's dtype, shape and byte range
 * relative to the end of the header, then the tensor bytes.  The index is built from the header
 * read with pread; the 1.2 GB of tensor bytes are never mapped: small tensors are read on demand
 * (ckpt_read) and the weight matrices stream from the open descriptor into device memory
 * (gpu_upload_file).  Lookup is a binary search over the index sorted by name. */
#ifndef NEMO_CKPT_H
#define NEMO_CKPT_H
#include <stddef.h>
#include <stdint.h>

typedef enum { CK_BF16, CK_F16, CK_F32, CK_OTHER } ck_dtype_t;

typedef struct {
    const char *name;
    ck_dtype_t dtype;
    size_t numel;
    uint64_t at, bytes; /* absolute file offset and length of the tensor's bytes */
} ck_tensor_t;

typedef struct ckpt ckpt_t;

ckpt_t *ckpt_open(const char *path, char *err, size_t errlen);
void ckpt_close(ckpt_t *c);
int ckpt_fd(const ckpt_t *c);
size_t ckpt_count(const ckpt_t *c);
const ck_tensor_t *ckpt_find(const ckpt_t *c, const char *name);
/* the tensor's bytes into dst (t->bytes long); 0 on success */
int ckpt_read(const ckpt_t *c, const ck_tensor_t *t, void *dst);

/* bf16 bits -> f32: the bits are the upper half of the f32 pattern (exact widening,
 * src/safetensors.h:32-36) */
static inline float ck_bf16(uint16_t v) {
    union { uint32_t u; float f; } w;
    w.u = (uint32_t)v << 16;
    return w.f;
}

#endif
