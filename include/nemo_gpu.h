/* The reference's GPU runtime interface, with its signatures (src/gpu.h:7-41), served by the HIP
 * layer of this library on one gfx950 GPU.
 *
 * A host written against the reference's gpu.h (its model.c launchers, encoder.c and decoder.c
 * dispatch sites) compiles against this header and links against libnemoasr_hip.so:
 *   gpu_create            src/gpu.h:20  the `metal_source` argument is accepted and not compiled:
 *                                       the gfx950 code object linked into the library is used
 *   gpu_buf_alloc         src/gpu.h:24  device memory, zero-filled (0 bytes -> a small buffer)
 *   gpu_buf_ptr           src/gpu.h:26  host address of a pinned mirror, coherent at batch edges:
 *                                       refreshed from the device after a batch, uploaded by the
 *                                       next gpu_begin (read and write between batches, through a
 *                                       pointer taken after the last gpu_end)
 *   gpu_dispatch          src/gpu.h:31  kernel by the reference's name; total threads (ignored:
 *                                       each launcher derives its own grid from the parameters)
 *   gpu_dispatch_groups   src/gpu.h:33  threadgroup counts (joint_partial reads groups_x: the
 *                                       number of partial-best groups per row)
 *   gpu_dispatch_groups_fc src/gpu.h:37 the function constants select no pipeline here: the
 *                                       kernel choice by (M, N, K) is this library's own
 *   gpu_begin / gpu_end / gpu_last_ms / gpu_last_error   src/gpu.h:29-41, same roles
 * Arguments follow src/gpu.m:98-101: argument i is a buffer (GPU_BUF: buffer + byte offset) or a
 * parameter block passed by value (GPU_BYTES), in the kernel's binding order of src/kernels.metal.
 * The parameter blocks are those of include/nemo_kernel_params.h (src/kernel_params.h:22-32).
 * Kernel names served: gemm_spec, gemm_mma, gemm_bf16, layernorm, layernorm2, attention_rel, glu,
 * dwconv_ln_silu, conv2d_c1_s2_relu, dwconv2d_s2, flatten_cf, copy_f32, fill_f32, lstm_cell,
 * joint_partial, argmax_reduce (every kernel of src/kernels.metal).
 * Not thread-safe, like the reference: one thread per gpu_t.
 */
#ifndef NEMO_GPU_REF_H
#define NEMO_GPU_REF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gpu gpu_t;
typedef struct gpu_buf gpu_buf_t;

/* src/gpu.h:10-15: a buffer argument (buf + byte offset) or inline parameter bytes */
typedef struct {
    gpu_buf_t *buf;
    size_t offset;
    const void *bytes;
    size_t size;
} gpu_arg_t;

#define GPU_BUF(b, off) ((gpu_arg_t){ (b), (size_t)(off), NULL, 0 })
#define GPU_BYTES(ptr) ((gpu_arg_t){ NULL, 0, (ptr), sizeof *(ptr) })

gpu_t *gpu_create(const char *source, char *err, size_t errlen);
void gpu_destroy(gpu_t *g);
const char *gpu_device_name(gpu_t *g);

gpu_buf_t *gpu_buf_alloc(gpu_t *g, size_t bytes);
void gpu_buf_free(gpu_buf_t *b);
void *gpu_buf_ptr(gpu_buf_t *b);
size_t gpu_buf_len(gpu_buf_t *b);

int gpu_begin(gpu_t *g);
int gpu_dispatch(gpu_t *g, const char *kernel, const gpu_arg_t *args, int nargs, uint32_t gx, uint32_t gy,
                 uint32_t gz, uint32_t tx, uint32_t ty, uint32_t tz);
int gpu_dispatch_groups(gpu_t *g, const char *kernel, const gpu_arg_t *args, int nargs, uint32_t groups_x,
                        uint32_t groups_y, uint32_t groups_z, uint32_t tx, uint32_t ty, uint32_t tz);
int gpu_dispatch_groups_fc(gpu_t *g, const char *kernel, const uint32_t *fc, int nfc, const gpu_arg_t *args,
                           int nargs, uint32_t groups_x, uint32_t groups_y, uint32_t groups_z, uint32_t tx,
                           uint32_t ty, uint32_t tz);
int gpu_end(gpu_t *g, char *err, size_t errlen);
double gpu_last_ms(gpu_t *g);
const char *gpu_last_error(gpu_t *g);

#ifdef __cplusplus
}
#endif
#endif
