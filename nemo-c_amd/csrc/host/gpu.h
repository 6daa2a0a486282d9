/* Thin C interface over the HIP runtime for one gfx950 GPU: device memory, the embedded kernel
 * code object, ordered launches on one stream, hipGraph capture and timing.
 *
 * Replaces the Metal layer of the reference (src/gpu.h:1-43, src/gpu.m:1-141):
 *   - gpu_create loads a gfx950 code object built at compile time (hipModuleLoadData) instead of
 *     compiling Metal source at run time; kernels are looked up by name and cached, which takes
 *     the place of the reference's pipeline cache keyed by name + function constants
 *     (src/gpu.m:63-87); specialisations are separate kernel symbols.
 *   - Buffers are device memory (zero-filled at allocation).  The reference's shared-storage
 *     pointer access is replaced by explicit stream-ordered uploads and downloads.
 *   - gpu_begin / gpu_end bracket ordered work on one stream; gpu_end waits for completion and
 *     reports the GPU time of the batch from hipEvents (src/gpu.m:124-139).
 * Single-threaded, like the reference.
 */
#ifndef NEMO_GPU_H
#define NEMO_GPU_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gpu gpu_t;
typedef struct gpu_buf gpu_buf_t;
typedef struct gpu_graph gpu_graph_t;

/* `source`: the reference passes its Metal source text here (src/gpu.h:20); the gfx950 code
 * object linked into this library is used instead and the argument is not read (NULL is fine). */
gpu_t *gpu_create(const char *source, char *err, size_t errlen);
void gpu_destroy(gpu_t *g);
const char *gpu_device_name(gpu_t *g);

gpu_buf_t *gpu_buf_alloc(gpu_t *g, size_t bytes); /* device memory, zero-filled; 0 bytes -> 256 */
void gpu_buf_free(gpu_buf_t *b);
void *gpu_buf_dptr(gpu_buf_t *b);                 /* device address */
size_t gpu_buf_len(gpu_buf_t *b);
/* Host address of a pinned mirror of the buffer (src/gpu.h:26), coherent at batch edges: refreshed
 * from the device when a batch has ended since, uploaded by the next gpu_begin. */
void *gpu_buf_ptr(gpu_buf_t *b);

/* pinned host memory for the host<->device staging on the hot path */
void *gpu_host_alloc(gpu_t *g, size_t bytes);
void gpu_host_free(void *p);

/* Synchronous copies (outside the hot path: load time, tests). */
int gpu_upload(gpu_t *g, void *dst_dev, const void *src, size_t n);
int gpu_download(gpu_t *g, void *dst, const void *src_dev, size_t n);
/* Stream-ordered copies between pinned host memory and the device (inside begin/end). */
int gpu_upload_async(gpu_t *g, void *dst_dev, const void *src_pinned, size_t n);
int gpu_download_async(gpu_t *g, void *dst_pinned, const void *src_dev, size_t n);

/* Load-time copy of byte ranges of an open file into device memory, synchronous: reader threads
 * pread pieces of at most a few MiB into pinned staging slots and queue each slot's copy
 * asynchronously; a slot is refilled once its copy has completed, so the disk or page-cache
 * reads overlap the PCIe transfers.  Returns 0, or -1 with the error in gpu_last_error. */
typedef struct {
    uint64_t off;   /* file offset */
    uint64_t bytes;
    void *dst;      /* device address */
} gpu_file_range_t;
int gpu_upload_file(gpu_t *g, int fd, const gpu_file_range_t *ranges, size_t n);

int gpu_begin(gpu_t *g);
/* Launch `kernel` with one by-value argument block of `args_size` bytes; grid in workgroups. */
int gpu_launch(gpu_t *g, const char *kernel, const void *args, size_t args_size,
               uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t by, uint32_t bz);
int gpu_end(gpu_t *g, char *err, size_t errlen);
/* End the batch without waiting for it: later work on the stream queues behind it at once.  The
 * host must not reuse what the batch reads from host memory (pinned staging) before
 * gpu_wait_deferred, which waits for that batch and returns its GPU time in ms (0 when none is
 * pending).  Launch errors already recorded are reported here, execution errors by the next end. */
int gpu_end_nowait(gpu_t *g, char *err, size_t errlen);
double gpu_wait_deferred(gpu_t *g);
double gpu_last_ms(gpu_t *g);
const char *gpu_last_error(gpu_t *g);
int gpu_sync(gpu_t *g);
/* Record an error for the current batch (gpu_end then fails with it); returns -1. */
int gpu_fail(gpu_t *g, const char *msg);

/* hipGraph capture of the launches between capture_begin and capture_end (inside begin/end). */
int gpu_capture_begin(gpu_t *g);
gpu_graph_t *gpu_capture_end(gpu_t *g);
int gpu_graph_launch(gpu_t *g, gpu_graph_t *gr);
void gpu_graph_free(gpu_graph_t *gr);
int gpu_capturing(const gpu_t *g);

/* Scratch of the split-K partial rows (GPU_SCRATCH_FLOATS allocated at creation): a larger request
 * grows it outside a capture and returns NULL (no error recorded) inside one.  Launches on one
 * gpu_t run in stream order, so they share it; it holds one pending residual update at a time. */
#define GPU_SCRATCH_FLOATS (1u << 20)
float *gpu_scratch_ws(gpu_t *g, size_t floats_needed);

/* Per-kernel timing on the launch stream: when a name is set, every launch of that kernel is
 * bracketed by a pair of hipEvents; gpu_timing_collect returns the mean duration in ms. */
int gpu_timing_set(gpu_t *g, const char *kernel, int max_launches);
int gpu_timing_collect(gpu_t *g, double *mean_ms, int *count, double *bytes);
/* Algorithmic HBM bytes and flops of the next launch (recorded with its timing); the flops of
 * the launches summed by the last gpu_timing_collect. */
void gpu_next_bytes(gpu_t *g, double bytes);
void gpu_next_flops(gpu_t *g, double flops);
double gpu_timing_last_flops(const gpu_t *g);

/* Device constant tables: the row indices 0..GPU_IOTA_N-1 and GPU_ZEROS_N zero floats (kernels
 * whose row map or bias is optional get these instead of NULL). */
#define GPU_IOTA_N 4096
#define GPU_ZEROS_N 8192
const int *gpu_iota(gpu_t *g);
const float *gpu_zeros(gpu_t *g);

/* Row policy of the kernel launchers on this context: 0 (default) picks GEMM and LayerNorm kernels by
 * row count; 1 always uses the many-row kernels (batched streams: every row's arithmetic is then
 * the same whatever the number of rows in the launch). */
void gpu_set_many_rows(gpu_t *g, int on);
/* HIP device index the context runs on. */
int gpu_device_index(const gpu_t *g);
/* Compute units of the device (0 when the query fails). */
int gpu_cu_count(gpu_t *g);
/* Device address of pinned host memory from gpu_host_alloc (kernels may store into it). */
void *gpu_host_dptr(gpu_t *g, void *host);
int gpu_many_rows(const gpu_t *g);

/* Number of kernel launches issued since creation (for tests and the launch-count check). */
uint64_t gpu_launch_count(const gpu_t *g);

#ifdef __cplusplus
}
#endif
#endif
