/* The allocation-free variant of nk_gemm_split (include/nemo_kernels.h: nk_gemm_split_noalloc).
 *
 * Its split-K scratch is a file-scope device array instead of memory the library allocates, so a
 * caller that must not allocate (code under graph capture, tight serving loops, harnesses that
 * forbid hipMalloc) can still run the K-split GEMMs.  The array lives on every GPU the library
 * runs on until the process ends.  In host code the array's name is only a stand-in: its device
 * address is taken once per device with hipGetSymbolAddress, with that device current, on the first
 * call there, and only that address is passed to kernels.  The array holds the partial rows of a
 * residual update between the GEMM and the fold that applies them; all calls on one GPU share it
 * and overwrite what the last call left (nothing in it has to start at zero), so calls that
 * overlap on one GPU race. */
#include <hip/hip_runtime.h>
#include <pthread.h>
#include <stdio.h>
#include "nemo_kernels.h"

extern "C" int gpu_device_index(const gpu_t *g);
extern "C" int gpu_fail(gpu_t *g, const char *msg);
extern "C" int nk_gemm_split_scratch(gpu_t *g, const float *A, const uint16_t *A2, uint32_t lda, const uint16_t *W,
                                     uint32_t ldw, const float *bias, float *C, uint16_t *C2, uint32_t ldc, const int *crow,
                                     uint32_t M, uint32_t N, uint32_t K, int act, int accumulate, float alpha, float *ws,
                                     size_t ws_floats);

/* partial rows of residual updates */
static __device__ __align__(256) float scratch[NK_NOALLOC_WS_FLOATS];

#define NOALLOC_MAX_DEVICES 64
static float *g_scratch[NOALLOC_MAX_DEVICES]; /* device address of `scratch` per device */
static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;

static float *scratch_on(gpu_t *g) {
    const int dev = gpu_device_index(g);
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return NULL;
    pthread_mutex_lock(&g_lock);
    float *p = g_scratch[dev];
    if (!p) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        if (e == hipSuccess) e = hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) p = NULL;
        if (cur >= 0 && cur != dev) (void)hipSetDevice(cur);
        g_scratch[dev] = p;
    }
    pthread_mutex_unlock(&g_lock);
    return p;
}

extern "C" int nk_gemm_split_noalloc(gpu_t *g, const float *A, const uint16_t *A2, uint32_t lda, const uint16_t *W,
                                     uint32_t ldw, const float *bias, float *C, uint16_t *C2, uint32_t ldc, const int *crow,
                                     uint32_t M, uint32_t N, uint32_t K, int act, int accumulate, float alpha) {
    float *p = scratch_on(g);
    if (!p) return gpu_fail(g, "gemm_split_noalloc: no address for the device scratch array");
    return nk_gemm_split_scratch(g, A, A2, lda, W, ldw, bias, C, C2, ldc, crow, M, N, K, act, accumulate, alpha, p,
                                 NK_NOALLOC_WS_FLOATS);
}
