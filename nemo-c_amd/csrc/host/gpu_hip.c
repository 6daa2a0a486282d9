/* HIP runtime layer for one gfx950 GPU (see gpu.h).  Plain C over the HIP runtime API. */
#include "gpu.h"
#include <errno.h>
#include <hip/hip_runtime_api.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* HIP extension (hip/hip_ext.h, which is C++-only): a module launch whose start / stop events
 * are stamped by the dispatch packet itself. */
hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t lx, uint32_t ly,
                                    uint32_t lz, size_t shared, hipStream_t stream, void **params, void **extra,
                                    hipEvent_t start, hipEvent_t stop, uint32_t flags);

/* gfx950 code object linked into the library (co_blob.S) */
extern const unsigned char nk_code_object_start[];
extern const unsigned char nk_code_object_end[];

#define GPU_MAX_FN 96
#define GPU_MAX_TIMED 32768

struct gpu {
    int dev;
    hipModule_t mod;
    hipStream_t stream;
    hipEvent_t ev0, ev1;
    hipEvent_t evd0, evd1; /* the bracket of a batch ended without waiting (gpu_end_nowait) */
    int deferred;
    double last_ms;
    int in_batch, capturing, failed;
    int many_rows;
    char name[256];
    char err[512];
    struct { char name[48]; hipFunction_t f; } fn[GPU_MAX_FN];
    int nfn;
    float *ws;
    size_t ws_floats;
    uint64_t launches;
    /* constant tables for kernels that take no optional pointers: rows 0..GPU_IOTA_N-1 and zeros */
    int *iota;
    float *zeros;
    /* per-kernel timing */
    char timed[48];
    hipEvent_t *tev;
    double *tbytes, next_bytes, *tflops, next_flops, last_flops;
    int tmax, tn;
    /* buffers with a host mirror (gpu_buf_ptr): uploaded at gpu_begin when the host may have
     * written them, marked device-newer at gpu_end */
    gpu_buf_t *mirrored;
};
struct gpu_buf {
    void *d;
    size_t len;
    gpu_t *g;
    void *host;           /* pinned mirror, allocated by the first gpu_buf_ptr */
    int host_dirty;       /* the host may have written the mirror since the last upload */
    int dev_newer;        /* a batch ended after the last download: the device copy may be newer */
    gpu_buf_t *next_mirrored;
};
struct gpu_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

static int fail(gpu_t *g, const char *what, hipError_t e) {
    if (!g->failed) snprintf(g->err, sizeof g->err, "%s: %s", what, hipGetErrorString(e));
    g->failed = 1;
    return -1;
}

int gpu_fail(gpu_t *g, const char *msg) {
    if (!g->failed) snprintf(g->err, sizeof g->err, "%s", msg);
    g->failed = 1;
    return -1;
}

gpu_t *gpu_create(const char *source, char *err, size_t errlen) {
    /* `source` is the reference's Metal source text (src/model.c:202); this library runs the gfx950
     * code object linked into it, so the argument is accepted and not compiled */
    (void)source;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        snprintf(err, errlen, "no HIP device (%s)", hipGetErrorString(e));
        return NULL;
    }
    hipDeviceProp_t prop;
    if ((e = hipSetDevice(0)) != hipSuccess || (e = hipGetDeviceProperties(&prop, 0)) != hipSuccess) {
        snprintf(err, errlen, "hip device 0: %s", hipGetErrorString(e));
        return NULL;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        snprintf(err, errlen, "device is %s; this build carries gfx950 code only", prop.gcnArchName);
        return NULL;
    }
    gpu_t *g = calloc(1, sizeof *g);
    g->dev = 0;
    snprintf(g->name, sizeof g->name, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    if ((e = hipModuleLoadData(&g->mod, nk_code_object_start)) != hipSuccess) {
        snprintf(err, errlen, "load gfx950 code object: %s", hipGetErrorString(e));
        free(g);
        return NULL;
    }
    if ((e = hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&g->ev0)) != hipSuccess || (e = hipEventCreate(&g->ev1)) != hipSuccess ||
        (e = hipEventCreate(&g->evd0)) != hipSuccess || (e = hipEventCreate(&g->evd1)) != hipSuccess) {
        snprintf(err, errlen, "stream/event: %s", hipGetErrorString(e));
        hipModuleUnload(g->mod);
        free(g);
        return NULL;
    }
    int *iota = malloc(GPU_IOTA_N * sizeof(int));
    for (int i = 0; i < GPU_IOTA_N; ++i) iota[i] = i;
    if ((e = hipMalloc((void **)&g->iota, GPU_IOTA_N * sizeof(int))) != hipSuccess ||
        (e = hipMemcpy(g->iota, iota, GPU_IOTA_N * sizeof(int), hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMalloc((void **)&g->zeros, GPU_ZEROS_N * sizeof(float))) != hipSuccess ||
        (e = hipMemset(g->zeros, 0, GPU_ZEROS_N * sizeof(float))) != hipSuccess ||
        (e = hipMalloc((void **)&g->ws, GPU_SCRATCH_FLOATS * sizeof(float))) != hipSuccess) {
        snprintf(err, errlen, "constant tables: %s", hipGetErrorString(e));
        free(iota);
        gpu_destroy(g);
        return NULL;
    }
    free(iota);
    g->ws_floats = GPU_SCRATCH_FLOATS;
    return g;
}

const int *gpu_iota(gpu_t *g) { return g->iota; }
void gpu_set_many_rows(gpu_t *g, int on) { g->many_rows = on != 0; }
int gpu_many_rows(const gpu_t *g) { return g->many_rows; }
int gpu_device_index(const gpu_t *g) { return g->dev; }

int gpu_cu_count(gpu_t *g) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, g->dev) != hipSuccess) return 0;
    return n;
}

void *gpu_host_dptr(gpu_t *g, void *host) {
    void *d = NULL;
    (void)g;
    if (!host || hipHostGetDevicePointer(&d, host, 0) != hipSuccess) return NULL;
    return d;
}
const float *gpu_zeros(gpu_t *g) { return g->zeros; }

void gpu_destroy(gpu_t *g) {
    if (!g) return;
    hipStreamSynchronize(g->stream);
    if (g->tev) {
        for (int i = 0; i < 2 * g->tmax; ++i) hipEventDestroy(g->tev[i]);
        free(g->tev);
        free(g->tbytes);
    }
    if (g->ws) hipFree(g->ws);
    if (g->iota) hipFree(g->iota);
    if (g->zeros) hipFree(g->zeros);
    hipEventDestroy(g->ev0);
    hipEventDestroy(g->ev1);
    hipEventDestroy(g->evd0);
    hipEventDestroy(g->evd1);
    hipStreamDestroy(g->stream);
    hipModuleUnload(g->mod);
    free(g);
}

const char *gpu_device_name(gpu_t *g) { return g->name; }
const char *gpu_last_error(gpu_t *g) { return g->err; }
double gpu_last_ms(gpu_t *g) { return g->last_ms; }
uint64_t gpu_launch_count(const gpu_t *g) { return g->launches; }
int gpu_capturing(const gpu_t *g) { return g->capturing; }

gpu_buf_t *gpu_buf_alloc(gpu_t *g, size_t bytes) {
    gpu_buf_t *b = calloc(1, sizeof *b);
    b->len = bytes ? bytes : 256;
    b->g = g;
    if (hipMalloc(&b->d, b->len) != hipSuccess) { free(b); return NULL; }
    if (hipMemset(b->d, 0, b->len) != hipSuccess) { hipFree(b->d); free(b); return NULL; }
    return b;
}
void gpu_buf_free(gpu_buf_t *b) {
    if (!b) return;
    if (b->host) {
        for (gpu_buf_t **p = &b->g->mirrored; *p; p = &(*p)->next_mirrored)
            if (*p == b) { *p = b->next_mirrored; break; }
        hipHostFree(b->host);
    }
    hipFree(b->d);
    free(b);
}

/* Host address of a buffer, as src/gpu.h:26 gives for Metal's shared storage.  Here the buffer
 * lives in device memory and the address is a pinned mirror of it, kept coherent at batch edges:
 *   - the mirror is refreshed from the device when a batch has ended since the last refresh;
 *   - every call marks the mirror as possibly written, and gpu_begin uploads such mirrors before
 *     the batch's first launch.
 * So the host reads results and writes inputs between batches through a pointer taken after the
 * last gpu_end (the reference's own discipline: no command buffer is in flight while the host
 * touches shared buffers).  Writes through a pointer taken before a later gpu_end are not seen.
 * The product path never calls this (it uses gpu_upload / gpu_download on device addresses). */
void *gpu_buf_ptr(gpu_buf_t *b) {
    if (!b) return NULL;
    gpu_t *g = b->g;
    if (!b->host) {
        if (hipHostMalloc(&b->host, b->len, hipHostMallocDefault) != hipSuccess) {
            b->host = NULL;
            gpu_fail(g, "gpu_buf_ptr: pinned host mirror unavailable");
            return NULL;
        }
        b->dev_newer = 1;
        b->next_mirrored = g->mirrored;
        g->mirrored = b;
    }
    if (b->dev_newer) {
        hipError_t e = hipStreamSynchronize(g->stream);
        if (e == hipSuccess) e = hipMemcpy(b->host, b->d, b->len, hipMemcpyDeviceToHost);
        if (e != hipSuccess) { fail(g, "gpu_buf_ptr refresh", e); return NULL; }
        b->dev_newer = 0;
    }
    b->host_dirty = 1;
    return b->host;
}

/* before a batch: device copies of the mirrors the host may have written */
static int upload_mirrors(gpu_t *g) {
    for (gpu_buf_t *b = g->mirrored; b; b = b->next_mirrored) {
        if (!b->host_dirty) continue;
        hipError_t e = hipMemcpyAsync(b->d, b->host, b->len, hipMemcpyHostToDevice, g->stream);
        if (e != hipSuccess) return fail(g, "gpu_begin: mirror upload", e);
        b->host_dirty = 0;
    }
    return 0;
}
static void mirrors_dev_newer(gpu_t *g) {
    for (gpu_buf_t *b = g->mirrored; b; b = b->next_mirrored) b->dev_newer = 1;
}
void *gpu_buf_dptr(gpu_buf_t *b) { return b ? b->d : NULL; }
size_t gpu_buf_len(gpu_buf_t *b) { return b->len; }

void *gpu_host_alloc(gpu_t *g, size_t bytes) {
    void *p = NULL;
    (void)g;
    if (hipHostMalloc(&p, bytes ? bytes : 64, hipHostMallocDefault) != hipSuccess) return NULL;
    memset(p, 0, bytes ? bytes : 64);
    return p;
}
void gpu_host_free(void *p) { if (p) hipHostFree(p); }

int gpu_upload(gpu_t *g, void *dst, const void *src, size_t n) {
    if (!n) return 0;
    hipError_t e = hipMemcpy(dst, src, n, hipMemcpyHostToDevice);
    return e == hipSuccess ? 0 : fail(g, "upload", e);
}
int gpu_download(gpu_t *g, void *dst, const void *src, size_t n) {
    if (!n) return 0;
    hipError_t e = hipStreamSynchronize(g->stream);
    if (e != hipSuccess) return fail(g, "download sync", e);
    e = hipMemcpy(dst, src, n, hipMemcpyDeviceToHost);
    return e == hipSuccess ? 0 : fail(g, "download", e);
}
int gpu_upload_async(gpu_t *g, void *dst, const void *src, size_t n) {
    if (!n) return 0;
    hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g->stream);
    return e == hipSuccess ? 0 : fail(g, "upload_async", e);
}
int gpu_download_async(gpu_t *g, void *dst, const void *src, size_t n) {
    if (!n) return 0;
    hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, g->stream);
    return e == hipSuccess ? 0 : fail(g, "download_async", e);
}

/* ---- file -> device loader ---------------------------------------------------------------- */

#define UPF_THREADS 4
#define UPF_SLOTS 2             /* staging slots per reader thread */
#define UPF_PIECE (8u << 20)    /* bytes per slot */

typedef struct {
    uint64_t off, bytes;
    char *dst;
} upf_piece_t;

typedef struct {
    gpu_t *g;
    int fd;
    const upf_piece_t *pc;
    size_t npc;
    char *stage;
    hipEvent_t ev[UPF_THREADS * UPF_SLOTS];
    pthread_mutex_t mu;
    size_t next;   /* next piece to take (under mu) */
    int failed;    /* set under mu; readers stop taking pieces */
    char msg[200];
} upf_t;

typedef struct {
    upf_t *u;
    int id;
} upf_worker_t;

static void upf_error(upf_t *u, const char *msg) {
    pthread_mutex_lock(&u->mu);
    if (!u->failed) snprintf(u->msg, sizeof u->msg, "%s", msg);
    u->failed = 1;
    pthread_mutex_unlock(&u->mu);
}

static void *upf_reader(void *arg) {
    const upf_worker_t *w = arg;
    upf_t *u = w->u;
    hipError_t e = hipSetDevice(u->g->dev);
    if (e != hipSuccess) { upf_error(u, hipGetErrorString(e)); return NULL; }
    int used[UPF_SLOTS] = { 0 }, k = 0;
    for (;;) {
        pthread_mutex_lock(&u->mu);
        const size_t i = u->failed ? u->npc : u->next++;
        pthread_mutex_unlock(&u->mu);
        if (i >= u->npc) break;
        const int slot = w->id * UPF_SLOTS + k;
        char *buf = u->stage + (size_t)slot * UPF_PIECE;
        if (used[k] && (e = hipEventSynchronize(u->ev[slot])) != hipSuccess) { upf_error(u, hipGetErrorString(e)); break; }
        const upf_piece_t *p = &u->pc[i];
        uint64_t got = 0;
        while (got < p->bytes) {
            const ssize_t r = pread(u->fd, buf + got, (size_t)(p->bytes - got), (off_t)(p->off + got));
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) {
                char msg[96];
                if (r < 0) snprintf(msg, sizeof msg, "weight file read failed (errno %d)", errno);
                else snprintf(msg, sizeof msg, "weight file shorter than its header says");
                upf_error(u, msg);
                return NULL;
            }
            got += (uint64_t)r;
        }
        if ((e = hipMemcpyAsync(p->dst, buf, p->bytes, hipMemcpyHostToDevice, u->g->stream)) != hipSuccess ||
            (e = hipEventRecord(u->ev[slot], u->g->stream)) != hipSuccess) {
            upf_error(u, hipGetErrorString(e));
            break;
        }
        used[k] = 1;
        k = (k + 1) % UPF_SLOTS;
    }
    return NULL;
}

int gpu_upload_file(gpu_t *g, int fd, const gpu_file_range_t *ranges, size_t n) {
    size_t npc = 0;
    for (size_t i = 0; i < n; ++i) npc += (size_t)((ranges[i].bytes + UPF_PIECE - 1) / UPF_PIECE);
    if (!npc) return 0;
    upf_t u = { .g = g, .fd = fd, .npc = npc };
    upf_piece_t *pc = malloc(npc * sizeof *pc);
    if (!pc) return gpu_fail(g, "upload_file: out of host memory");
    size_t j = 0;
    for (size_t i = 0; i < n; ++i)
        for (uint64_t o = 0; o < ranges[i].bytes; o += UPF_PIECE) {
            const uint64_t b = ranges[i].bytes - o < UPF_PIECE ? ranges[i].bytes - o : UPF_PIECE;
            pc[j++] = (upf_piece_t){ ranges[i].off + o, b, (char *)ranges[i].dst + o };
        }
    u.pc = pc;
    /* work queued elsewhere on the device (the zero fill of fresh buffers) lands first */
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) { free(pc); return fail(g, "upload_file sync", e); }
    const int nthr = npc < UPF_THREADS ? (int)npc : UPF_THREADS;
    e = hipHostMalloc((void **)&u.stage, (size_t)nthr * UPF_SLOTS * UPF_PIECE, hipHostMallocDefault);
    if (e != hipSuccess) { free(pc); return fail(g, "staging buffer", e); }
    int nev = 0;
    while (nev < nthr * UPF_SLOTS && (e = hipEventCreateWithFlags(&u.ev[nev], hipEventDisableTiming)) == hipSuccess) ++nev;
    pthread_mutex_init(&u.mu, NULL);
    pthread_t th[UPF_THREADS];
    upf_worker_t wk[UPF_THREADS];
    int started = 0;
    if (nev == nthr * UPF_SLOTS)
        for (; started < nthr; ++started) {
            wk[started] = (upf_worker_t){ &u, started };
            if (pthread_create(&th[started], NULL, upf_reader, &wk[started])) break;
        }
    else
        upf_error(&u, hipGetErrorString(e));
    if (started == 0 && !u.failed) upf_error(&u, "cannot start a reader thread");
    for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
    /* the readers have queued every copy they took; wait for them before the staging goes */
    e = hipStreamSynchronize(g->stream);
    if (e != hipSuccess) upf_error(&u, hipGetErrorString(e));
    for (int i = 0; i < nev; ++i) hipEventDestroy(u.ev[i]);
    hipHostFree(u.stage);
    pthread_mutex_destroy(&u.mu);
    free(pc);
    if (u.failed) return gpu_fail(g, u.msg);
    return 0;
}

static hipFunction_t lookup(gpu_t *g, const char *kernel) {
    for (int i = 0; i < g->nfn; ++i)
        if (!strcmp(g->fn[i].name, kernel)) return g->fn[i].f;
    hipFunction_t f = NULL;
    hipError_t e = hipModuleGetFunction(&f, g->mod, kernel);
    if (e != hipSuccess) {
        char what[96];
        snprintf(what, sizeof what, "kernel %s", kernel);
        fail(g, what, e);
        return NULL;
    }
    if (g->nfn < GPU_MAX_FN) {
        snprintf(g->fn[g->nfn].name, sizeof g->fn[g->nfn].name, "%s", kernel);
        g->fn[g->nfn].f = f;
        g->nfn++;
    }
    return f;
}

/* timing selection: an exact kernel name, or a prefix ending in '*' */
static int timed_name(const char *sel, const char *kernel) {
    const size_t n = strlen(sel);
    if (n && sel[n - 1] == '*') return !strncmp(sel, kernel, n - 1);
    return !strcmp(sel, kernel);
}

int gpu_begin(gpu_t *g) {
    g->failed = 0;
    g->err[0] = 0;
    g->in_batch = 1;
    if (g->mirrored && upload_mirrors(g)) return -1;
    hipError_t e = hipEventRecord(g->ev0, g->stream);
    return e == hipSuccess ? 0 : fail(g, "begin", e);
}

int gpu_launch(gpu_t *g, const char *kernel, const void *args, size_t args_size,
               uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t by, uint32_t bz) {
    if (!gx || !gy || !gz) return 0;
    hipFunction_t f = lookup(g, kernel);
    if (!f) return -1;
    /* Every kernel takes one by-value struct: its address is the one entry of kernelParams.  The
     * runtime copies the argument block into the launch (and into the graph node when the stream
     * is being captured), so the caller's struct may go out of scope right after this call. */
    (void)args_size;
    void *kp[] = { (void *)args };
    const int timed = !g->capturing && g->tev && g->tn < g->tmax && timed_name(g->timed, kernel);
    hipError_t e;
    if (timed) {
        /* the start / stop events are stamped by the dispatch itself: the kernel's execution time */
        e = hipExtModuleLaunchKernel(f, gx * bx, gy * by, gz * bz, bx, by, bz, 0, g->stream, kp, NULL,
                                     g->tev[2 * g->tn], g->tev[2 * g->tn + 1], 0);
        g->tbytes[g->tn] = g->next_bytes;
        g->tflops[g->tn] = g->next_flops;
        g->tn++;
    } else {
        e = hipModuleLaunchKernel(f, gx, gy, gz, bx, by, bz, 0, g->stream, kp, NULL);
    }
    g->next_bytes = 0.0;
    g->next_flops = 0.0;
    g->launches++;
    if (e != hipSuccess) {
        char what[96];
        snprintf(what, sizeof what, "launch %s", kernel);
        return fail(g, what, e);
    }
    return 0;
}

int gpu_sync(gpu_t *g) {
    hipError_t e = hipStreamSynchronize(g->stream);
    return e == hipSuccess ? 0 : fail(g, "sync", e);
}

int gpu_end(gpu_t *g, char *err, size_t errlen) {
    hipError_t e = hipEventRecord(g->ev1, g->stream);
    if (e == hipSuccess) e = hipEventSynchronize(g->ev1);
    if (e != hipSuccess) fail(g, "end", e);
    float ms = 0.0f;
    if (!g->failed && hipEventElapsedTime(&ms, g->ev0, g->ev1) == hipSuccess) g->last_ms = ms;
    g->in_batch = 0;
    mirrors_dev_newer(g);
    if (g->failed) {
        if (errlen) snprintf(err, errlen, "gpu: %s", g->err);
        return -1;
    }
    return 0;
}

int gpu_end_nowait(gpu_t *g, char *err, size_t errlen) {
    if (g->deferred) gpu_wait_deferred(g); /* one deferred bracket at a time */
    hipError_t e = hipEventRecord(g->ev1, g->stream);
    if (e != hipSuccess) fail(g, "end", e);
    g->in_batch = 0;
    mirrors_dev_newer(g);
    if (g->failed) {
        if (errlen) snprintf(err, errlen, "gpu: %s", g->err);
        return -1;
    }
    hipEvent_t t0 = g->evd0, t1 = g->evd1;
    g->evd0 = g->ev0;
    g->evd1 = g->ev1;
    g->ev0 = t0;
    g->ev1 = t1;
    g->deferred = 1;
    return 0;
}

double gpu_wait_deferred(gpu_t *g) {
    if (!g->deferred) return 0.0;
    g->deferred = 0;
    float ms = 0.0f;
    if (hipEventSynchronize(g->evd1) != hipSuccess || hipEventElapsedTime(&ms, g->evd0, g->evd1) != hipSuccess) return 0.0;
    return ms;
}

int gpu_capture_begin(gpu_t *g) {
    hipError_t e = hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return fail(g, "capture begin", e);
    g->capturing = 1;
    return 0;
}

gpu_graph_t *gpu_capture_end(gpu_t *g) {
    gpu_graph_t *gr = calloc(1, sizeof *gr);
    hipError_t e = hipStreamEndCapture(g->stream, &gr->graph);
    g->capturing = 0;
    if (e != hipSuccess) { fail(g, "capture end", e); free(gr); return NULL; }
    if (g->failed) { hipGraphDestroy(gr->graph); free(gr); return NULL; }
    e = hipGraphInstantiate(&gr->exec, gr->graph, NULL, NULL, 0);
    if (e != hipSuccess) { fail(g, "graph instantiate", e); hipGraphDestroy(gr->graph); free(gr); return NULL; }
    return gr;
}

int gpu_graph_launch(gpu_t *g, gpu_graph_t *gr) {
    hipError_t e = hipGraphLaunch(gr->exec, g->stream);
    return e == hipSuccess ? 0 : fail(g, "graph launch", e);
}

void gpu_graph_free(gpu_graph_t *gr) {
    if (!gr) return;
    hipGraphExecDestroy(gr->exec);
    hipGraphDestroy(gr->graph);
    free(gr);
}

float *gpu_scratch_ws(gpu_t *g, size_t floats) {
    if (floats > g->ws_floats) {
        if (g->capturing) return NULL;
        hipStreamSynchronize(g->stream);
        float *p = NULL;
        if (hipMalloc((void **)&p, floats * sizeof(float)) != hipSuccess) return NULL;
        if (g->ws) hipFree(g->ws);
        g->ws = p;
        g->ws_floats = floats;
    }
    return g->ws;
}

int gpu_timing_set(gpu_t *g, const char *kernel, int max_launches) {
    if (g->tev) {
        for (int i = 0; i < 2 * g->tmax; ++i) hipEventDestroy(g->tev[i]);
        free(g->tev);
        free(g->tbytes);
        free(g->tflops);
        g->tev = NULL;
        g->tbytes = NULL;
        g->tflops = NULL;
    }
    g->tn = g->tmax = 0;
    g->timed[0] = 0;
    if (!kernel || max_launches <= 0) return 0;
    if (max_launches > GPU_MAX_TIMED) max_launches = GPU_MAX_TIMED;
    g->tev = calloc((size_t)max_launches * 2, sizeof(hipEvent_t));
    g->tbytes = calloc((size_t)max_launches, sizeof(double));
    g->tflops = calloc((size_t)max_launches, sizeof(double));
    for (int i = 0; i < 2 * max_launches; ++i)
        if (hipEventCreate(&g->tev[i]) != hipSuccess) return fail(g, "timing events", hipErrorOutOfMemory);
    g->tmax = max_launches;
    snprintf(g->timed, sizeof g->timed, "%s", kernel);
    return 0;
}

void gpu_next_bytes(gpu_t *g, double bytes) { g->next_bytes = bytes; }
void gpu_next_flops(gpu_t *g, double flops) { g->next_flops = flops; }
double gpu_timing_last_flops(const gpu_t *g) { return g->last_flops; }

int gpu_timing_collect(gpu_t *g, double *mean_ms, int *count, double *bytes) {
    *mean_ms = 0.0;
    *count = 0;
    if (bytes) *bytes = 0.0;
    if (!g->tev) return 0;
    hipStreamSynchronize(g->stream);
    double sum = 0.0;
    g->last_flops = 0.0;
    for (int i = 0; i < g->tn; ++i) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, g->tev[2 * i], g->tev[2 * i + 1]) != hipSuccess) return fail(g, "timing", hipErrorInvalidValue);
        sum += ms;
        if (bytes) *bytes += g->tbytes[i];
        g->last_flops += g->tflops[i];
    }
    *count = g->tn;
    *mean_ms = g->tn ? sum / g->tn : 0.0;
    g->tn = 0;
    return 0;
}
