/* Kernel launchers and the GEMM kernel policy (see include/nemo_kernels.h).
 * Host-side shape and alignment checks turn unsupported arguments into errors before any
 * launch, so a kernel never sees a shape its grid or indexing does not cover. */
#include "nemo_kernels.h"
#include "gpu.h"
#include "../kernel_params.h"
#include <stdio.h>
#include <string.h>

static int g_force = 0;
static int g_split = -1; /* many-row residual updates: -1 K split chosen by tile count, 0 never, 1 always */
static int g_mx_tile = -1; /* many-row tile: -1 by tile count, else 0 128x128, 1 64x128, 2 64x64 where it divides */

int nk_gemm_mx_tile(int t) {
    const int prev = g_mx_tile;
    g_mx_tile = t < 0 || t > 2 ? -1 : t;
    return prev;
}

int nk_gemm_ksplit(int mode) {
    const int prev = g_split;
    g_split = mode < 0 ? -1 : mode > 0 ? 1 : 0;
    return prev;
}

/* Blocks of the many-row residual updates' K sum, a function of K alone (so a row's result does
 * not depend on how many rows share the launch): 2 blocks of 512 for K = 1024, K/1024 blocks for
 * larger multiples of 1024, else one. */
static uint32_t mx_kblocks(uint32_t K) {
    if (K == 1024) return 2;
    if (K >= 2048 && K % 1024 == 0 && K / 1024 <= 8) return K / 1024;
    return 1;
}

int nk_gemm_force(int kind) {
    int prev = g_force;
    g_force = kind;
    return prev;
}

/* argument errors are recorded like launch failures: gpu_end then reports them */
static int bad(gpu_t *g, const char *what) { return gpu_fail(g, what); }

static int aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

enum { K_FR = 2, K_MR = 3, K_GEMV = 4, K_MM_OLD = 5 };

/* few-row MFMA kernel plan: W wavefronts of SPW K steps (32 wide) per workgroup, K split over KS
 * workgroups (KS > 1 only for accumulating GEMMs with no bias and no activation, whose shares are
 * written as partial rows and added into C in share order by resid_fold; it puts four times as
 * many workgroups on the small-N matrices). */
typedef struct { uint32_t W, SPW, KS; } fr_plan_t;

static int fr_ok(uint32_t M, uint32_t K, int act) {
    return M <= NK_FEW_ROWS && K % 32 == 0 && K <= 4608 && (act != NK_ACT_GLU || K <= 1024);
}

static int g_fr_ksplit = 1; /* few-row residual updates: K split over four workgroups (1) or not (0) */

int nk_gemm_fr_ksplit(int on) {
    const int prev = g_fr_ksplit;
    g_fr_ksplit = on != 0;
    return prev;
}

static fr_plan_t fr_plan(uint32_t nout, uint32_t K, int act, int accumulate, int has_bias, int ln) {
    const uint32_t S = K / 32;
    fr_plan_t p = { 4, 8, 1 };
    if (ln) { /* K == 1024: eight wavefronts of four K steps (two LayerNorm rows each) */
        p.W = 8;
        p.SPW = 4;
        return p;
    }
    if (act == NK_ACT_GLU) return p;
    if (g_fr_ksplit && accumulate && act == NK_ACT_NONE && !has_bias && (nout + 15) / 16 < 128 && S % 4 == 0 &&
        S / 4 <= 32) {
        p.KS = 4;
        p.SPW = S / 4 <= 8 ? 2 : 8;
        return p;
    }
    if (S <= 32) return p;
    if (S <= 64) { p.W = 8; return p; }
    p.W = 16;
    p.SPW = S <= 128 ? 8 : 9;
    return p;
}

static const char *fr_name(fr_plan_t p, int act, int ln, int fold) {
    static char buf[40];
    /* the LayerNorm-fused GLU kernels pack 8 value / gate row pairs into one MFMA operand */
    snprintf(buf, sizeof buf, "gemm_fr%s%s_w%us%u%s", ln ? "_ln" : "",
             act == NK_ACT_GLU ? (ln ? "_glu8" : "_glu") : "", p.W, p.SPW, fold ? "_f" : "");
    return buf;
}

static int pick(uint32_t M, uint32_t N, uint32_t K, int act) {
    /* 5-8 rows: the 1024-row matrices (one weight row per wavefront, 256 workgroups: one per CU),
     * measured faster than the few-row MFMA kernel there (out / pw2 at 7 rows 5.0 against 5.9 us);
     * 640 rows (160 workgroups) were not */
    const int gemv_ok = (M <= 2 && K <= 64 * 8 * 9) || (M <= 4 && K <= 64 * 8 * 2) ||
                        (M <= 8 && K <= 64 * 8 * 2 && N == 1024 && act != NK_ACT_GLU);
    if ((g_force == K_GEMV || g_force == 1) && gemv_ok) return K_GEMV;
    if (g_force == K_FR && fr_ok(M, K, act)) return K_FR;
    if ((g_force == K_MR || g_force == K_MM_OLD) && K % 32 == 0) return K_MR;
    /* 3-4 rows of the wide matrices (N >= 3072: QKV, FF up): the few-row MFMA kernel, measured
     * faster than the GEMV there (QKV at 4 rows 6.1 against 10.1 us, FF up 6.5 against 8.2 us);
     * the narrower ones stay on the GEMV (pw1 5.9 against 7.1 us, out 3.7 against 5.9 us) */
    if (gemv_ok && M >= 3 && N >= 3072 && fr_ok(M, K, act)) return K_FR;
    if (gemv_ok) return K_GEMV;
    if (fr_ok(M, K, act)) return K_FR;
    return K_MR;
}

/* weight-streaming GEMV shape: chunks per lane per row (KCH) and weight rows per wavefront (NC) */
static void gemv_shape(uint32_t N, uint32_t K, int act, uint32_t *kch, uint32_t *nc) {
    const uint32_t nch = K / 8;
    *kch = nch <= 64 ? 1 : nch <= 128 ? 2 : nch <= 256 ? 4 : nch <= 512 ? 8 : 9;
    if (act == NK_ACT_GLU) { *nc = (*kch <= 4 && N / 2 >= 2048) ? 4 : 2; return; }
    const uint32_t maxnc = *kch <= 4 ? 4 : 2;
    *nc = (N >= 4096 && maxnc >= 4) ? 4 : (N >= 2048 ? 2 : 1);
}

const char *nk_gemm_kernel_name(uint32_t M, uint32_t N, uint32_t K, int act) {
    static char buf[32];
    uint32_t kch, nc;
    switch (pick(M, N, K, act)) {
    case K_GEMV:
        gemv_shape(N, K, act, &kch, &nc);
        snprintf(buf, sizeof buf, "gemv_r%u_n%u_k%u", M, nc, kch);
        return buf;
    case K_FR: return fr_name(fr_plan(act == NK_ACT_GLU ? N / 2 : N, K, act, 0, 1, 0), act, 0, 0);
    default: return "gemm_m*";
    }
}

typedef struct {
    int mode;
    const float *g1, *b1, *g2, *b2;
    float *out, *tmp;
    float eps;
    const nk_resid_t *pend; /* a pending residual update applied to A first (may be NULL) */
    float *fold_out;        /* receives A with the update applied */
} ln_pro_t;

/* Many-row GEMM on the direct-to-LDS MFMA kernels (kernels/nk_mx.hip).  Tile choice: the largest
 * of 128x128, 64x128, 64x64 whose tile count reaches about 400 workgroups; otherwise the smallest
 * tile that divides the output columns.  Residual updates (accumulate, no bias, no activation, no
 * row map) run on the _acc kernels: their K sum is blocked (mx_kblocks), below ~400 tiles K is
 * split one block per workgroup, and the sums go to partial rows in the scratch (nparts of them,
 * same bits either way); *pend then describes the update still to apply (NkFoldArgs).
 * Returns 1 when no tile divides the output columns (the caller falls back), -2 when a fixed
 * scratch region is too small, else the launch status. */
typedef struct {
    float *ws; /* fixed region (no allocation; a launch that needs more is refused), or NULL */
    size_t ws_floats;
} mx_scratch_t;

static int launch_mx_s(gpu_t *g, NkGemmArgs *a, uint32_t M, uint32_t nout, uint32_t K, int glu, int resid,
                       const mx_scratch_t *sc, nk_resid_t *pend) {
    /* split-row A (_s) and split-row outputs (_so) variants */
    const char *sfx = a->A2 ? (a->C2 ? "_s_so" : "_s") : (a->C2 ? "_so" : "");
    static const struct { const char *name, *glu_name, *acc_name; uint32_t bm, bn; } cfg[] = {
        { "gemm_mx128x128", "gemm_mx128x128_glu", "gemm_mx128x128_acc", 128, 128 },
        { "gemm_mx64x128", "gemm_mx64x128_glu", "gemm_mx64x128_acc", 64, 128 },
        { "gemm_mx64x64", "gemm_mx64x64_glu", "gemm_mx64x64_acc", 64, 64 },
    };
    int pick_i = -1, last_ok = -1;
    uint32_t tiles = 0;
    const uint32_t kb = resid ? mx_kblocks(K) : 1;
    for (int i = 0; i < 3; ++i) {
        const uint32_t cols = glu ? cfg[i].bn / 2 : cfg[i].bn;
        if (nout % cols) continue;
        const uint32_t t = ((M + cfg[i].bm - 1) / cfg[i].bm) * (nout / cols);
        if (cfg[i].bm == 128 && (M < 512 || a->A2)) continue; /* split rows: one workgroup per CU */
        last_ok = i;
        /* two workgroups per CU: the largest tile with at least ~400 workgroups (residual updates:
         * tiles x K blocks, the split below) was the fastest at every measured shape (448 to 3584
         * rows, N 1024 to 4096, K 1024 and 4096) */
        if ((a->A2 ? t * kb : t) >= 400) { pick_i = i; tiles = t; break; }
    }
    if (last_ok < 0) return 1;
    if (g_mx_tile >= 0 && nout % (glu ? cfg[g_mx_tile].bn / 2 : cfg[g_mx_tile].bn) == 0) pick_i = g_mx_tile;
    if (pick_i >= 0) {
        const uint32_t cols = glu ? cfg[pick_i].bn / 2 : cfg[pick_i].bn;
        tiles = ((M + cfg[pick_i].bm - 1) / cfg[pick_i].bm) * (nout / cols);
    }
    if (pick_i < 0) {
        pick_i = last_ok;
        const uint32_t cols = glu ? cfg[pick_i].bn / 2 : cfg[pick_i].bn;
        tiles = ((M + cfg[pick_i].bm - 1) / cfg[pick_i].bm) * (nout / cols);
    }
    uint32_t kz = 1;
    a->kblocks = 1;
    if (resid) {
        a->kblocks = mx_kblocks(K);
        /* split below ~400 tiles (measured on 64 x 64 tiles: about 448 workgroups at 448 rows) */
        if (a->kblocks > 1 && (g_split == 1 || (g_split < 0 && tiles < 400))) kz = a->kblocks;
        const size_t need = (size_t)kz * M * nout;
        if (sc && sc->ws) {
            /* a fixed region too small for the split may still hold the unsplit partial rows (same
             * bits: the K blocks are summed in the same order either way) */
            if (need > sc->ws_floats && kz > 1 && (size_t)M * nout <= sc->ws_floats) kz = 1;
            if ((size_t)kz * M * nout > sc->ws_floats) return -2;
            a->ws = sc->ws;
        } else {
            a->ws = gpu_scratch_ws(g, need);
            if (!a->ws && kz > 1) { /* a capture that cannot grow the scratch: unsplit, same bits */
                kz = 1;
                a->ws = gpu_scratch_ws(g, (size_t)M * nout);
            }
            if (!a->ws) return bad(g, "gemm: residual-update scratch unavailable (size it before capture)");
        }
        pend->parts = a->ws;
        pend->nparts = kz;
        pend->alpha = a->alpha;
    }
    const uint32_t tm = (M + cfg[pick_i].bm - 1) / cfg[pick_i].bm;
    a->splits = kz;
    /* at most 8 row tiles per group: an XCD's 64 resident workgroups then cover about 8 row tiles x 8
     * column tiles, whose A panels stay in its L2 while the weight columns stream past (at 3584
     * rows: L2 fetch -18% on FF up, -12% on QKV against 14-row groups; 2-4% faster) */
    a->group_m = tm <= 8 ? tm : 8;
    const uint32_t total = tiles * kz, per = (total + 7) / 8;
    char name[40];
    snprintf(name, sizeof name, "%s%s", resid ? cfg[pick_i].acc_name : glu ? cfg[pick_i].glu_name : cfg[pick_i].name, sfx);
    return gpu_launch(g, name, a, sizeof *a, 8 * per, 1, 1, 256, 1, 1);
}

static int launch_mx(gpu_t *g, NkGemmArgs *a, uint32_t M, uint32_t nout, uint32_t K, int glu, int resid) {
    nk_resid_t pend = { 0 };
    const int rc = launch_mx_s(g, a, M, nout, K, glu, resid, NULL, &pend);
    if (rc || !resid) return rc;
    return nk_resid_fold(g, a->C, a->ldc, M, nout, &pend);
}

int nk_resid_fold(gpu_t *g, float *C, uint32_t ldc, uint32_t M, uint32_t N, const nk_resid_t *pend) {
    if (!M || !pend || !pend->nparts) return 0;
    if (N % 4 || ldc % 4 || (uintptr_t)C % 16) return bad(g, "resid_fold: N, ldc multiples of 4, C 16-byte aligned");
    NkFoldArgs f = { C, pend->parts, M, N, ldc, pend->nparts, pend->alpha, 0 };
    return gpu_launch(g, "resid_fold", &f, sizeof f, (uint32_t)(((uint64_t)M * (N / 4) + 255) / 256), 1, 1, 256, 1, 1);
}

/* The many-row GEMM with split-row operands (the batched encoder's activations between kernels):
 * exactly one of A (f32 rows of lda floats) and A2 (split rows, lda bf16 elements, K hi then K lo)
 * and one of C (f32, += when accumulating, row map crow) and C2 (split rows of the nout outputs,
 * ldc bf16 elements; no accumulate, no row map, no GLU).  With pend set, a residual update
 * (accumulate, no bias, no activation, no row map) leaves C untouched and returns the update in
 * *pend for the next LayerNorm (nk_layernorm2_split) or nk_resid_fold to apply; otherwise C is
 * updated by the call. */
static int gemm_split_core(gpu_t *g, const float *A, const uint16_t *A2, uint32_t lda, const uint16_t *W, uint32_t ldw,
                           const float *bias, float *C, uint16_t *C2, uint32_t ldc, const int *crow, uint32_t M,
                           uint32_t N, uint32_t K, int act, int accumulate, float alpha, const mx_scratch_t *sc,
                           nk_resid_t *pend) {
    if (pend) memset(pend, 0, sizeof *pend);
    if (!M) return 0;
    const int glu = act == NK_ACT_GLU;
    const uint32_t nout = glu ? N / 2 : N;
    if (!N || !K || (glu && (N & 1)) || K % 32 || (A2 && K % NK_MX_KS_SPLIT) || !A == !A2 || !C == !C2)
        return bad(g, "gemm_split: one A form, one C form, K % 32 == 0 (K % 64 == 0 with split-row A)");
    if (!aligned16(W) || ldw % 8 || K > ldw) return bad(g, "gemm_split: W 16-byte aligned, ldw % 8 == 0, K <= ldw");
    if (A ? (!aligned16(A) || lda % 4 || K > lda) : (!aligned16(A2) || lda % 8 || 2 * K > lda))
        return bad(g, "gemm_split: A 16-byte aligned rows of at least K values (split: 2K, lda % 8 == 0)");
    if (C2 && (glu || accumulate || crow || ldc < 2 * nout || ldc % 4 || (uintptr_t)C2 % 8))
        return bad(g, "gemm_split: split outputs take no GLU, accumulate or row map; ldc >= 2 nout");
    if (C && ldc < nout) return bad(g, "gemm_split: ldc < output width");
    const int resid = accumulate && !bias && act == NK_ACT_NONE && !crow && nout % 4 == 0;
    if (pend && !resid) return bad(g, "gemm_split: a deferred update needs accumulate, no bias, activation or row map");
    NkGemmArgs a;
    memset(&a, 0, sizeof a);
    a.A = A; a.A2 = A2; a.W = W; a.bias = bias; a.C = C; a.C2 = C2; a.crow = crow;
    a.M = M; a.N = N; a.K = K; a.lda = lda; a.ldw = ldw; a.ldc = ldc;
    a.act = (uint32_t)act; a.accumulate = (uint32_t)(accumulate != 0); a.alpha = alpha; a.splits = 1;
    gpu_next_bytes(g, 2.0 * N * K + 4.0 * M * K + 4.0 * M * nout * (accumulate ? 2 : 1) + (bias ? 4.0 * N : 0.0));
    gpu_next_flops(g, 2.0 * M * N * K);
    nk_resid_t local;
    const int rc = launch_mx_s(g, &a, M, nout, K, glu, resid, sc, pend ? pend : &local);
    if (rc == -2) return bad(g, "gemm_split: the K split of this shape needs more than the fixed scratch holds");
    if (rc == 1) return bad(g, "gemm_split: no tile divides the output columns");
    if (rc || !resid || pend) return rc;
    return nk_resid_fold(g, C, ldc, M, nout, &local);
}

int nk_gemm_split(gpu_t *g, const float *A, const uint16_t *A2, uint32_t lda, const uint16_t *W, uint32_t ldw,
                  const float *bias, float *C, uint16_t *C2, uint32_t ldc, const int *crow, uint32_t M, uint32_t N,
                  uint32_t K, int act, int accumulate, float alpha) {
    return gemm_split_core(g, A, A2, lda, W, ldw, bias, C, C2, ldc, crow, M, N, K, act, accumulate, alpha, NULL, NULL);
}

int nk_gemm_resid(gpu_t *g, const float *A, const uint16_t *A2, uint32_t lda, const uint16_t *W, uint32_t ldw, float *C,
                  uint32_t ldc, uint32_t M, uint32_t N, uint32_t K, float alpha, nk_resid_t *pend) {
    return gemm_split_core(g, A, A2, lda, W, ldw, NULL, C, NULL, ldc, NULL, M, N, K, NK_ACT_NONE, 1, alpha, NULL, pend);
}

/* nk_gemm_split on a fixed scratch region the caller provides (the allocation-free entry point,
 * noalloc.hip): a residual update whose partial rows need more than the region holds is refused
 * before anything is launched. */
int nk_gemm_split_scratch(gpu_t *g, const float *A, const uint16_t *A2, uint32_t lda, const uint16_t *W, uint32_t ldw,
                          const float *bias, float *C, uint16_t *C2, uint32_t ldc, const int *crow, uint32_t M,
                          uint32_t N, uint32_t K, int act, int accumulate, float alpha, float *ws, size_t ws_floats) {
    const mx_scratch_t sc = { ws, ws_floats };
    return gemm_split_core(g, A, A2, lda, W, ldw, bias, C, C2, ldc, crow, M, N, K, act, accumulate, alpha, &sc, NULL);
}

int nk_gemm_argmax(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                   unsigned long long *keys, uint32_t keys_ld, uint32_t M, uint32_t N, uint32_t K, uint32_t V) {
    return nk_gemm_argmax_rows(g, A, lda, W, ldw, bias, keys, keys_ld, M, N, K, V, NULL, 0);
}

int nk_gemm_argmax_rows(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                        unsigned long long *keys, uint32_t keys_ld, uint32_t M, uint32_t N, uint32_t K, uint32_t V,
                        const int *mrows, uint32_t mrows_mul) {
    if (!M) return 0;
    if (N % 64 || K % 32 || V > N || keys_ld < 2 * (N / 64) || !aligned16(A) || !aligned16(W) || lda % 4 || ldw % 8)
        return bad(g, "gemm_argmax: N % 64 == 0, K % 32 == 0, V <= N, keys_ld >= N/32, aligned operands");
    NkGemmArgs a;
    memset(&a, 0, sizeof a);
    a.A = A; a.W = W; a.bias = bias; a.M = M; a.N = N; a.K = K; a.lda = lda; a.ldw = ldw; a.ldc = N;
    a.alpha = 1.0f; a.splits = 1; a.keys = keys; a.keys_ld = keys_ld; a.keys_n = V;
    a.mrows = mrows; a.mrows_mul = mrows_mul;
    const uint32_t tm = (M + 63) / 64, tiles = tm * (N / 64), per = (tiles + 7) / 8;
    a.group_m = tm <= 8 ? tm : 8;
    gpu_next_flops(g, 2.0 * M * N * K);
    return gpu_launch(g, "gemm_mx64x64_argmax", &a, sizeof a, 8 * per, 1, 1, 256, 1, 1);
}

/* The GEMM with an optional LayerNorm prologue on A.  The weight-streaming GEMV (K <= 1024) and the
 * few-row MFMA kernel (K == 1024) apply it in their prologue; other kernels get it from separate
 * LayerNorm launches into ln.tmp.  With pend_out set, a residual update whose kernel splits K
 * (the few-row kernel) is left pending: its partial rows are returned in *pend_out and C is not
 * touched; otherwise *pend_out is emptied and C updated. */
#define FR_FOLD_PARTS 4 /* partial rows the few-row kernel's fold prologue takes */
static int gemm_core_p(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                       float *C, uint32_t ldc, const int *crow, uint32_t M, uint32_t N, uint32_t K, int act,
                       int accumulate, float alpha, const ln_pro_t *ln, nk_resid_t *pend_out);
static int gemm_core(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                     float *C, uint32_t ldc, const int *crow, uint32_t M, uint32_t N, uint32_t K, int act,
                     int accumulate, float alpha, const ln_pro_t *ln) {
    return gemm_core_p(g, A, lda, W, ldw, bias, C, ldc, crow, M, N, K, act, accumulate, alpha, ln, NULL);
}
static int gemm_core_p(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                       float *C, uint32_t ldc, const int *crow, uint32_t M, uint32_t N, uint32_t K, int act,
                       int accumulate, float alpha, const ln_pro_t *ln, nk_resid_t *pend_out) {
    if (pend_out) memset(pend_out, 0, sizeof *pend_out);
    if (!M) return 0;
    if (!N || !K || (act == NK_ACT_GLU && (N & 1))) return bad(g, "gemm: bad shape");
    if (!aligned16(A) || !aligned16(W) || lda % 4 || ldw % 8 || K % 8 || K > lda || K > ldw)
        return bad(g, "gemm: A/W must be 16-byte aligned with lda % 4 == 0, ldw % 8 == 0, K % 8 == 0");
    const uint32_t nout = act == NK_ACT_GLU ? N / 2 : N;
    if (ldc < nout) return bad(g, "gemm: ldc < output width");
    /* batched streams: always the many-row kernels (a row's result then does not depend on how many
     * other rows share the launch) */
    const int kind = gpu_many_rows(g) && !g_force && K % 32 == 0 ? K_MR : pick(M, N, K, act);
    const int ln_fused = ln && ln->mode && K == lda &&
                         ((kind == K_GEMV && K <= 1024) || (kind == K_FR && K == 1024 && M <= 16));
    const int fold = ln && ln->mode && ln->pend && ln->pend->nparts;
    if (ln && ln->mode && ln->fold_out && !fold) {
        /* nothing pending: the output rows are A itself */
        if (ln->fold_out == A || lda % 4) return bad(g, "gemm: a pending update needs its own output rows");
        if (nk_copy2d(g, A, lda, ln->fold_out, lda, M, K)) return -1;
        ln_pro_t plain = *ln;
        plain.fold_out = NULL;
        return gemm_core(g, ln->fold_out, lda, W, ldw, bias, C, ldc, crow, M, N, K, act, accumulate, alpha, &plain);
    }
    const int fold_fused = fold && ln_fused &&
                           ((kind == K_GEMV && K % 4 == 0 && M <= 4) || (kind == K_FR && ln->pend->nparts <= FR_FOLD_PARTS));
    if (fold) {
        if (ln->fold_out && (ln->fold_out == A || lda % 4)) return bad(g, "gemm: a pending update needs its own output rows");
        if (!fold_fused) {
            /* kernels without the fold prologue: apply the update to a copy of A, then as usual */
            if (!ln->fold_out) return bad(g, "gemm: this kernel applies a pending update only through output rows (Xf)");
            if (nk_copy2d(g, A, lda, ln->fold_out, lda, M, K)) return -1;
            if (nk_resid_fold(g, ln->fold_out, lda, M, K, ln->pend)) return -1;
            ln_pro_t plain = *ln;
            plain.pend = NULL;
            plain.fold_out = NULL;
            return gemm_core(g, ln->fold_out, lda, W, ldw, bias, C, ldc, crow, M, N, K, act, accumulate, alpha, &plain);
        }
    }
    if (ln && ln->mode && !ln_fused) {
        /* unfused LayerNorm: out = LN1(A) (if requested), tmp = LN(...) feeds the GEMM */
        if (!ln->tmp || K != lda) return bad(g, "gemm: LayerNorm prologue needs a scratch buffer");
        if (ln->mode == 2) {
            float *y1 = ln->out ? ln->out : ln->tmp;
            if (nk_layernorm2(g, A, ln->g1, ln->b1, ln->g2, ln->b2, y1, ln->tmp, M, K, ln->eps)) return -1;
        } else {
            if (nk_layernorm(g, A, ln->g1, ln->b1, ln->tmp, M, K, ln->eps)) return -1;
            if (ln->out && nk_copy(g, ln->tmp, ln->out, M * K)) return -1;
        }
        return gemm_core(g, ln->tmp, lda, W, ldw, bias, C, ldc, crow, M, N, K, act, accumulate, alpha, NULL);
    }
    NkGemmArgs a;
    memset(&a, 0, sizeof a);
    a.A = A; a.W = W; a.bias = bias; a.C = C; a.crow = crow;
    a.M = M; a.N = N; a.K = K; a.lda = lda; a.ldw = ldw; a.ldc = ldc;
    a.act = (uint32_t)act; a.accumulate = (uint32_t)(accumulate != 0); a.alpha = alpha; a.splits = 1;
    if (ln && ln->mode) {
        if (K != lda) return bad(g, "gemm: LayerNorm prologue needs K == lda");
        a.ln_mode = (uint32_t)ln->mode; a.ln_g1 = ln->g1; a.ln_b1 = ln->b1; a.ln_g2 = ln->g2; a.ln_b2 = ln->b2;
        a.ln_out = ln->out; a.ln_eps = ln->eps;
    }
    /* algorithmic HBM bytes: every weight once, A once, C written (and read when accumulating) */
    gpu_next_bytes(g, 2.0 * N * K + 4.0 * M * K + 4.0 * M * nout * (accumulate ? 2 : 1) + (bias ? 4.0 * N : 0.0));
    gpu_next_flops(g, 2.0 * M * N * K);
    char name[32];
    if (kind == K_GEMV) {
        /* the GEMV reads bias and the row map unconditionally */
        if (N > GPU_ZEROS_N) return bad(g, "gemm: N too large for the GEMV");
        if (!a.bias) a.bias = gpu_zeros(g);
        if (!a.crow) a.crow = gpu_iota(g);
        uint32_t kch, nc;
        gemv_shape(N, K, act, &kch, &nc);
        const uint32_t per_wave = act == NK_ACT_GLU ? nc / 2 : nc;
        const uint32_t waves = (nout + per_wave - 1) / per_wave;
        if (fold) {
            /* the workgroups apply the pending update to A in their prologue (gemv_*_f) */
            a.fold = ln->pend->parts;
            a.fold_n = ln->pend->nparts;
            a.fold_alpha = ln->pend->alpha;
            a.fold_out = ln->fold_out;
        }
        snprintf(name, sizeof name, "gemv_r%u_n%u_k%u%s", M, nc, kch, fold ? "_f" : "");
        return gpu_launch(g, name, &a, sizeof a, (waves + 3) / 4, 1, 1, 256, 1, 1);
    }
    if (K % 32) return bad(g, "gemm: K % 32 != 0 for the MFMA kernels");
    if (kind == K_FR) {
        /* the few-row kernel reads bias and the row map unconditionally */
        if (N > GPU_ZEROS_N) return bad(g, "gemm: N too large for the few-row kernel");
        const fr_plan_t p = fr_plan(nout, K, act, accumulate && !crow && nout % 4 == 0 && ldc % 4 == 0 &&
                                    ((uintptr_t)C & 15) == 0, bias != NULL, ln_fused);
        if (!a.bias) a.bias = gpu_zeros(g);
        if (!a.crow) a.crow = gpu_iota(g);
        const uint32_t tc = ln_fused && act == NK_ACT_GLU ? 8 : 16; /* output columns per workgroup */
        const uint32_t tiles = (nout + tc - 1) / tc;
        if (fold) {
            /* the LayerNorm prologue adds the pending update to A first (gemm_fr_ln*_f) */
            a.fold = ln->pend->parts;
            a.fold_n = ln->pend->nparts;
            a.fold_alpha = ln->pend->alpha;
            a.fold_out = ln->fold_out;
        }
        if (p.KS > 1) {
            /* the K shares' partial rows: left pending for the caller, or folded into C in share
             * order by a second launch */
            a.ws = gpu_scratch_ws(g, (size_t)p.KS * M * nout);
            if (!a.ws) return bad(g, "gemm: split-K scratch unavailable (size it before capture)");
            if (gpu_launch(g, fr_name(p, act, ln_fused, 0), &a, sizeof a, tiles, p.KS, 1, 64 * p.W, 1, 1)) return -1;
            const nk_resid_t pend = { a.ws, p.KS, alpha };
            if (pend_out) {
                *pend_out = pend;
                return 0;
            }
            return nk_resid_fold(g, C, ldc, M, nout, &pend);
        }
        return gpu_launch(g, fr_name(p, act, ln_fused, fold), &a, sizeof a, tiles, p.KS, 1, 64 * p.W, 1, 1);
    }
    const int glu = act == NK_ACT_GLU;
    if (g_force != K_MM_OLD) {
        /* the deferred (partial-row) residual update writes rows 0..M-1 of C through resid_fold: only
         * without a row map and on the layout the fold takes; otherwise the plain add-into-C epilogue */
        const int resid = accumulate && !bias && act == NK_ACT_NONE && !crow && nout % 4 == 0 && ldc % 4 == 0 &&
                          ((uintptr_t)C & 15) == 0;
        const int rc = launch_mx(g, &a, M, nout, K, glu, resid);
        if (rc <= 0) return rc;
    }
    /* many rows, first-generation kernels: 128 x 128 tiles when they fill the GPU, else 64 x 64 */
    if (nout % (glu ? 64 : 128) == 0) {
        const uint32_t t128 = ((M + 127) / 128) * (nout / (glu ? 64 : 128));
        if (t128 >= 240)
            return gpu_launch(g, glu ? "gemm_mm128_glu" : "gemm_mm128", &a, sizeof a, nout / (glu ? 64 : 128),
                              (M + 127) / 128, 1, 256, 1, 1);
    }
    if (nout % (glu ? 32 : 64) == 0)
        return gpu_launch(g, glu ? "gemm_mm64_glu" : "gemm_mm64", &a, sizeof a, nout / (glu ? 32 : 64), (M + 63) / 64,
                          1, 256, 1, 1);
    if (glu) return bad(g, "gemm: GLU needs N/2 to be a multiple of 32");
    return gpu_launch(g, "gemm_mr", &a, sizeof a, (N + 63) / 64, (M + 63) / 64, 1, 256, 1, 1);
}

int nk_gemm_rows(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                 float *C, uint32_t ldc, const int *crow, uint32_t M, uint32_t N, uint32_t K, int act, int accumulate,
                 float alpha) {
    return gemm_core(g, A, lda, W, ldw, bias, C, ldc, crow, M, N, K, act, accumulate, alpha, NULL);
}

int nk_gemm(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias, float *C,
            uint32_t ldc, uint32_t M, uint32_t N, uint32_t K, int act, int accumulate, float alpha) {
    return gemm_core(g, A, lda, W, ldw, bias, C, ldc, NULL, M, N, K, act, accumulate, alpha, NULL);
}

int nk_gemm_ln(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias, float *C,
               uint32_t ldc, const int *crow, uint32_t M, uint32_t N, uint32_t K, int act, int accumulate, float alpha,
               int ln_mode, const float *g1, const float *b1, const float *g2, const float *b2, float *ln_out,
               float *tmp, float eps) {
    const ln_pro_t ln = { ln_mode, g1, b1, g2, b2, ln_out, tmp, eps, NULL, NULL };
    if (ln_mode < 0 || ln_mode > 2) return bad(g, "gemm: ln_mode must be 0, 1 or 2");
    return gemm_core(g, A, lda, W, ldw, bias, C, ldc, crow, M, N, K, act, accumulate, alpha, &ln);
}

int nk_gemm_pend(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, float *C, uint32_t ldc,
                 uint32_t M, uint32_t N, uint32_t K, float alpha, nk_resid_t *pend) {
    if (!pend) return bad(g, "gemm_pend: pend is required");
    return gemm_core_p(g, A, lda, W, ldw, NULL, C, ldc, NULL, M, N, K, NK_ACT_NONE, 1, alpha, NULL, pend);
}

int nk_gemm_ln_pend(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                    float *C, uint32_t ldc, const int *crow, uint32_t M, uint32_t N, uint32_t K, int act, int accumulate,
                    float alpha, int ln_mode, const float *g1, const float *b1, const float *g2, const float *b2,
                    float *ln_out, float *tmp, float eps, const nk_resid_t *pend, float *Xf) {
    const ln_pro_t ln = { ln_mode, g1, b1, g2, b2, ln_out, tmp, eps, pend, Xf };
    if (ln_mode < 1 || ln_mode > 2) return bad(g, "gemm: a pending update needs a LayerNorm prologue (ln_mode 1 or 2)");
    return gemm_core(g, A, lda, W, ldw, bias, C, ldc, crow, M, N, K, act, accumulate, alpha, &ln);
}

/* The many-row LayerNorm: one wavefront per row and per workgroup, so the rows spread over every
 * CU. */
static int launch_ln_rows(gpu_t *g, const NkLnArgs *a, uint32_t M) {
    return gpu_launch(g, "layernorm_rows", a, sizeof *a, M, 1, 1, 64, 1, 1);
}

int nk_layernorm2(gpu_t *g, const float *X, const float *g1, const float *b1, const float *g2, const float *b2,
                  float *Y1, float *Y2, uint32_t M, uint32_t D, float eps) {
    if (!M) return 0;
    if (!D || D > NK_ROW_MAX || D % 4) return bad(g, "layernorm: D must be a positive multiple of 4, at most 4096");
    NkLnArgs a = { X, g1, b1, g2, b2, Y1, Y2, M, D, eps, 0, NULL, NULL, 0, 0.0f };
    /* many rows: a wavefront per row (D <= 1024), no barriers */
    if ((M > 16 || gpu_many_rows(g)) && D <= 1024) {
        return launch_ln_rows(g, &a, M);
    }
    return gpu_launch(g, "layernorm", &a, sizeof a, M, 1, 1, NK_LN_THREADS, 1, 1);
}

int nk_layernorm2_split(gpu_t *g, float *X, const nk_resid_t *pend, const float *g1, const float *b1, const float *g2,
                        const float *b2, float *Y1, uint16_t *Ys, uint32_t M, uint32_t D, float eps) {
    if (!M) return 0;
    if (!D || D > 1024 || D % 4 || !Ys || (uintptr_t)Ys % 8 || (g2 && !Y1))
        return bad(g, "layernorm_split: D a positive multiple of 4, at most 1024, a split output (and Y1 when paired)");
    NkLnArgs a = { X, g1, b1, g2, b2, g2 ? Y1 : NULL, NULL, M, D, eps, 0, Ys, NULL, 0, 0.0f };
    if (g2) a.Y2 = Y1; /* any non-NULL Y2 selects the pair; its rows go to Ys */
    if (pend && pend->nparts) {
        a.P = pend->parts;
        a.nparts = pend->nparts;
        a.palpha = pend->alpha;
    }
    return launch_ln_rows(g, &a, M);
}

int nk_layernorm(gpu_t *g, const float *X, const float *gamma, const float *beta, float *Y, uint32_t M, uint32_t D,
                 float eps) {
    return nk_layernorm2(g, X, gamma, beta, NULL, NULL, Y, NULL, M, D, eps);
}

int nk_attention_rel(gpu_t *g, const float *Q, uint32_t ldq, const float *K, const float *V, uint32_t ldk,
                     const float *P, const float *bias_u, const float *bias_v, float *O, uint32_t c, uint32_t L,
                     uint32_t Lmax, uint32_t H, uint32_t dh, uint32_t D, float scale) {
    if (!c) return 0;
    if (dh != 128 || H * dh != D) return bad(g, "attention: head_dim must be 128");
    if (L > NK_ATT_MAX_L || L > Lmax || c > L || c > Lmax) return bad(g, "attention: window exceeds the table");
    if ((uintptr_t)K % 8 || (uintptr_t)P % 8 || ldk % 2) return bad(g, "attention: K/P must be 8-byte aligned");
    if ((uintptr_t)Q % 16 || (uintptr_t)K % 16 || (uintptr_t)V % 16 || ldq % 4 || ldk % 4)
        return bad(g, "attention: Q/K/V must be 16-byte aligned");
    NkAttnArgs a = { Q, K, V, P, bias_u, bias_v, O, NULL, NULL, c, L, Lmax, H, dh, D, ldq, ldk, scale, 0 };
    return gpu_launch(g, "attention_rel", &a, sizeof a, H, c, 1, 512, 1, 1);
}

int nk_attention_rel_desc(gpu_t *g, const float *kv, uint32_t ld, const int *desc, const float *P, const float *bias_u,
                          const float *bias_v, float *O, uint32_t c, uint32_t Lmax, uint32_t H, uint32_t dh, uint32_t D,
                          float scale) {
    if (!c) return 0;
    if (dh != 128 || H * dh != D || c > Lmax || Lmax > NK_ATT_MAX_L) return bad(g, "attention: head_dim must be 128");
    if ((uintptr_t)kv % 16 || ld % 4) return bad(g, "attention: cache must be 16-byte aligned");
    NkAttnArgs a = { kv, kv + D, kv + 2 * D, P, bias_u, bias_v, O, desc, NULL, c, 0, Lmax, H, dh, D, ld, ld, scale, 0 };
    return gpu_launch(g, "attention_rel", &a, sizeof a, H, c, 1, 512, 1, 1);
}

int nk_dwconv_ln_silu(gpu_t *g, const float *din, const float *W, const float *gamma, const float *beta, float *Y,
                      uint32_t c, uint32_t D, uint32_t taps, float eps) {
    if (!c) return 0;
    if (D > NK_ROW_MAX || D % 4 || taps != NK_CONV_TAPS) return bad(g, "dwconv: 9 taps, D a multiple of 4, at most 4096");
    NkDwArgs a = { din, W, gamma, beta, Y, NULL, NULL, c, D, taps, eps };
    return gpu_launch(g, "dwconv_ln_silu", &a, sizeof a, c, 1, 1, NK_LN_THREADS, 1, 1);
}

int nk_dwconv_ln_silu_desc(gpu_t *g, const float *din_base, const int *desc, const float *W, const float *gamma,
                           const float *beta, float *Y, uint32_t c, uint32_t D, uint32_t taps, float eps) {
    if (!c) return 0;
    if (D > NK_ROW_MAX || D % 4 || taps != NK_CONV_TAPS) return bad(g, "dwconv: 9 taps, D a multiple of 4, at most 4096");
    NkDwArgs a = { din_base, W, gamma, beta, Y, desc, NULL, c, D, taps, eps };
    return gpu_launch(g, "dwconv_ln_silu", &a, sizeof a, c, 1, 1, NK_LN_THREADS, 1, 1);
}

/* measured at one row (80 ms chunks): 8 columns per wavefront (128 workgroups) and one weight row
 * per wavefront were the fastest of {4, 8, 16} x {1, 2, 4} */
static int g_attn_cpw = 8, g_dw_nc = 1;

int nk_fuse_shape(int attn_cpw, int dw_nc) {
    const int prev = g_attn_cpw * 16 + g_dw_nc;
    if (attn_cpw == 4 || attn_cpw == 8 || attn_cpw == 16) g_attn_cpw = attn_cpw;
    if (dw_nc == 1 || dw_nc == 2 || dw_nc == 4) g_dw_nc = dw_nc;
    return prev;
}

int nk_attention_out_desc(gpu_t *g, const float *kv, uint32_t ld, const int *desc, const float *P, const float *bias_u,
                          const float *bias_v, uint32_t c, uint32_t Lmax, uint32_t H, uint32_t dh, uint32_t D,
                          float scale, const uint16_t *Wo, uint32_t ldw, float *C, uint32_t ldc, float alpha) {
    if (!c) return 0;
    if (ldc % 4 || (uintptr_t)C % 16) return bad(g, "attention_out: C 16-byte aligned, ldc % 4 == 0");
    nk_resid_t pend;
    if (nk_attention_out_desc_pend(g, kv, ld, desc, P, bias_u, bias_v, c, Lmax, H, dh, D, scale, Wo, ldw, alpha, &pend))
        return -1;
    return nk_resid_fold(g, C, ldc, c, D, &pend);
}

int nk_attention_out_desc_pend(gpu_t *g, const float *kv, uint32_t ld, const int *desc, const float *P,
                               const float *bias_u, const float *bias_v, uint32_t c, uint32_t Lmax, uint32_t H,
                               uint32_t dh, uint32_t D, float scale, const uint16_t *Wo, uint32_t ldw, float alpha,
                               nk_resid_t *pend) {
    memset(pend, 0, sizeof *pend);
    if (!c) return 0;
    if (dh != 128 || H * dh != D || c > 4 || c > Lmax || Lmax > NK_ATT_MAX_L || D % (8u * (uint32_t)g_attn_cpw))
        return bad(g, "attention_out: head_dim 128, c <= 4, D a multiple of the column tile");
    if ((uintptr_t)kv % 16 || ld % 4 || !aligned16(Wo) || ldw % 8 || ldw < D)
        return bad(g, "attention_out: aligned cache and weights, ldw >= D");
    NkAttnOutArgs p;
    memset(&p, 0, sizeof p);
    p.at = (NkAttnArgs){ kv, kv + D, kv + 2 * D, P, bias_u, bias_v, NULL, desc, NULL, c, 0, Lmax, H, dh, D, ld, ld, scale, 0 };
    p.Wo = Wo;
    /* per-head partial rows [H][c][D]: the update C + alpha * (((0 + h0) + h1) + ...) is left pending */
    p.ws = gpu_scratch_ws(g, (size_t)c * D * H);
    if (!p.ws) return bad(g, "attention_out: scratch unavailable (size it before capture)");
    p.ldw = ldw;
    p.ldc = D;
    p.alpha = alpha;
    gpu_next_bytes(g, 2.0 * D * D + 4.0 * 2 * c * D);
    gpu_next_flops(g, 2.0 * c * D * D);
    const uint32_t cols = 8u * (uint32_t)g_attn_cpw;
    char name[32];
    snprintf(name, sizeof name, "attention_rel_out_c%d", g_attn_cpw);
    if (gpu_launch(g, name, &p, sizeof p, H, D / cols, c, 512, 1, 1)) return -1;
    pend->parts = p.ws;
    pend->nparts = H;
    pend->alpha = alpha;
    return 0;
}

int nk_dwconv_pw_desc(gpu_t *g, const float *din_base, const int *desc, const float *dw_w, const float *gamma,
                      const float *beta, float eps, const uint16_t *W, uint32_t ldw, float *C, uint32_t ldc, uint32_t c,
                      uint32_t D, uint32_t N, int accumulate, float alpha) {
    if (!c) return 0;
    if (c > 2 || D > 1024 || D % 8 || !N || N > GPU_ZEROS_N)
        return bad(g, "dwconv_pw: c <= 2, D <= 1024 and a multiple of 8, N <= the zero-bias length");
    if (!aligned16(W) || ldw % 8 || ldw < D || ldc < N || (uintptr_t)din_base % 16)
        return bad(g, "dwconv_pw: aligned operands, ldw >= D, ldc >= N");
    NkGemvDwArgs p;
    memset(&p, 0, sizeof p);
    p.g.W = W; p.g.bias = gpu_zeros(g); p.g.C = C; p.g.crow = gpu_iota(g);
    p.g.M = c; p.g.N = N; p.g.K = D; p.g.lda = D; p.g.ldw = ldw; p.g.ldc = ldc;
    p.g.act = NK_ACT_NONE; p.g.accumulate = (uint32_t)(accumulate != 0); p.g.alpha = alpha; p.g.splits = 1;
    p.d = (NkDwArgs){ din_base, dw_w, gamma, beta, NULL, desc, NULL, c, D, NK_CONV_TAPS, eps };
    gpu_next_bytes(g, 2.0 * N * D + 4.0 * c * N * (accumulate ? 2 : 1));
    gpu_next_flops(g, 2.0 * c * N * D);
    const uint32_t kch = D / 8 <= 64 ? 1 : 2, nc = (uint32_t)g_dw_nc, waves = (N + nc - 1) / nc;
    char name[32];
    snprintf(name, sizeof name, "gemv_dw_r%u_n%u_k%u", c, nc, kch);
    return gpu_launch(g, name, &p, sizeof p, (waves + 3) / 4, 1, 1, 256, 1, 1);
}

int nk_attention_rel_rows(gpu_t *g, const float *kv, uint32_t ld, const int *rows, uint32_t M, const float *P,
                          const float *bias_u, const float *bias_v, float *O, uint32_t Lmax, uint32_t H, uint32_t dh,
                          uint32_t D, float scale) {
    if (!M) return 0;
    if (dh != 128 || H * dh != D || Lmax > NK_ATT_MAX_L) return bad(g, "attention: head_dim must be 128");
    if ((uintptr_t)kv % 16 || ld % 4) return bad(g, "attention: cache must be 16-byte aligned");
    NkAttnArgs a = { kv, kv + D, kv + 2 * D, P, bias_u, bias_v, O, NULL, rows, 0, 0, Lmax, H, dh, D, ld, ld, scale, 0 };
    return gpu_launch(g, "attention_rel", &a, sizeof a, H, M, 1, 512, 1, 1);
}

int nk_attention_rel_chunks(gpu_t *g, const float *kv, uint32_t ld, const int *chunks, uint32_t nchunks, const float *P,
                            const float *bias_u, const float *bias_v, float *O, uint32_t Lmax, uint32_t H, uint32_t dh,
                            uint32_t D, float scale) {
    if (!nchunks) return 0;
    if (dh != 128 || H * dh != D) return bad(g, "attention: head_dim must be 128");
    if ((uintptr_t)kv % 16 || ld % 4 || (uintptr_t)P % 16 || D % 4) return bad(g, "attention: cache must be 16-byte aligned");
    NkAttnChunkArgs a = { kv, P, bias_u, bias_v, O, chunks, H, dh, D, ld, Lmax, scale, NULL };
    return gpu_launch(g, "attention_rel_chunks", &a, sizeof a, H, nchunks, 1, 256, 1, 1);
}

int nk_attention_rel_chunks_split(gpu_t *g, const float *kv, uint32_t ld, const int *chunks, uint32_t nchunks,
                                  const float *P, const float *bias_u, const float *bias_v, uint16_t *Os, uint32_t Lmax,
                                  uint32_t H, uint32_t dh, uint32_t D, float scale) {
    if (!nchunks) return 0;
    if (dh != 128 || H * dh != D) return bad(g, "attention: head_dim must be 128");
    if ((uintptr_t)kv % 16 || ld % 4 || (uintptr_t)P % 16 || D % 4 || !Os) return bad(g, "attention: cache must be 16-byte aligned");
    NkAttnChunkArgs a = { kv, P, bias_u, bias_v, NULL, chunks, H, dh, D, ld, Lmax, scale, Os };
    return gpu_launch(g, "attention_rel_chunks", &a, sizeof a, H, nchunks, 1, 256, 1, 1);
}

int nk_dwconv_ln_silu_rows(gpu_t *g, const float *din_base, const int *rows, uint32_t M, const float *W,
                           const float *gamma, const float *beta, float *Y, uint32_t D, uint32_t taps, float eps) {
    return nk_dwconv_ln_silu_rows_split(g, din_base, rows, M, W, gamma, beta, Y, NULL, D, taps, eps);
}

int nk_dwconv_ln_silu_rows_split(gpu_t *g, const float *din_base, const int *rows, uint32_t M, const float *W,
                                 const float *gamma, const float *beta, float *Y, uint16_t *Ys, uint32_t D, uint32_t taps,
                                 float eps) {
    if (!M) return 0;
    if (D > NK_ROW_MAX || D % 4 || taps != NK_CONV_TAPS) return bad(g, "dwconv: 9 taps, D a multiple of 4, at most 4096");
    if (!Y == !Ys || (uintptr_t)Ys % 8) return bad(g, "dwconv: one output form");
    NkDwArgs a = { din_base, W, gamma, beta, Y, NULL, rows, M, D, taps, eps, Ys };
    return gpu_launch(g, "dwconv_ln_silu", &a, sizeof a, M, 1, 1, NK_LN_THREADS, 1, 1);
}

static uint32_t blocks_for(uint64_t n) { return (uint32_t)((n + 255) / 256); }

/* output columns per workgroup of the subsampling convs: one (every output its own workgroup, one
 * memory round trip) unless the batch has thousands of output positions, then eight (fewer
 * workgroups, the filter taps loaded once for eight columns) */
static uint32_t conv_fb(uint32_t T1, uint32_t F1, uint32_t batch) { return (uint64_t)T1 * F1 * batch >= 4096 ? 8 : 1; }

int nk_conv2d_c1_s2_relu_b(gpu_t *g, const float *X, const float *W, const float *bias, float *Y, uint32_t T,
                           uint32_t F, uint32_t T1, uint32_t F1, uint32_t C, uint32_t batch) {
    const uint32_t fb = conv_fb(T1, F1, batch);
    NkConvArgs a = { X, W, bias, Y, T, F, T1, F1, C, fb, T * F, T1 * F1 * C };
    return gpu_launch(g, "conv2d_c1_s2_relu", &a, sizeof a, T1 * ((F1 + fb - 1) / fb), batch, 1, 256, 1, 1);
}

int nk_dwconv2d_s2_b(gpu_t *g, const float *X, const float *W, const float *bias, float *Y, uint32_t T, uint32_t F,
                     uint32_t T1, uint32_t F1, uint32_t C, uint32_t batch) {
    const uint32_t fb = conv_fb(T1, F1, batch);
    NkConvArgs a = { X, W, bias, Y, T, F, T1, F1, C, fb, T * F * C, T1 * F1 * C };
    return gpu_launch(g, "dwconv2d_s2", &a, sizeof a, T1 * ((F1 + fb - 1) / fb), batch, 1, 256, 1, 1);
}

int nk_conv2d_c1_dw_s2_b(gpu_t *g, const float *X, const float *W0, const float *b0, const float *W2,
                         const float *b2, float *Y, uint32_t T, uint32_t F, uint32_t T1, uint32_t F1, uint32_t T2,
                         uint32_t F2, uint32_t C, uint32_t batch) {
    if (F > NK_CONV02_FMAX) return gpu_fail(g, "nk_conv2d_c1_dw_s2: more than 256 mel bins");
    if (!T2 || !F2 || !batch) return 0;
    /* whole output rows per workgroup when there are enough rows to fill the GPU; one column per
     * workgroup for a single stream's few rows (measured: 8.6 us against 16.3 us with 4 columns
     * for a 24-row window, 112 us with whole rows for 64 windows of 65 rows) */
    const uint64_t rows = (uint64_t)T2 * batch;
    const uint32_t fb = rows >= 1024 ? F2 : rows >= 256 ? 4 : 1;
    NkConv02Args a = { X, W0, b0, W2, b2, Y, T, F, T1, F1, T2, F2, C, fb, T * F, T2 * F2 * C };
    return gpu_launch(g, "conv2d_c1_dw_s2", &a, sizeof a, T2 * ((F2 + fb - 1) / fb), batch, 1, 256, 1, 1);
}

int nk_mel_frames(gpu_t *g, const float *span, const int *tab, uint32_t F, const float *win, const float *fb,
                  const int *fb_lo, const int *fb_hi, const double *tw_re, const double *tw_im, const uint16_t *rev,
                  float *out) {
    if (!F) return 0;
    NkMelArgs a = { span, tab, win, fb, fb_lo, fb_hi, tw_re, tw_im, rev, out, F, 0 };
    return gpu_launch(g, "mel_frames", &a, sizeof a, F, 1, 1, 256, 1, 1);
}

int nk_flatten_cf_b(gpu_t *g, const float *X, float *Y, uint32_t T, uint32_t F, uint32_t C, uint32_t batch) {
    NkFlatArgs a = { X, Y, T, F, C, 0 };
    return gpu_launch(g, "flatten_cf", &a, sizeof a, blocks_for((uint64_t)T * F * C), batch, 1, 256, 1, 1);
}

int nk_conv2d_c1_s2_relu(gpu_t *g, const float *X, const float *W, const float *bias, float *Y, uint32_t T,
                         uint32_t F, uint32_t T1, uint32_t F1, uint32_t C) {
    return nk_conv2d_c1_s2_relu_b(g, X, W, bias, Y, T, F, T1, F1, C, 1);
}

int nk_dwconv2d_s2(gpu_t *g, const float *X, const float *W, const float *bias, float *Y, uint32_t T, uint32_t F,
                   uint32_t T1, uint32_t F1, uint32_t C) {
    return nk_dwconv2d_s2_b(g, X, W, bias, Y, T, F, T1, F1, C, 1);
}

int nk_flatten_cf(gpu_t *g, const float *X, float *Y, uint32_t T, uint32_t F, uint32_t C) {
    return nk_flatten_cf_b(g, X, Y, T, F, C, 1);
}

int nk_gather_rows(gpu_t *g, const float *src, uint32_t src_ld, const int *map, float *dst, uint32_t dst_ld,
                   uint32_t rows, uint32_t cols) {
    if (!rows) return 0;
    NkGatherArgs a = { src, dst, map, rows, cols, src_ld, dst_ld };
    return gpu_launch(g, "gather_rows", &a, sizeof a, blocks_for((uint64_t)rows * cols), 1, 1, 256, 1, 1);
}

int nk_scatter_rows(gpu_t *g, const float *src, uint32_t src_ld, const int *map, float *dst, uint32_t dst_ld,
                    uint32_t rows, uint32_t cols) {
    if (!rows) return 0;
    NkGatherArgs a = { src, dst, map, rows, cols, src_ld, dst_ld };
    return gpu_launch(g, "scatter_rows", &a, sizeof a, blocks_for((uint64_t)rows * cols), 1, 1, 256, 1, 1);
}

int nk_lstm_input_rows(gpu_t *g, const uint16_t *embed, const int *tok, const float *xsrc, const float *hc,
                       const int *hrow, float *A, uint32_t n, uint32_t P, uint32_t blank) {
    if (!n) return 0;
    NkLstmInArgs a = { embed, tok, xsrc, hc, hrow, A, n, P, blank, 0 };
    return gpu_launch(g, "lstm_input_rows", &a, sizeof a, blocks_for(2 * P), n, 1, 256, 1, 1);
}

int nk_lstm_cell_rows(gpu_t *g, const float *gates, float *hc, const int *crow_in, const int *crow_out,
                      const int *hrow_out, float *hout, uint32_t n, uint32_t P) {
    if (!n) return 0;
    NkLstmRowsArgs a = { gates, hc, crow_in, crow_out, hrow_out, hout, n, P };
    return gpu_launch(g, "lstm_cell_rows", &a, sizeof a, blocks_for(P), n, 1, 256, 1, 1);
}

int nk_joint_in_rows(gpu_t *g, const float *enc, const float *pred, const int *erow, const int *prow, float *jin,
                     uint32_t rows, uint32_t J) {
    if (!rows) return 0;
    NkJointInArgs a = { enc, pred, erow, prow, jin, rows, J };
    return gpu_launch(g, "joint_in_rows", &a, sizeof a, blocks_for(J), rows, 1, 256, 1, 1);
}

int nk_argmax_rows(gpu_t *g, const float *logits, uint32_t ld, uint32_t rows, uint32_t V, int *out) {
    if (!rows) return 0;
    NkArgmaxRowsArgs a = { logits, out, rows, V, ld, 0 };
    return gpu_launch(g, "argmax_rows", &a, sizeof a, rows, 1, 1, 256, 1, 1);
}

int nk_copy(gpu_t *g, const float *src, float *dst, uint32_t n) {
    NkCopyArgs a = { src, dst, n, 0 };
    return gpu_launch(g, "copy_f32", &a, sizeof a, blocks_for(n), 1, 1, 256, 1, 1);
}

int nk_copy2d(gpu_t *g, const float *src, uint32_t src_ld, float *dst, uint32_t dst_ld, uint32_t rows, uint32_t cols) {
    NkCopy2dArgs a = { src, dst, rows, cols, src_ld, dst_ld };
    return gpu_launch(g, "copy2d_f32", &a, sizeof a, blocks_for((uint64_t)rows * cols), 1, 1, 256, 1, 1);
}

int nk_fill(gpu_t *g, float *dst, uint32_t n, float value) {
    NkFillArgs a = { dst, n, value };
    return gpu_launch(g, "fill_f32", &a, sizeof a, blocks_for(n), 1, 1, 256, 1, 1);
}

int nk_compact(gpu_t *g, float *base, uint64_t stride, uint32_t nbuf, uint32_t rows, uint32_t cols, uint32_t src_row,
               uint32_t dst_row) {
    if (!rows || !nbuf) return 0;
    if (src_row < dst_row + rows && dst_row < src_row + rows) return bad(g, "compact: overlapping rows");
    NkCompactArgs a = { base, stride, nbuf, rows, cols, src_row, dst_row, 0 };
    if (cols % 4 == 0 && stride % 4 == 0 && (uintptr_t)base % 16 == 0)
        return gpu_launch(g, "compact_rows4", &a, sizeof a, blocks_for((uint64_t)rows * cols / 4), nbuf, 1, 256, 1, 1);
    return gpu_launch(g, "compact_rows", &a, sizeof a, blocks_for((uint64_t)rows * cols), nbuf, 1, 256, 1, 1);
}


/* ---- kernels of the reference-shaped dispatch only (gpu_ref.c) -------------------------------- */
int nk_glu(gpu_t *g, const float *X, float *Y, uint32_t M, uint32_t D) {
    if (!M || !D) return 0;
    NkGluArgs a = { X, Y, M, D };
    return gpu_launch(g, "glu_rows", &a, sizeof a, blocks_for(D), M, 1, 256, 1, 1);
}

int nk_lstm_cell(gpu_t *g, const float *gates, const float *c_in, float *c_out, float *h_out, uint32_t H) {
    if (!H) return 0;
    NkLstmCellArgs a = { gates, c_in, c_out, h_out, H };
    return gpu_launch(g, "lstm_cell_vec", &a, sizeof a, blocks_for(H), 1, 1, 256, 1, 1);
}

int nk_joint_partial(gpu_t *g, const float *enc, const float *pred, const uint16_t *W, const float *bias,
                     float *part_v, int *part_i, uint32_t V, uint32_t H, uint32_t enc_row, uint32_t enc_ld,
                     uint32_t groups, uint32_t rows) {
    if (!rows || !groups) return 0;
    if (H % 4 || H > NK_JOINT_MAX_H || ((uintptr_t)W & 7))
        return bad(g, "joint_partial: H % 4 == 0, H <= 1024, W 8-byte aligned");
    NkJointPartArgs a = { enc, pred, W, bias, part_v, part_i, V, H, enc_row, enc_ld, groups };
    return gpu_launch(g, "joint_partial_groups", &a, sizeof a, groups, rows, 1, 512, 1, 1);
}

int nk_argmax_reduce(gpu_t *g, const float *part_v, const int *part_i, int *out, uint32_t n, uint32_t rows) {
    if (!rows) return 0;
    NkArgmaxPartArgs a = { part_v, part_i, out, n };
    return gpu_launch(g, "argmax_partials", &a, sizeof a, rows, 1, 1, 256, 1, 1);
}
