/* The reference's dispatch interface (src/gpu.h:29-41) on this library's launchers.
 *
 * A dispatch names a kernel of src/kernels.metal and binds argument i as a buffer + byte offset or
 * as an inline parameter block (src/gpu.m:90-101).  Here a table maps each name to the launcher of
 * the same computation: the buffer arguments become device addresses (buffer base + offset), the
 * parameter block (include/nemo_kernel_params.h, src/kernel_params.h:22-32) is unpacked into the
 * launcher's sizes.  Each launcher derives its own grid from those sizes, so the reference's grid
 * is not used, with one exception: joint_partial takes the number of partial-best groups per row
 * and the row count from the threadgroup grid (src/decoder.c:86), since its output layout depends
 * on them.  Function constants (gemm_spec / gemm_mma specialisations) choose nothing here: the
 * GEMM kernel is picked by this library's policy from (M, N, K).
 * Every argument is checked (count, kind, parameter block size, offset inside its buffer) before
 * anything is launched; a mismatch fails the batch with a message, like a bad pipeline would. */
#include "gpu.h"
#include "nemo_gpu.h"
#include "nemo_kernel_params.h"
#include "nemo_kernels.h"
#include <stdio.h>
#include <string.h>

typedef struct {
    void *p[8];          /* device address of each buffer argument */
    const void *params;  /* the parameter block */
    uint32_t groups_x, groups_y;
} ref_call_t;

typedef int (*ref_fn)(gpu_t *g, const ref_call_t *c);

/* gemm_spec / gemm_mma / gemm_bf16: A, W, bias (A when has_bias == 0), C, GemmParams
 * (src/kernels.metal:12-16, :58-62, :132-136; src/model.c:70-99) */
static int r_gemm(gpu_t *g, const ref_call_t *c) {
    const GemmParams *p = c->params;
    if (p->act > 3) return gpu_fail(g, "gemm: act must be 0..3");
    return nk_gemm(g, c->p[0], p->lda, c->p[1], p->ldw, p->has_bias ? c->p[2] : NULL, c->p[3], p->ldc, p->M, p->N,
                   p->K, (int)p->act, (int)p->accumulate, p->alpha);
}
/* X, gamma, beta, Y, LnParams (src/kernels.metal:258-262) */
static int r_layernorm(gpu_t *g, const ref_call_t *c) {
    const LnParams *p = c->params;
    return nk_layernorm(g, c->p[0], c->p[1], c->p[2], c->p[3], p->M, p->D, p->eps);
}
/* X, g1, b1, g2, b2, Y1, Y2, LnParams (src/kernels.metal:212-219) */
static int r_layernorm2(gpu_t *g, const ref_call_t *c) {
    const LnParams *p = c->params;
    return nk_layernorm2(g, c->p[0], c->p[1], c->p[2], c->p[3], c->p[4], c->p[5], c->p[6], p->M, p->D, p->eps);
}
/* Q, K, V, P, bias_u, bias_v, O, AttnParams (src/kernels.metal:293-300) */
static int r_attention(gpu_t *g, const ref_call_t *c) {
    const AttnParams *p = c->params;
    if (p->ldq != p->ldk) return gpu_fail(g, "attention_rel: Q and K/V rows must share one stride (ldq == ldk)");
    return nk_attention_rel(g, c->p[0], p->ldq, c->p[1], c->p[2], p->ldk, c->p[3], c->p[4], c->p[5], c->p[6], p->c,
                            p->L, p->Lmax, p->H, p->dh, p->D, p->scale);
}
/* X, Y, GluParams (src/kernels.metal:349-356) */
static int r_glu(gpu_t *g, const ref_call_t *c) {
    const GluParams *p = c->params;
    return nk_glu(g, c->p[0], c->p[1], p->M, p->D);
}
/* din, W, gamma, beta, Y, DwParams (src/kernels.metal:361-366) */
static int r_dwconv(gpu_t *g, const ref_call_t *c) {
    const DwParams *p = c->params;
    return nk_dwconv_ln_silu(g, c->p[0], c->p[1], c->p[2], c->p[3], c->p[4], p->c, p->D, p->taps, p->eps);
}
/* X, W, bias, Y, Conv2dParams (src/kernels.metal:413-417, :435-439) */
static int r_conv0(gpu_t *g, const ref_call_t *c) {
    const Conv2dParams *p = c->params;
    return nk_conv2d_c1_s2_relu(g, c->p[0], c->p[1], c->p[2], c->p[3], p->T, p->F, p->T1, p->F1, p->C);
}
static int r_dwconv2d(gpu_t *g, const ref_call_t *c) {
    const Conv2dParams *p = c->params;
    return nk_dwconv2d_s2(g, c->p[0], c->p[1], c->p[2], c->p[3], p->T, p->F, p->T1, p->F1, p->C);
}
/* X, Y, FlatParams (src/kernels.metal:457-462) */
static int r_flatten(gpu_t *g, const ref_call_t *c) {
    const FlatParams *p = c->params;
    return nk_flatten_cf(g, c->p[0], c->p[1], p->T, p->F, p->C);
}
/* src, dst, CountParams / dst, FillParams (src/kernels.metal:464-472) */
static int r_copy(gpu_t *g, const ref_call_t *c) {
    const CountParams *p = c->params;
    return nk_copy(g, c->p[0], c->p[1], p->n);
}
static int r_fill(gpu_t *g, const ref_call_t *c) {
    const FillParams *p = c->params;
    return nk_fill(g, c->p[0], p->n, p->value);
}
/* gates, c_in, c_out, h_out, LstmParams (src/kernels.metal:474-486) */
static int r_lstm(gpu_t *g, const ref_call_t *c) {
    const LstmParams *p = c->params;
    return nk_lstm_cell(g, c->p[0], c->p[1], c->p[2], c->p[3], p->H);
}
/* enc, pred, W, bias, part_v, part_i, JointParams; grid (groups, rows) (src/kernels.metal:490-496) */
static int r_joint(gpu_t *g, const ref_call_t *c) {
    const JointParams *p = c->params;
    return nk_joint_partial(g, c->p[0], c->p[1], c->p[2], c->p[3], c->p[4], c->p[5], p->V, p->H, p->enc_row, p->enc_ld,
                            c->groups_x, c->groups_y);
}
/* part_v, part_i, out, CountParams; grid (rows) (src/kernels.metal:522-525) */
static int r_argmax(gpu_t *g, const ref_call_t *c) {
    const CountParams *p = c->params;
    return nk_argmax_reduce(g, c->p[0], c->p[1], c->p[2], p->n, c->groups_x);
}

static const struct {
    const char *name;
    int nbuf;          /* buffer arguments, then one parameter block */
    size_t psize;
    ref_fn fn;
} k_table[] = {
    { "gemm_spec", 4, sizeof(GemmParams), r_gemm },
    { "gemm_mma", 4, sizeof(GemmParams), r_gemm },
    { "gemm_bf16", 4, sizeof(GemmParams), r_gemm },
    { "layernorm", 4, sizeof(LnParams), r_layernorm },
    { "layernorm2", 7, sizeof(LnParams), r_layernorm2 },
    { "attention_rel", 7, sizeof(AttnParams), r_attention },
    { "glu", 2, sizeof(GluParams), r_glu },
    { "dwconv_ln_silu", 5, sizeof(DwParams), r_dwconv },
    { "conv2d_c1_s2_relu", 4, sizeof(Conv2dParams), r_conv0 },
    { "dwconv2d_s2", 4, sizeof(Conv2dParams), r_dwconv2d },
    { "flatten_cf", 2, sizeof(FlatParams), r_flatten },
    { "copy_f32", 2, sizeof(CountParams), r_copy },
    { "fill_f32", 1, sizeof(FillParams), r_fill },
    { "lstm_cell", 4, sizeof(LstmParams), r_lstm },
    { "joint_partial", 6, sizeof(JointParams), r_joint },
    { "argmax_reduce", 3, sizeof(CountParams), r_argmax },
};

static int dispatch(gpu_t *g, const char *kernel, const gpu_arg_t *args, int nargs, uint32_t groups_x,
                    uint32_t groups_y) {
    char msg[160];
    if (!kernel) return gpu_fail(g, "dispatch: no kernel name");
    for (size_t k = 0; k < sizeof k_table / sizeof *k_table; ++k) {
        if (strcmp(k_table[k].name, kernel)) continue;
        const int nb = k_table[k].nbuf;
        if (nargs != nb + 1 || !args) {
            snprintf(msg, sizeof msg, "dispatch %s: %d arguments, expected %d buffers and a parameter block", kernel,
                     nargs, nb);
            return gpu_fail(g, msg);
        }
        ref_call_t c;
        memset(&c, 0, sizeof c);
        for (int i = 0; i < nb; ++i) {
            if (!args[i].buf || args[i].offset >= gpu_buf_len(args[i].buf)) {
                snprintf(msg, sizeof msg, "dispatch %s: argument %d must be a buffer with its offset inside it", kernel, i);
                return gpu_fail(g, msg);
            }
            c.p[i] = (char *)gpu_buf_dptr(args[i].buf) + args[i].offset;
        }
        if (args[nb].buf || !args[nb].bytes || args[nb].size != k_table[k].psize) {
            snprintf(msg, sizeof msg, "dispatch %s: argument %d must be its %zu-byte parameter block", kernel, nb,
                     k_table[k].psize);
            return gpu_fail(g, msg);
        }
        c.params = args[nb].bytes;
        c.groups_x = groups_x;
        c.groups_y = groups_y;
        return k_table[k].fn(g, &c);
    }
    snprintf(msg, sizeof msg, "no kernel %s", kernel);
    return gpu_fail(g, msg);
}

static uint32_t groups_of(uint32_t threads, uint32_t per) { return per ? (threads + per - 1) / per : 0; }

int gpu_dispatch(gpu_t *g, const char *kernel, const gpu_arg_t *args, int nargs, uint32_t gx, uint32_t gy, uint32_t gz,
                 uint32_t tx, uint32_t ty, uint32_t tz) {
    (void)gz;
    (void)tz;
    return dispatch(g, kernel, args, nargs, groups_of(gx, tx), groups_of(gy, ty));
}

int gpu_dispatch_groups(gpu_t *g, const char *kernel, const gpu_arg_t *args, int nargs, uint32_t groups_x,
                        uint32_t groups_y, uint32_t groups_z, uint32_t tx, uint32_t ty, uint32_t tz) {
    (void)groups_z;
    (void)tx;
    (void)ty;
    (void)tz;
    return dispatch(g, kernel, args, nargs, groups_x, groups_y);
}

int gpu_dispatch_groups_fc(gpu_t *g, const char *kernel, const uint32_t *fc, int nfc, const gpu_arg_t *args, int nargs,
                           uint32_t groups_x, uint32_t groups_y, uint32_t groups_z, uint32_t tx, uint32_t ty,
                           uint32_t tz) {
    if (nfc < 0 || (nfc > 0 && !fc)) return gpu_fail(g, "dispatch: bad function constants");
    return gpu_dispatch_groups(g, kernel, args, nargs, groups_x, groups_y, groups_z, tx, ty, tz);
}
