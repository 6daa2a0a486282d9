#include "model.h"
#include "nemo_kernels.h"
#include "ckpt.h"
#include "../kernel_params.h"
#include <fcntl.h>
#include <math.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec / 1e6;
}

static char *slurp(const char *path, size_t *len) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    char *b = malloc((size_t)n + 1);
    if (n < 0 || fread(b, 1, (size_t)n, f) != (size_t)n) { fclose(f); free(b); return NULL; }
    fclose(f);
    b[n] = 0;
    *len = (size_t)n;
    return b;
}

/* config.json: the keys the reference reads and its defaults for absent ones (src/model.c:125-172),
 * as a table of (section, key, default) -> integer field. */
typedef struct { const char *section, *key; int dflt; size_t field; } cfg_key_t;
#define CFG_FIELD(f) offsetof(model_cfg_t, f)
static const cfg_key_t k_cfg_keys[] = {
    { "encoder", "feat_in", 128, CFG_FIELD(feat_in) },
    { "encoder", "n_layers", 24, CFG_FIELD(n_layers) },
    { "encoder", "d_model", 1024, CFG_FIELD(d_model) },
    { "encoder", "n_heads", 8, CFG_FIELD(n_heads) },
    { "encoder", "ff_expansion_factor", 4, CFG_FIELD(d_ff) },          /* scaled by d_model below */
    { "encoder", "subsampling_factor", 8, CFG_FIELD(subsampling) },
    { "encoder", "subsampling_conv_channels", 256, CFG_FIELD(sub_channels) },
    { "encoder", "conv_kernel_size", 9, CFG_FIELD(conv_kernel) },
    { "prompt", "num_prompts", 128, CFG_FIELD(num_prompts) },
    { "prompt", "prompt_hidden", 2048, CFG_FIELD(prompt_hidden) },
    { "decoder", "pred_hidden", 640, CFG_FIELD(pred_hidden) },
    { "decoder", "pred_rnn_layers", 2, CFG_FIELD(pred_layers) },
    { "decoder", "vocab_size", 13087, CFG_FIELD(vocab_size) },
    { "joint", "joint_hidden", 640, CFG_FIELD(joint_hidden) },
    { "joint", "num_classes", 13087, CFG_FIELD(num_classes) },         /* + 1 (blank) below */
    { NULL, "max_symbols", 10, CFG_FIELD(max_symbols) },                /* top level */
};

static int cfg_int(const jn_t *sec, const char *key, int dflt) { return (int)jn_num(jn_get(sec, key), dflt); }

/* The shapes the kernels and launch plans are written for; anything else is refused at load. */
static const char *unsupported(const model_cfg_t *g) {
    if (g->pred_layers != 2) return "a prediction network of other than 2 LSTM layers";
    if (g->head_dim != 128) return "an attention head width other than 128";
    if (g->conv_kernel != 9 || g->subsampling != 8) return "a conv kernel other than 9 or subsampling other than 8";
    if (g->d_model % 32 || g->d_model > NK_ROW_MAX || g->prompt_hidden % 32 || g->sub_channels % 32)
        return "model widths that are not multiples of 32 (or above the row limit)";
    if (g->pred_hidden % 8 || g->joint_hidden % 8 || g->joint_hidden > NK_JOINT_MAX_H) return "decoder widths";
    if (g->num_classes > 32 * NK_DEC_GROUPS) return "a vocabulary above the joint kernels' limit";
    return NULL;
}

static int read_config(model_t *m, char *err, size_t errlen) {
    const jn_t *root = m->config, *pre = jn_get(root, "preprocessor"), *enc = jn_get(root, "encoder");
    const jn_t *prm = jn_get(root, "prompt");
    if (!pre || !enc || !prm || !jn_get(root, "decoder") || !jn_get(root, "joint")) {
        snprintf(err, errlen, "config.json: need the preprocessor, encoder, prompt, decoder and joint sections");
        return -1;
    }
    model_cfg_t *g = &m->cfg;
    for (size_t i = 0; i < sizeof k_cfg_keys / sizeof k_cfg_keys[0]; ++i) {
        const cfg_key_t *k = &k_cfg_keys[i];
        *(int *)((char *)g + k->field) = cfg_int(k->section ? jn_get(root, k->section) : root, k->key, k->dflt);
    }
    g->d_ff *= g->d_model;
    g->head_dim = g->n_heads > 0 ? g->d_model / g->n_heads : 0;
    g->blank_id = g->vocab_size;
    g->num_classes += 1;
    g->ln_eps = 1e-5f;
    /* att_context_size: [[left, right], ...], the trained (left, right) pairs */
    const jn_t *ctx = jn_get(enc, "att_context_size");
    g->n_trained = 0;
    for (size_t i = 0; i < jn_len(ctx) && g->n_trained < 8; ++i) {
        g->att_left = (int)jn_num(jn_at(jn_at(ctx, i), 0), 56);
        g->trained_right[g->n_trained++] = (int)jn_num(jn_at(jn_at(ctx, i), 1), 13);
    }
    g->att_right_default = (int)jn_num(jn_at(jn_get(root, "default_att_context_size"), 1), 13);
    const char *why = unsupported(g);
    if (why) {
        snprintf(err, errlen, "config.json: unsupported architecture (%s)", why);
        return -1;
    }
    if (cfg_int(pre, "sample_rate", 16000) != 16000 || cfg_int(pre, "features", 128) != 128) {
        snprintf(err, errlen, "config.json: the front end must be 16 kHz, 128 mel bins");
        return -1;
    }
    /* attention window: left context + the widest trained chunk + the two extra rows a final
     * boundary window can yield */
    int widest = 0;
    for (int i = 0; i < g->n_trained; ++i) widest = g->trained_right[i] > widest ? g->trained_right[i] : widest;
    m->Lmax = g->att_left + widest + 1 + 2;
    if (m->Lmax > NK_ATT_MAX_L) {
        snprintf(err, errlen, "config.json: attention window of %d rows, the kernels take %d", m->Lmax, NK_ATT_MAX_L);
        return -1;
    }
    m->prompt_dict = jn_get(prm, "prompt_dictionary");
    if (vocab_load(jn_get(root, "vocabulary"), &m->vocab)) {
        snprintf(err, errlen, "config.json: no vocabulary");
        return -1;
    }
    return 0;
}

int model_right_context_trained(const model_t *m, int right) {
    for (int i = 0; i < m->cfg.n_trained; ++i) if (m->cfg.trained_right[i] == right) return 1;
    return 0;
}
int model_prompt_index(const model_t *m, const char *lang) {
    const jn_t *v = jn_get(m->prompt_dict, lang);
    return v ? (int)jn_num(v, -1) : -1;
}

/* ---- tensor lists ------------------------------------------------------------------------- */
typedef struct { char name[128]; size_t numel; const uint16_t **dst; } breq_t;
typedef struct { char name[128]; size_t numel; const float **dst; } freq_t;
typedef struct {
    breq_t *b; size_t nb, cb;
    freq_t *f; size_t nf, cf;
} reqs_t;

static void addb(reqs_t *r, const char *name, size_t numel, const uint16_t **dst) {
    if (r->nb == r->cb) { r->cb = r->cb ? 2 * r->cb : 64; r->b = realloc(r->b, r->cb * sizeof *r->b); }
    snprintf(r->b[r->nb].name, sizeof r->b[r->nb].name, "%s", name);
    r->b[r->nb].numel = numel;
    r->b[r->nb].dst = dst;
    r->nb++;
}
static void addf(reqs_t *r, const char *name, size_t numel, const float **dst) {
    if (r->nf == r->cf) { r->cf = r->cf ? 2 * r->cf : 64; r->f = realloc(r->f, r->cf * sizeof *r->f); }
    snprintf(r->f[r->nf].name, sizeof r->f[r->nf].name, "%s", name);
    r->f[r->nf].numel = numel;
    r->f[r->nf].dst = dst;
    r->nf++;
}

/* Every tensor the model reads must be present, bf16 and of the expected element count (the
 * reference's checks, src/model.c:41-47). */
static const ck_tensor_t *need(const ckpt_t *ck, const char *name, size_t numel, char *err, size_t errlen) {
    const ck_tensor_t *t = ckpt_find(ck, name);
    if (!t) snprintf(err, errlen, "checkpoint has no tensor %s", name);
    else if (t->dtype != CK_BF16) snprintf(err, errlen, "checkpoint tensor %s: expected bf16", name);
    else if (numel && t->numel != numel) snprintf(err, errlen, "checkpoint tensor %s: %zu elements, expected %zu", name, t->numel, numel);
    else return t;
    return NULL;
}

/* a bf16 tensor widened to f32 on the host */
static int read_widened(const ckpt_t *ck, const ck_tensor_t *t, float *dst) {
    uint16_t *raw = malloc(t->bytes ? t->bytes : 2);
    if (!raw || ckpt_read(ck, t, raw)) { free(raw); return -1; }
    for (size_t k = 0; k < t->numel; ++k) dst[k] = ck_bf16(raw[k]);
    free(raw);
    return 0;
}

#define WALIGN 4096
static size_t up_to(size_t x, size_t a) { return (x + a - 1) / a * a; }

model_t *model_load(const char *dir, char *err, size_t errlen) {
    const double t0 = now_ms();
    model_t *m = calloc(1, sizeof *m);
    m->prompt_index = -1;
    char path[4096];
    size_t len = 0;
    snprintf(path, sizeof path, "%s/config.json", dir);
    char *txt = slurp(path, &len);
    if (!txt) { snprintf(err, errlen, "cannot read %s", path); free(m); return NULL; }
    char jerr[160];
    m->config = jn_parse(txt, len, jerr, sizeof jerr);
    free(txt);
    if (!m->config) { snprintf(err, errlen, "config.json: %s", jerr); free(m); return NULL; }
    if (read_config(m, err, errlen)) { model_free(m); return NULL; }
    gpu_buf_t *wpos_d = NULL;
    snprintf(path, sizeof path, "%s/model.safetensors", dir);
    ckpt_t *st = ckpt_open(path, err, errlen);
    if (!st) { model_free(m); return NULL; }
    m->gpu = gpu_create(NULL, err, errlen);
    if (!m->gpu) { ckpt_close(st); model_free(m); return NULL; }

    const model_cfg_t *g = &m->cfg;
    const size_t D = (size_t)g->d_model, CH = (size_t)g->sub_channels, FF = (size_t)g->d_ff, nl = (size_t)g->n_layers;
    const size_t PH = (size_t)g->prompt_hidden, NP = (size_t)g->num_prompts, P = (size_t)g->pred_hidden;
    const size_t J = (size_t)g->joint_hidden, V = (size_t)g->num_classes;
    int freq = g->feat_in;
    for (int i = 0; i < 3; ++i) freq = freq / 2 + 1;
    m->sub_freq_out = freq;
    if ((CH * (size_t)freq) % 32) { snprintf(err, errlen, "unsupported subsampling output width"); ckpt_close(st); model_free(m); return NULL; }
    m->L = calloc(nl, sizeof *m->L);

    reqs_t r = { 0 };
    char n[160];
    const char *pe = "encoder.pre_encode.";
#define PB(suffix, numel, dst) do { snprintf(n, sizeof n, "%s%s", pe, suffix); addb(&r, n, numel, dst); } while (0)
#define PF(suffix, numel, dst) do { snprintf(n, sizeof n, "%s%s", pe, suffix); addf(&r, n, numel, dst); } while (0)
    PF("conv.0.weight", CH * 9, &m->conv0_w); PF("conv.0.bias", CH, &m->conv0_b);
    PF("conv.2.weight", CH * 9, &m->conv2_w); PF("conv.2.bias", CH, &m->conv2_b);
    PB("conv.3.weight", CH * CH, &m->conv3_w); PF("conv.3.bias", CH, &m->conv3_b);
    PF("conv.5.weight", CH * 9, &m->conv5_w); PF("conv.5.bias", CH, &m->conv5_b);
    PB("conv.6.weight", CH * CH, &m->conv6_w); PF("conv.6.bias", CH, &m->conv6_b);
    PB("out.weight", D * CH * (size_t)freq, &m->pre_out_w); PF("out.bias", D, &m->pre_out_b);
    const uint16_t *qkv_tail = NULL; /* k and v land right after q; only q's address is kept */
    for (size_t l = 0; l < nl; ++l) {
        layer_dev_t *L = &m->L[l];
#define LB(suffix, numel, dst) do { snprintf(n, sizeof n, "encoder.layers.%zu.%s", l, suffix); addb(&r, n, numel, dst); } while (0)
#define LF(suffix, numel, dst) do { snprintf(n, sizeof n, "encoder.layers.%zu.%s", l, suffix); addf(&r, n, numel, dst); } while (0)
        LB("feed_forward1.linear1.weight", FF * D, &L->ff1_w1);
        LB("feed_forward1.linear2.weight", D * FF, &L->ff1_w2);
        /* q, k, v consecutive: one [3D][D] matrix (src/model.c:240-242) */
        LB("self_attn.linear_q.weight", D * D, &L->wqkv);
        LB("self_attn.linear_k.weight", D * D, &qkv_tail);
        LB("self_attn.linear_v.weight", D * D, &qkv_tail);
        LB("self_attn.linear_out.weight", D * D, &L->wo);
        LB("conv.pointwise_conv1.weight", 2 * D * D, &L->pw1);
        LB("conv.pointwise_conv2.weight", D * D, &L->pw2);
        LB("feed_forward2.linear1.weight", FF * D, &L->ff2_w1);
        LB("feed_forward2.linear2.weight", D * FF, &L->ff2_w2);
        LF("norm_feed_forward1.weight", D, &L->ln_ff1_g); LF("norm_feed_forward1.bias", D, &L->ln_ff1_b);
        LF("norm_self_att.weight", D, &L->ln_att_g); LF("norm_self_att.bias", D, &L->ln_att_b);
        LF("norm_conv.weight", D, &L->ln_conv_g); LF("norm_conv.bias", D, &L->ln_conv_b);
        LF("norm_feed_forward2.weight", D, &L->ln_ff2_g); LF("norm_feed_forward2.bias", D, &L->ln_ff2_b);
        LF("norm_out.weight", D, &L->ln_out_g); LF("norm_out.bias", D, &L->ln_out_b);
        LF("conv.batch_norm.weight", D, &L->bn_g); LF("conv.batch_norm.bias", D, &L->bn_b);
        LF("conv.depthwise_conv.weight", D * 9, &L->dw_w);
        LF("self_attn.pos_bias_u", D, &L->bias_u); LF("self_attn.pos_bias_v", D, &L->bias_v);
#undef LB
#undef LF
    }
    addb(&r, "prompt_kernel.0.weight", PH * (D + NP), &m->prompt_w0);
    addb(&r, "prompt_kernel.2.weight", D * PH, &m->prompt_w2);
    addf(&r, "prompt_kernel.2.bias", D, &m->prompt_b2);
    addb(&r, "joint.enc.weight", J * D, &m->joint_enc_w); addf(&r, "joint.enc.bias", J, &m->joint_enc_b);
    for (int l = 0; l < 2; ++l) {
        snprintf(n, sizeof n, "decoder.prediction.dec_rnn.lstm.%d.Wx", l); addb(&r, n, 4 * P * P, &m->lstm_wx[l]);
        snprintf(n, sizeof n, "decoder.prediction.dec_rnn.lstm.%d.Wh", l); addb(&r, n, 4 * P * P, &m->lstm_wh[l]);
        snprintf(n, sizeof n, "decoder.prediction.dec_rnn.lstm.%d.bias", l); addf(&r, n, 4 * P, &m->lstm_b[l]);
    }
    addb(&r, "joint.pred.weight", J * P, &m->joint_pred_w); addf(&r, "joint.pred.bias", J, &m->joint_pred_b);
    addb(&r, "joint.joint_net.2.weight", V * J, &m->joint_out_w); addf(&r, "joint.joint_net.2.bias", V, &m->joint_out_b);
    addb(&r, "decoder.prediction.embed.weight", (size_t)(g->vocab_size + 1) * P, &m->embed_dev);
#undef PB
#undef PF

    /* validate every tensor, size the arenas */
    size_t wbytes = 0, fcount = 0;
    const ck_tensor_t **bt = calloc(r.nb, sizeof *bt), **ft = calloc(r.nf, sizeof *ft);
    int ok = 1;
    for (size_t i = 0; i < r.nb && ok; ++i) {
        if (!(bt[i] = need(st, r.b[i].name, r.b[i].numel, err, errlen))) ok = 0;
        else {
            /* q|k|v pack tightly so the three form one matrix */
            const int packed = strstr(r.b[i].name, "linear_k.weight") || strstr(r.b[i].name, "linear_v.weight");
            wbytes = (packed ? wbytes : up_to(wbytes, WALIGN)) + bt[i]->bytes;
        }
    }
    for (size_t i = 0; i < r.nf && ok; ++i) {
        if (!(ft[i] = need(st, r.f[i].name, r.f[i].numel, err, errlen))) ok = 0;
        else fcount += up_to(ft[i]->numel, 64);
    }
    const ck_tensor_t *emb = ok ? need(st, "decoder.prediction.embed.weight", (size_t)(g->vocab_size + 1) * P, err, errlen) : NULL;
    const ck_tensor_t *w0 = ok ? need(st, "prompt_kernel.0.weight", PH * (D + NP), err, errlen) : NULL;
    const ck_tensor_t *b0 = ok ? need(st, "prompt_kernel.0.bias", PH, err, errlen) : NULL;
    const ck_tensor_t *wpos0 = ok ? need(st, "encoder.layers.0.self_attn.linear_pos.weight", D * D, err, errlen) : NULL;
    if (!ok || !emb || !w0 || !b0 || !wpos0) goto fail;
    m->warena = gpu_buf_alloc(m->gpu, wbytes);
    m->farena = gpu_buf_alloc(m->gpu, fcount * sizeof(float));
    if (!m->warena || !m->farena) { snprintf(err, errlen, "cannot allocate the weight arenas (%zu MB)", wbytes >> 20); goto fail; }
    m->warena_bytes = wbytes;
    /* the per-layer linear_pos weights feed the position tables only: they go to a temporary
       buffer with the same file -> device copy as the arena */
    wpos_d = gpu_buf_alloc(m->gpu, nl * D * D * sizeof(uint16_t));
    if (!wpos_d) { snprintf(err, errlen, "cannot allocate the position weights"); goto fail; }
    {
        char *wbase = gpu_buf_dptr(m->warena);
        gpu_file_range_t *rg = calloc(r.nb + nl, sizeof *rg);
        size_t off = 0;
        for (size_t i = 0; i < r.nb; ++i) {
            const int packed = strstr(r.b[i].name, "linear_k.weight") || strstr(r.b[i].name, "linear_v.weight");
            if (!packed) off = up_to(off, WALIGN);
            rg[i] = (gpu_file_range_t){ bt[i]->at, bt[i]->bytes, wbase + off };
            *r.b[i].dst = (const uint16_t *)(wbase + off);
            off += bt[i]->bytes;
        }
        int urc = 0;
        for (size_t l = 0; l < nl && !urc; ++l) {
            snprintf(n, sizeof n, "encoder.layers.%zu.self_attn.linear_pos.weight", l);
            const ck_tensor_t *t = need(st, n, D * D, err, errlen);
            if (!t) urc = -2;
            else rg[r.nb + l] = (gpu_file_range_t){ t->at, t->bytes, (uint16_t *)gpu_buf_dptr(wpos_d) + l * D * D };
        }
        if (!urc) {
            urc = gpu_upload_file(m->gpu, ckpt_fd(st), rg, r.nb + nl);
            if (urc) snprintf(err, errlen, "weight upload: %s", gpu_last_error(m->gpu));
        }
        free(rg);
        if (urc) goto fail;
        float *fh = calloc(fcount ? fcount : 1, sizeof(float));
        float *fbase = gpu_buf_dptr(m->farena);
        size_t fo = 0;
        int rrc = !fh;
        for (size_t i = 0; i < r.nf && !rrc; ++i) {
            rrc = read_widened(st, ft[i], fh + fo);
            *r.f[i].dst = fbase + fo;
            fo += up_to(ft[i]->numel, 64);
        }
        const int rc = rrc ? -1 : gpu_upload(m->gpu, fbase, fh, fcount * sizeof(float));
        free(fh);
        if (rrc) { snprintf(err, errlen, "%s: reading the small tensors failed", path); goto fail; }
        if (rc) { snprintf(err, errlen, "param upload: %s", gpu_last_error(m->gpu)); goto fail; }
    }
    /* host copies: embedding rows (read per emitted token) and the prompt fold inputs */
    m->embed_host = malloc(emb->bytes);
    m->b0_host = malloc(PH * sizeof(float));
    m->w0_prompt_host = malloc(PH * NP * sizeof(float));
    {
        uint16_t *w = malloc(w0->bytes);
        int rrc = !m->embed_host || !m->b0_host || !m->w0_prompt_host || !w;
        if (!rrc) rrc = ckpt_read(st, emb, m->embed_host) || ckpt_read(st, w0, w) || read_widened(st, b0, m->b0_host);
        for (size_t i = 0; i < PH && !rrc; ++i)
            for (size_t p = 0; p < NP; ++p) m->w0_prompt_host[i * NP + p] = ck_bf16(w[i * (D + NP) + D + p]);
        free(w);
        if (rrc) { snprintf(err, errlen, "%s: reading the embedding and prompt tensors failed", path); goto fail; }
    }
    m->b0_eff_buf = gpu_buf_alloc(m->gpu, PH * sizeof(float));
    m->prompt_b0_eff = gpu_buf_dptr(m->b0_eff_buf);

    /* relative position tables (src/model.c:286-306): sinusoid rows for positions Lmax-1 .. -(Lmax-1)
       in double on the host, then ptab[l] = pe . wpos[l]^T on the GPU */
    {
        const int Pr = 2 * m->Lmax - 1;
        float *peh = malloc((size_t)Pr * D * sizeof(float));
        for (int row = 0; row < Pr; ++row) {
            const double pos = (double)(m->Lmax - 1 - row);
            for (size_t i = 0; i < D / 2; ++i) {
                const double div = exp((double)(2 * i) * -(log(10000.0) / (double)D));
                peh[(size_t)row * D + 2 * i] = (float)sin(pos * div);
                peh[(size_t)row * D + 2 * i + 1] = (float)cos(pos * div);
            }
        }
        gpu_buf_t *pe_d = gpu_buf_alloc(m->gpu, (size_t)Pr * D * sizeof(float));
        m->ptab_buf = gpu_buf_alloc(m->gpu, nl * (size_t)Pr * D * sizeof(float));
        int rc = !pe_d || !m->ptab_buf;
        if (!rc) rc = gpu_upload(m->gpu, gpu_buf_dptr(pe_d), peh, (size_t)Pr * D * sizeof(float));
        free(peh);
        if (!rc) {
            gpu_begin(m->gpu);
            for (size_t l = 0; l < nl; ++l) {
                float *dst = (float *)gpu_buf_dptr(m->ptab_buf) + l * (size_t)Pr * D;
                nk_gemm(m->gpu, gpu_buf_dptr(pe_d), (uint32_t)D, (uint16_t *)gpu_buf_dptr(wpos_d) + l * D * D, (uint32_t)D,
                        NULL, dst, (uint32_t)D, (uint32_t)Pr, (uint32_t)D, (uint32_t)D, NK_ACT_NONE, 0, 1.0f);
                m->L[l].ptab = dst;
            }
            rc = gpu_end(m->gpu, err, errlen);
        } else {
            snprintf(err, errlen, "position table: %s", gpu_last_error(m->gpu));
        }
        gpu_buf_free(pe_d);
        gpu_buf_free(wpos_d);
        wpos_d = NULL;
        if (rc) goto fail;
    }
    free(bt);
    free(ft);
    free(r.b);
    free(r.f);
    ckpt_close(st);
    m->load_ms = now_ms() - t0;
    return m;
fail:
    gpu_buf_free(wpos_d);
    free(bt);
    free(ft);
    free(r.b);
    free(r.f);
    ckpt_close(st);
    model_free(m);
    return NULL;
}

/* src/model.c:312-322: the one-hot prompt folds into the first prompt layer's bias,
 * b_eff = b0 + W0[:, D + idx], in f32 on the host, uploaded once. */
int model_set_language(model_t *m, const char *lang, char *err, size_t errlen) {
    const int idx = model_prompt_index(m, lang);
    if (idx < 0 || idx >= m->cfg.num_prompts) { snprintf(err, errlen, "unknown language prompt %s", lang); return -1; }
    const size_t PH = (size_t)m->cfg.prompt_hidden, NP = (size_t)m->cfg.num_prompts;
    float *b = malloc(PH * sizeof(float));
    for (size_t i = 0; i < PH; ++i) b[i] = m->b0_host[i] + m->w0_prompt_host[i * NP + (size_t)idx];
    const int rc = gpu_upload(m->gpu, (void *)m->prompt_b0_eff, b, PH * sizeof(float));
    free(b);
    if (rc) { snprintf(err, errlen, "prompt bias upload: %s", gpu_last_error(m->gpu)); return -1; }
    m->prompt_index = idx;
    return 0;
}

void model_free(model_t *m) {
    if (!m) return;
    gpu_buf_free(m->warena);
    gpu_buf_free(m->farena);
    gpu_buf_free(m->ptab_buf);
    gpu_buf_free(m->b0_eff_buf);
    if (m->gpu) gpu_destroy(m->gpu);
    free(m->L);
    free(m->embed_host);
    free(m->b0_host);
    free(m->w0_prompt_host);
    vocab_release(&m->vocab);
    jn_free(m->config);
    free(m);
}
