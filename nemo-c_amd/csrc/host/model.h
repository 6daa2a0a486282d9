/* Model configuration and weights resident in HBM.
 *
 * Reads config.json and model.safetensors with the keys, tensor names and checks of the reference
 * (src/model.c:41-67 tensor checks, :125-172 config, :215-282 tensor list, :286-306 position
 * table, :312-322 prompt fold).  Layout on the device:
 *   - one bf16 weight arena, 4 KB-aligned matrices, in the order a chunk reads them
 *     (pre-encode, then per layer ff1, qkv, out, pw1, pw2, ff2, then prompt, joint, decoder);
 *     q, k and v are packed into one [3D][D] matrix for the fused QKV GEMM;
 *   - one f32 arena for norms, biases, depthwise and subsampling conv weights;
 *   - per-layer relative-position tables [2*Lmax-1][D] (f32), computed on the GPU at load.
 */
#ifndef NEMO_MODEL_H
#define NEMO_MODEL_H
#include "gpu.h"
#include "json.h"
#include "tokenizer.h"
#include <stdint.h>

typedef struct {
    int n_layers, d_model, n_heads, head_dim, d_ff, subsampling, sub_channels, conv_kernel, feat_in;
    int num_prompts, prompt_hidden, pred_hidden, pred_layers, vocab_size, blank_id, joint_hidden, num_classes;
    int max_symbols, att_left, att_right_default, trained_right[8], n_trained;
    float ln_eps;
} model_cfg_t;

typedef struct { /* device addresses */
    const uint16_t *ff1_w1, *ff1_w2, *ff2_w1, *ff2_w2, *wqkv, *wo, *pw1, *pw2;
    const float *ln_ff1_g, *ln_ff1_b, *ln_att_g, *ln_att_b, *ln_conv_g, *ln_conv_b, *ln_ff2_g, *ln_ff2_b;
    const float *ln_out_g, *ln_out_b, *bn_g, *bn_b, *dw_w, *bias_u, *bias_v;
    const float *ptab;
} layer_dev_t;

typedef struct model {
    model_cfg_t cfg;
    jn_t *config;
    const jn_t *prompt_dict;
    vocab_t vocab;
    gpu_t *gpu;
    gpu_buf_t *warena, *farena, *ptab_buf, *b0_eff_buf;
    size_t warena_bytes;
    layer_dev_t *L;
    int Lmax, sub_freq_out, prompt_index;
    /* subsampling */
    const float *conv0_w, *conv0_b, *conv2_w, *conv2_b, *conv3_b, *conv5_w, *conv5_b, *conv6_b, *pre_out_b;
    const uint16_t *conv3_w, *conv6_w, *pre_out_w;
    /* prompt */
    const uint16_t *prompt_w0, *prompt_w2;
    const float *prompt_b0_eff, *prompt_b2;
    float *b0_host;          /* prompt_kernel.0.bias widened */
    float *w0_prompt_host;   /* prompt_kernel.0.weight columns D..D+NP-1 widened, [PH][NP] */
    /* decoder + joint */
    const uint16_t *lstm_wx[2], *lstm_wh[2], *joint_enc_w, *joint_pred_w, *joint_out_w;
    const float *lstm_b[2], *joint_enc_b, *joint_pred_b, *joint_out_b;
    uint16_t *embed_host;    /* [vocab+1][pred_hidden] bf16 (host copy) */
    const uint16_t *embed_dev; /* the same table in the weight arena, read by the device decoder loop */
    double load_ms;
} model_t;

model_t *model_load(const char *dir, char *err, size_t errlen);
void model_free(model_t *m);
int model_prompt_index(const model_t *m, const char *lang);
int model_set_language(model_t *m, const char *lang, char *err, size_t errlen);
int model_right_context_trained(const model_t *m, int right);

#endif
