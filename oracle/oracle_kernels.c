/* ORACLE — test infrastructure only (see oracle.h).  CPU restatement of the reference kernels
 * in src/kernels.metal and the launcher parameters in src/model.c. */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

void or_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

static inline float bf(uint16_t v) { /* src/safetensors.h:32-36, src/kernels.metal:4 */
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)v << 16;
    return c.f;
}

/* src/kernels.metal:6-7: sigmoid = 1/(1+exp(-v)), SiLU = v/(1+exp(-v)) (a division, not v*sigmoid) */
float or_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }
float or_silu(float v) { return v / (1.0f + expf(-v)); }

/* GEMM with fused epilogue: src/kernels.metal:9-48 (gemm_bf16), :51-118 (gemm_spec), :120-208
 * (gemm_mma); semantics of the epilogue at :95-117 and :179-206; parameters from src/model.c:70-99.
 *   act 0/1/2: C[m][n] (=|+=) alpha * act(sum_k A[m][k] W[n][k] + bias[n])
 *   act 3 (GLU): N is the full weight height, output width N/2:
 *                C[m][j] (=|+=) (sa_j + b_j) * sigmoid(sb_{j+N/2} + b_{j+N/2}) * alpha
 * Each dot product is summed in f32 in increasing k; four columns are interleaved only to break
 * the add dependency chain, which leaves each column's order unchanged. */
/* Numerics study switch (not the reference's semantics, which is mode 0): the GEMMs' A operand as
 * f32 (0), rounded to bf16 (1), or as the bf16 pair hi = RNE(a), lo = RNE(a - hi) summed (2; the
 * split the batched GPU GEMMs feed their bf16 MFMAs).  Used by oracle/study_a_precision.py. */
static int g_a_mode;
void or_set_gemm_a_mode(int mode) { g_a_mode = mode; }
static float rne_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}
static float a_val(float a) {
    if (g_a_mode == 1) return rne_bf16(a);
    if (g_a_mode == 2) {
        const float hi = rne_bf16(a);
        return hi + rne_bf16(a - hi);
    }
    return a;
}

void or_gemm(const float *A, long lda, const uint16_t *W, long ldw, const float *bias,
             float *C, long ldc, int M, int N, int K, int act, int accumulate, float alpha) {
    const int glu = act == OR_ACT_GLU;
    const int nout = glu ? N / 2 : N;
    float *Ar = NULL;
    if (g_a_mode) {
        Ar = malloc(sizeof(float) * (size_t)M * (size_t)K);
        for (int m = 0; m < M; ++m)
            for (int k = 0; k < K; ++k) Ar[(size_t)m * K + k] = a_val(A[(size_t)m * lda + k]);
        A = Ar;
        lda = K;
    }
#pragma omp parallel
    {
        float *w = malloc(sizeof(float) * (size_t)K * 2);
        float *acc = malloc(sizeof(float) * (size_t)M * 2);
#pragma omp for schedule(static)
        for (int j = 0; j < nout; ++j) {
            const int na = j, nb = glu ? j + N / 2 : -1;
            for (int k = 0; k < K; ++k) w[k] = bf(W[(size_t)na * ldw + k]);
            if (glu) for (int k = 0; k < K; ++k) w[K + k] = bf(W[(size_t)nb * ldw + k]);
            for (int m = 0; m < M; ++m) {
                const float *a = A + (size_t)m * lda;
                float s0 = 0.0f, s1 = 0.0f;
                for (int k = 0; k < K; ++k) {
                    s0 += a[k] * w[k];
                    if (glu) s1 += a[k] * w[K + k];
                }
                acc[2 * m] = s0;
                acc[2 * m + 1] = s1;
            }
            for (int m = 0; m < M; ++m) {
                float v;
                if (glu) {
                    const float va = acc[2 * m] + (bias ? bias[na] : 0.0f);
                    const float vb = acc[2 * m + 1] + (bias ? bias[nb] : 0.0f);
                    v = va * or_sigmoid(vb) * alpha;
                } else {
                    v = acc[2 * m] + (bias ? bias[na] : 0.0f);
                    if (act == OR_ACT_SILU) v = or_silu(v);
                    else if (act == OR_ACT_RELU) v = v > 0.0f ? v : 0.0f;
                    v *= alpha;
                }
                float *c = C + (size_t)m * ldc + j;
                *c = accumulate ? (*c + v) : v;
            }
        }
        free(w);
        free(acc);
    }
    free(Ar);
}

/* One LayerNorm row: src/kernels.metal:257-288.  mean = sum/D; var = sum((x-mean)^2)/D (biased);
 * inv = 1/sqrt(var + eps); y = (x - mean) * inv * gamma + beta. */
static void ln_row(const float *x, const float *g, const float *b, float *y, int D, float eps) {
    float s = 0.0f;
    for (int i = 0; i < D; ++i) s += x[i];
    const float mean = s / (float)D;
    float v = 0.0f;
    for (int i = 0; i < D; ++i) { const float d = x[i] - mean; v += d * d; }
    const float inv = 1.0f / sqrtf(v / (float)D + eps);
    for (int i = 0; i < D; ++i) y[i] = (x[i] - mean) * inv * g[i] + b[i];
}

void or_layernorm(const float *X, const float *g, const float *b, float *Y, int M, int D, float eps) {
    for (int m = 0; m < M; ++m) ln_row(X + (size_t)m * D, g, b, Y + (size_t)m * D, D, eps);
}

/* Paired LayerNorm: src/kernels.metal:210-255.  Y1 = LN(X; g1,b1), Y2 = LN(Y1; g2,b2). */
void or_layernorm2(const float *X, const float *g1, const float *b1, const float *g2, const float *b2,
                   float *Y1, float *Y2, int M, int D, float eps) {
    for (int m = 0; m < M; ++m) {
        ln_row(X + (size_t)m * D, g1, b1, Y1 + (size_t)m * D, D, eps);
        ln_row(Y1 + (size_t)m * D, g2, b2, Y2 + (size_t)m * D, D, eps);
    }
}

/* Relative-position attention: src/kernels.metal:290-348, host parameters src/encoder.c:189-194.
 * For head h and query i (0 <= i < c), key j (0 <= j < L):
 *   prow = (Lmax - L) + (c - 1 - i + j)       (relative position (L - c + i) - j)
 *   s_j  = ((q + u) . K_j + (q + v) . P[prow]) * scale, over the head's dh dims
 *   O_i  = sum_j softmax(s)_j V_j             (no mask inside the chunk)            */
void or_attention_rel(const float *Q, long ldq, const float *K, const float *V, long ldk, const float *P,
                      const float *bu, const float *bv, float *O, int c, int L, int Lmax, int H, int dh, int D,
                      float scale) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int h = 0; h < H; ++h)
        for (int i = 0; i < c; ++i) {
            const int off = h * dh;
            float qu[256], qv[256], s[256];
            for (int d = 0; d < dh; ++d) {
                const float q = Q[(size_t)i * ldq + off + d];
                qu[d] = q + bu[off + d];
                qv[d] = q + bv[off + d];
            }
            float mx = -INFINITY;
            for (int j = 0; j < L; ++j) {
                const int prow = (Lmax - L) + (c - 1 - i + j);
                const float *k = K + (size_t)j * ldk + off, *p = P + (size_t)prow * D + off;
                float a = 0.0f;
                for (int d = 0; d < dh; ++d) a += qu[d] * k[d] + qv[d] * p[d];
                s[j] = a * scale;
                if (s[j] > mx) mx = s[j];
            }
            float sum = 0.0f;
            for (int j = 0; j < L; ++j) { s[j] = expf(s[j] - mx); sum += s[j]; }
            for (int j = 0; j < L; ++j) s[j] = s[j] / sum;
            for (int d = 0; d < dh; ++d) {
                float acc = 0.0f;
                for (int j = 0; j < L; ++j) acc += s[j] * V[(size_t)j * ldk + off + d];
                O[(size_t)i * D + off + d] = acc;
            }
        }
}

/* Causal depthwise conv + LayerNorm + SiLU: src/kernels.metal:359-409.
 * din holds (taps-1) history rows then the c new rows; W is [D][taps], no conv bias.
 *   v_ch = sum_tap W[ch][tap] * din[t + tap][ch];  y = SiLU(LN(v)). */
void or_dwconv_ln_silu(const float *din, const float *W, const float *g, const float *b, float *Y,
                       int c, int D, int taps, float eps) {
    float *v = malloc(sizeof(float) * (size_t)D);
    for (int t = 0; t < c; ++t) {
        for (int ch = 0; ch < D; ++ch) {
            float acc = 0.0f;
            for (int tap = 0; tap < taps; ++tap) acc += W[ch * taps + tap] * din[(size_t)(t + tap) * D + ch];
            v[ch] = acc;
        }
        ln_row(v, g, b, Y + (size_t)t * D, D, eps);
        for (int ch = 0; ch < D; ++ch) Y[(size_t)t * D + ch] = or_silu(Y[(size_t)t * D + ch]);
    }
    free(v);
}

/* Subsampling conv 0: src/kernels.metal:411-432. 1 -> C channels, 3x3, stride 2, causal padding
 * (2 before, 1 after) on time and frequency, + bias, ReLU.  X [T][F] -> Y [T1][F1][C]. */
void or_conv2d_c1_s2_relu(const float *X, const float *W, const float *bias, float *Y, int T, int F, int T1, int F1, int C) {
#pragma omp parallel for schedule(static)
    for (int t1 = 0; t1 < T1; ++t1)
        for (int f1 = 0; f1 < F1; ++f1)
            for (int o = 0; o < C; ++o) {
                float acc = bias[o];
                for (int kh = 0; kh < 3; ++kh) {
                    const int ti = 2 * t1 + kh - 2;
                    if (ti < 0 || ti >= T) continue;
                    for (int kw = 0; kw < 3; ++kw) {
                        const int fi = 2 * f1 + kw - 2;
                        if (fi < 0 || fi >= F) continue;
                        acc += W[o * 9 + kh * 3 + kw] * X[(size_t)ti * F + fi];
                    }
                }
                Y[((size_t)t1 * F1 + f1) * C + o] = acc > 0.0f ? acc : 0.0f;
            }
}

/* Depthwise 3x3 stride-2 conv, same causal padding, + bias, no activation:
 * src/kernels.metal:434-454.  X [T][F][C] -> Y [T1][F1][C]. */
void or_dwconv2d_s2(const float *X, const float *W, const float *bias, float *Y, int T, int F, int T1, int F1, int C) {
#pragma omp parallel for schedule(static)
    for (int t1 = 0; t1 < T1; ++t1)
        for (int f1 = 0; f1 < F1; ++f1)
            for (int ch = 0; ch < C; ++ch) {
                float acc = bias[ch];
                for (int kh = 0; kh < 3; ++kh) {
                    const int ti = 2 * t1 + kh - 2;
                    if (ti < 0 || ti >= T) continue;
                    for (int kw = 0; kw < 3; ++kw) {
                        const int fi = 2 * f1 + kw - 2;
                        if (fi < 0 || fi >= F) continue;
                        acc += W[ch * 9 + kh * 3 + kw] * X[((size_t)ti * F + fi) * C + ch];
                    }
                }
                Y[((size_t)t1 * F1 + f1) * C + ch] = acc;
            }
}

/* Channel-major flatten [T][F][C] -> [T][C*F]: src/kernels.metal:456-462. */
void or_flatten_cf(const float *X, float *Y, int T, int F, int C) {
    for (int t = 0; t < T; ++t)
        for (int f = 0; f < F; ++f)
            for (int ch = 0; ch < C; ++ch) Y[(size_t)t * C * F + (size_t)ch * F + f] = X[((size_t)t * F + f) * C + ch];
}

/* LSTM cell: src/kernels.metal:474-486.  gates [4H] in order i, f, g, o (already Wx x + b + Wh h).
 *   c' = sigmoid(f) c + sigmoid(i) tanh(g);  h' = sigmoid(o) tanh(c'). */
void or_lstm_cell(const float *gates, const float *c_in, float *c_out, float *h_out, int H) {
    for (int i = 0; i < H; ++i) {
        const float ig = or_sigmoid(gates[i]);
        const float fg = or_sigmoid(gates[H + i]);
        const float gg = tanhf(gates[2 * H + i]);
        const float og = or_sigmoid(gates[3 * H + i]);
        const float c = fg * c_in[i] + ig * gg;
        c_out[i] = c;
        h_out[i] = og * tanhf(c);
    }
}

/* Joint + argmax: src/kernels.metal:488-550 (joint_partial, argmax_reduce).
 *   r = max(enc + pred, 0);  score_n = W[n] . r + b[n];  best = argmax, lowest n on ties. */
int or_joint_argmax(const float *enc, const float *pred, const uint16_t *W, const float *bias, int V, int H,
                    float *best_value, float *logits) {
    float r[4096];
    for (int i = 0; i < H; ++i) { const float v = enc[i] + pred[i]; r[i] = v > 0.0f ? v : 0.0f; }
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int n = 0; n < V; ++n) {
        const uint16_t *w = W + (size_t)n * H;
        float acc = 0.0f;
        for (int k = 0; k < H; ++k) acc += r[k] * bf(w[k]);
        acc += bias[n];
        if (logits) logits[n] = acc;
        if (acc > bv || (acc == bv && n < bi)) { bv = acc; bi = n; }
    }
    if (best_value) *best_value = bv;
    return bi;
}

/* Relative positional table: src/model.c:286-306.  pe rows r = 0..2*Lmax-2 hold position
 * Lmax-1-r: pe[r][2i] = sin(pos * div_i), pe[r][2i+1] = cos(pos * div_i),
 * div_i = exp(2i * -(ln 10000 / D)), computed in double and rounded to f32; then
 * ptab = pe . wpos^T with the GEMM above. */
void or_ptab(const uint16_t *wpos, int D, int Lmax, float *out) {
    const int P = 2 * Lmax - 1;
    float *pe = malloc(sizeof(float) * (size_t)P * D);
    for (int r = 0; r < P; ++r) {
        const double pos = (double)(Lmax - 1 - r);
        for (int i = 0; i < D / 2; ++i) {
            const double div = exp((double)(2 * i) * -(log(10000.0) / (double)D));
            pe[(size_t)r * D + 2 * i] = (float)sin(pos * div);
            pe[(size_t)r * D + 2 * i + 1] = (float)cos(pos * div);
        }
    }
    or_gemm(pe, D, wpos, D, NULL, out, D, P, D, D, OR_ACT_NONE, 0, 1.0f);
    free(pe);
}
