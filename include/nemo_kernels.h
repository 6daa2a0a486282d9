/* nemoasr-mi355x kernel-level C ABI: the launchers of the streaming hot path.
 *
 * Every pointer argument is a device address (from gpu_buf_dptr); sizes are element counts.
 * Launches are ordered on the library's one stream and must sit between gpu_begin / gpu_end
 * (or inside a capture).  Return 0, or -1 with the message in gpu_last_error().
 *
 * These replace the reference's launchers and dispatch sites:
 *   nk_gemm             k_gemm                       src/model.c:70-99 (policy + dispatch)
 *   nk_layernorm        k_layernorm                  src/model.c:106-111
 *   nk_layernorm2       k_layernorm2                 src/model.c:100-105
 *   nk_copy / nk_fill   k_copy / k_fill              src/model.c:112-122
 *   nk_attention_rel    attention_rel dispatch       src/encoder.c:158-165
 *   nk_dwconv_ln_silu   dwconv_ln_silu dispatch      src/encoder.c:172-174
 *   nk_conv2d_c1_s2_relu, nk_dwconv2d_s2, nk_flatten_cf   subsampling dispatches src/encoder.c:120-142
 *   nk_compact          compact_caches               src/encoder.c:199-211 (one launch for all layers)
 *   nk_lstm_cell_rows   lstm_cell dispatch           src/decoder.c:71-73 (rows of many streams)
 *   nk_joint_in_rows + nk_gemm_argmax_rows (or nk_gemm + nk_argmax_rows)
 *                       joint + argmax dispatches    src/decoder.c:79-90 (rows of many streams)
 * The single stream's LSTM, joint and argmax run inside the device-resident greedy loop
 * (csrc/host/decoder.c, kernels dec_step / dec_pred / dec_joint), which has no per-kernel launcher.
 *
 * The GPU runtime has two faces.  This library's own host uses the one below: one launch call with
 * workgroup counts and one by-value argument struct of device pointers per kernel
 * (nemo-c_amd/csrc/kernel_params.h), device addresses from gpu_buf_dptr, explicit uploads and
 * downloads, hipGraph capture.  A host written against the reference's runtime (src/gpu.h:7-41:
 * buffers bound by index, GPU_BUF / GPU_BYTES arguments, dispatch by total threads, by groups or
 * by groups with function constants, host-addressable buffers) uses include/nemo_gpu.h and the
 * reference's parameter blocks in include/nemo_kernel_params.h; both faces share gpu_create,
 * gpu_buf_alloc, gpu_begin / gpu_end and the kernels.
 */
#ifndef NEMO_KERNELS_H
#define NEMO_KERNELS_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gpu gpu_t;
typedef struct gpu_buf gpu_buf_t;

/* ---- runtime (src/gpu.h:20-41) ---------------------------------------------------------------- */
gpu_t *gpu_create(const char *source, char *err, size_t errlen);
void gpu_destroy(gpu_t *g);
const char *gpu_device_name(gpu_t *g);
gpu_buf_t *gpu_buf_alloc(gpu_t *g, size_t bytes);
void gpu_buf_free(gpu_buf_t *b);
void *gpu_buf_dptr(gpu_buf_t *b);
size_t gpu_buf_len(gpu_buf_t *b);
int gpu_upload(gpu_t *g, void *dst_dev, const void *src, size_t n);
int gpu_download(gpu_t *g, void *dst, const void *src_dev, size_t n);
int gpu_begin(gpu_t *g);
int gpu_end(gpu_t *g, char *err, size_t errlen);
double gpu_last_ms(gpu_t *g);
const char *gpu_last_error(gpu_t *g);
int gpu_timing_set(gpu_t *g, const char *kernel, int max_launches);
/* mean duration (ms), launch count and summed algorithmic bytes of the timed launches */
int gpu_timing_collect(gpu_t *g, double *mean_ms, int *count, double *bytes);
uint64_t gpu_launch_count(const gpu_t *g);
/* hipGraph capture of the launches between capture_begin and capture_end (inside begin/end);
 * gpu_graph_launch replays it on the stream. */
typedef struct gpu_graph gpu_graph_t;
int gpu_capture_begin(gpu_t *g);
gpu_graph_t *gpu_capture_end(gpu_t *g);
int gpu_graph_launch(gpu_t *g, gpu_graph_t *gr);
void gpu_graph_free(gpu_graph_t *gr);

/* ---- GEMM ------------------------------------------------------------------------------------
 * C[m][n] (= or +=) alpha * act(sum_k A[m][k] W[n][k] + bias[n]); W bf16 [N][ldw]; act 0 none,
 * 1 SiLU, 2 ReLU, 3 GLU (output N/2 columns, a_j * sigmoid(b_{j+N/2})).  bias may be NULL.
 * Requirements: K % 32 == 0 (M > 4) or K % 8 == 0 (M <= 4); A, W 16-byte aligned; lda % 4 == 0;
 * ldw % 8 == 0. */
int nk_gemm(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
            float *C, uint32_t ldc, uint32_t M, uint32_t N, uint32_t K, int act, int accumulate, float alpha);
/* Same, with output row m written to row crow[m] of C (crow: device int array of M entries). */
int nk_gemm_rows(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                 float *C, uint32_t ldc, const int *crow, uint32_t M, uint32_t N, uint32_t K, int act, int accumulate,
                 float alpha);
/* Same, with a LayerNorm prologue on A when K is the row width (ln_mode 1: A' = LN(A; g1,b1);
 * 2: A' = LN(LN(A; g1,b1); g2,b2)).  ln_out (optional) receives LN(A; g1,b1).  For M <= 4 the
 * LayerNorm runs inside the GEMV; otherwise it is launched separately into `tmp` (M*K floats). */
int nk_gemm_ln(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias, float *C,
               uint32_t ldc, const int *crow, uint32_t M, uint32_t N, uint32_t K, int act, int accumulate, float alpha,
               int ln_mode, const float *g1, const float *b1, const float *g2, const float *b2, float *ln_out,
               float *tmp, float eps);
/* Row argmax of A W^T + bias over the first V columns without storing the scores: keys[m][p] is
 * the best packed (score, lowest column) key of column part p of row m (N/32 parts; the largest
 * key wins, and its low 32 bits hold 0xffffffff - column).  N % 64 == 0. */
int nk_gemm_argmax(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                   unsigned long long *keys, uint32_t keys_ld, uint32_t M, uint32_t N, uint32_t K, uint32_t V);
/* Same, computing only the first min(M, *mrows * mrows_mul) rows, a count read on the device (the
 * launch covers M rows; mrows NULL: all M). */
int nk_gemm_argmax_rows(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                        unsigned long long *keys, uint32_t keys_ld, uint32_t M, uint32_t N, uint32_t K, uint32_t V,
                        const int *mrows, uint32_t mrows_mul);
/* K split of the many-row residual updates (accumulate, no bias, no activation): -1 (default) by
 * tile count, 0 never, 1 always where K has more than one block.  All three give the same bits.
 * Returns the previous setting. */
int nk_gemm_ksplit(int mode);
/* Many-row tile: -1 (default) by tile count, else 0 128x128, 1 64x128, 2 64x64 where it divides
 * the output columns.  Returns the previous setting. */
int nk_gemm_mx_tile(int t);
/* Few-row residual updates (5..16 rows): 1 (default) splits K over four workgroups whose partial
 * rows are added in split order by a second launch, 0 keeps K in one workgroup (more wavefronts).
 * Returns the previous setting. */
int nk_gemm_fr_ksplit(int on);
/* Kernel selection: 0 automatic (by row count), 1 first-generation VALU GEMV (M <= 4),
 * 2 few-row MFMA (M <= 16), 3 many-row MFMA, 4 weight-streaming GEMV (M <= 4),
 * 5 first-generation many-row MFMA (register-staged).
 * Returns the previous setting. */
int nk_gemm_force(int kind);
/* Split rows: a row of K activations stored as K bf16 hi = RNE(a) then K bf16 lo = RNE(a - hi),
 * the operand form the many-row MFMA kernels multiply (hi and lo each against the bf16 weights).
 * A producer that writes them saves every consumer GEMM the split (its K loop then has no vector
 * work) and gives the same bits.  The batched encoder keeps the activations between its kernels in
 * this form.  nk_gemm_split: the many-row GEMM with exactly one of A (f32 rows) / A2 (split rows,
 * lda in bf16 elements >= 2K) and one of C (f32) / C2 (split rows of the nout outputs, ldc >= 2 nout;
 * no accumulate, row map or GLU). */
int nk_gemm_split(gpu_t *g, const float *A, const uint16_t *A2, uint32_t lda, const uint16_t *W, uint32_t ldw,
                  const float *bias, float *C, uint16_t *C2, uint32_t ldc, const int *crow, uint32_t M, uint32_t N,
                  uint32_t K, int act, int accumulate, float alpha);
/* A many-row residual update left pending: C += alpha * A W^T is computed as nparts partial rows
 * (the K blocks' sums) in the context's scratch and applied later, in block order, by the kernel
 * that reads C next: nk_layernorm2_split (the batched encoder: every residual update is followed by
 * a LayerNorm of the residual) or nk_resid_fold.  The same bits as nk_gemm_split's update.  The
 * scratch holds one pending update at a time. */
typedef struct {
    const float *parts;
    uint32_t nparts;
    float alpha;
} nk_resid_t;
int nk_gemm_resid(gpu_t *g, const float *A, const uint16_t *A2, uint32_t lda, const uint16_t *W, uint32_t ldw, float *C,
                  uint32_t ldc, uint32_t M, uint32_t N, uint32_t K, float alpha, nk_resid_t *pend);
int nk_resid_fold(gpu_t *g, float *C, uint32_t ldc, uint32_t M, uint32_t N, const nk_resid_t *pend);
/* A few-row residual update C += alpha * A W^T (no bias, activation or row map) whose kernel may
 * split K (the few-row MFMA kernel, 5-16 rows): its partial rows are returned in *pend and C is not
 * touched, for the next nk_gemm_ln_pend on C to add in share order; when the kernel does not split
 * K, C is updated and *pend is empty.  The partial rows live in the context's scratch, which holds
 * one pending update at a time. */
int nk_gemm_pend(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, float *C, uint32_t ldc,
                 uint32_t M, uint32_t N, uint32_t K, float alpha, nk_resid_t *pend);
/* nk_gemm_ln on A with a pending residual update (pend, may be NULL or empty) applied first:
 * Xf = A + alpha * (((0 + p0) + p1) + ...) (the bits of nk_resid_fold), and the GEMM's LayerNorm
 * prologue reads Xf.  Xf (rows of lda floats, not A) receives the updated rows: the residual
 * stream after the update; it may be NULL when they are not needed (the LayerNorm output carries
 * the stream on) and the kernel folds in its prologue.  The weight-streaming GEMV (M <= 4,
 * K <= 1024) and the few-row MFMA kernel (M <= 16, K == 1024, at most 4 parts) apply the update in
 * their prologue, no extra launch; other kernels get a copy into Xf and an nk_resid_fold first.
 * Parts are [nparts][M][K] (part stride M * K). */
int nk_gemm_ln_pend(gpu_t *g, const float *A, uint32_t lda, const uint16_t *W, uint32_t ldw, const float *bias,
                    float *C, uint32_t ldc, const int *crow, uint32_t M, uint32_t N, uint32_t K, int act, int accumulate,
                    float alpha, int ln_mode, const float *g1, const float *b1, const float *g2, const float *b2,
                    float *ln_out, float *tmp, float eps, const nk_resid_t *pend, float *Xf);
/* nk_gemm_split without any allocation.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The split-K partial sums live in a static device array
 * of NK_NOALLOC_WS_FLOATS floats per GPU (held until the process ends): the partial rows of a
 * residual update (at most NK_NOALLOC_WS_FLOATS = parts x M x N floats; a larger one is refused with
 * an error before any launch).  Every call on a GPU shares its array and overwrites what the last
 * call left there (nothing in it needs to start at zero): calls that overlap on one GPU race.  Same
 * arguments and results (bit for bit) as nk_gemm_split. */
#define NK_NOALLOC_WS_FLOATS (4u << 20)
int nk_gemm_split_noalloc(gpu_t *g, const float *A, const uint16_t *A2, uint32_t lda, const uint16_t *W, uint32_t ldw,
                          const float *bias, float *C, uint16_t *C2, uint32_t ldc, const int *crow, uint32_t M,
                          uint32_t N, uint32_t K, int act, int accumulate, float alpha);
/* LayerNorm of M rows (D <= 1024, one wavefront per row) whose GEMM-feeding output goes to Ys as
 * split rows (row stride 2D): the single LayerNorm (g2 NULL) writes only Ys; the pair writes
 * LN(X; g1, b1) to Y1 (f32) and LN(Y1; g2, b2) to Ys.  With pend (from nk_gemm_resid, may be NULL)
 * the pending residual update is applied to X first and X is written back. */
int nk_layernorm2_split(gpu_t *g, float *X, const nk_resid_t *pend, const float *g1, const float *b1, const float *g2,
                        const float *b2, float *Y1, uint16_t *Ys, uint32_t M, uint32_t D, float eps);
/* Name of the kernel nk_gemm would launch for these shapes (for profiling and tests). */
const char *nk_gemm_kernel_name(uint32_t M, uint32_t N, uint32_t K, int act);

/* ---- norms, attention, convolution ----------------------------------------------------------- */
int nk_layernorm(gpu_t *g, const float *X, const float *gamma, const float *beta, float *Y, uint32_t M, uint32_t D,
                 float eps);
int nk_layernorm2(gpu_t *g, const float *X, const float *g1, const float *b1, const float *g2, const float *b2,
                  float *Y1, float *Y2, uint32_t M, uint32_t D, float eps);
int nk_attention_rel(gpu_t *g, const float *Q, uint32_t ldq, const float *K, const float *V, uint32_t ldk,
                     const float *P, const float *bias_u, const float *bias_v, float *O, uint32_t c, uint32_t L,
                     uint32_t Lmax, uint32_t H, uint32_t dh, uint32_t D, float scale);
int nk_dwconv_ln_silu(gpu_t *g, const float *din, const float *W, const float *gamma, const float *beta, float *Y,
                      uint32_t c, uint32_t D, uint32_t taps, float eps);
/* Variants that take the cache position from a device chunk descriptor (int[4 + 16]:
 * pos, cache_len, L, c, then pos + i per row) so a captured graph replays at any position.
 * kv: K/V cache base with rows of `ld` floats (q | k | v); din_base: conv cache base. */
int nk_attention_rel_desc(gpu_t *g, const float *kv, uint32_t ld, const int *desc, const float *P, const float *bias_u,
                          const float *bias_v, float *O, uint32_t c, uint32_t Lmax, uint32_t H, uint32_t dh, uint32_t D,
                          float scale);
int nk_dwconv_ln_silu_desc(gpu_t *g, const float *din_base, const int *desc, const float *W, const float *gamma,
                           const float *beta, float *Y, uint32_t c, uint32_t D, uint32_t taps, float eps);
/* Launch fusions of the single-stream chunk (descriptor window, c <= 4 rows):
 * C[i] += alpha * attention_i . Wo^T for the c rows (attention as nk_attention_rel_desc); Wo [D][ldw]
 * bf16, D % 128 == 0.  Each head's share of the product is written as a partial row and the H rows
 * are added in head order: by an nk_resid_fold launch (nk_attention_out_desc), or left pending in
 * *pend for the next LayerNorm-fused GEMM (nk_attention_out_desc_pend + nk_gemm_ln_pend).
 * Replaces nk_attention_rel_desc + nk_gemm(O, Wo, accumulate). */
int nk_attention_out_desc(gpu_t *g, const float *kv, uint32_t ld, const int *desc, const float *P, const float *bias_u,
                          const float *bias_v, uint32_t c, uint32_t Lmax, uint32_t H, uint32_t dh, uint32_t D,
                          float scale, const uint16_t *Wo, uint32_t ldw, float *C, uint32_t ldc, float alpha);
int nk_attention_out_desc_pend(gpu_t *g, const float *kv, uint32_t ld, const int *desc, const float *P,
                               const float *bias_u, const float *bias_v, uint32_t c, uint32_t Lmax, uint32_t H,
                               uint32_t dh, uint32_t D, float scale, const uint16_t *Wo, uint32_t ldw, float alpha,
                               nk_resid_t *pend);
/* C[i][n] (= or +=) alpha * sum_k y_i[k] W[n][k] with y = SiLU(LN(dwconv(din))) of the c <= 2 rows
 * (as nk_dwconv_ln_silu_desc; 9 taps, D <= 1024, D % 8 == 0).  Bit-identical to that launch
 * followed by nk_gemm(y, W, no bias, no activation). */
int nk_dwconv_pw_desc(gpu_t *g, const float *din_base, const int *desc, const float *dw_w, const float *gamma,
                      const float *beta, float eps, const uint16_t *W, uint32_t ldw, float *C, uint32_t ldc, uint32_t c,
                      uint32_t D, uint32_t N, int accumulate, float alpha);
/* Shapes of the fused kernels: output columns per wavefront of the attention fusion (4, 8 or 16) and
 * weight rows per wavefront of the conv fusion (1, 2 or 4).  0 leaves a setting; returns the
 * previous settings as attn * 16 + dw. */
int nk_fuse_shape(int attn_cpw, int dw_nc);
/* Batched streams: output row m is described by rows[4m .. 4m+3] = { cache row of the chunk row,
 * its index i in its stream's chunk, that chunk's rows c, the stream's cached rows } (device). */
int nk_attention_rel_rows(gpu_t *g, const float *kv, uint32_t ld, const int *rows, uint32_t M, const float *P,
                          const float *bias_u, const float *bias_v, float *O, uint32_t Lmax, uint32_t H, uint32_t dh,
                          uint32_t D, float scale);
/* Whole chunks of batched streams: chunks[4k..4k+3] = { cache row of chunk k's first row, its
 * first output row, its rows c (<= 16), its stream's cached rows } with cached + c <= 80. */
int nk_attention_rel_chunks(gpu_t *g, const float *kv, uint32_t ld, const int *chunks, uint32_t nchunks, const float *P,
                            const float *bias_u, const float *bias_v, float *O, uint32_t Lmax, uint32_t H, uint32_t dh,
                            uint32_t D, float scale);
/* Same, output as split rows (row stride 2D) to Os. */
int nk_attention_rel_chunks_split(gpu_t *g, const float *kv, uint32_t ld, const int *chunks, uint32_t nchunks,
                                  const float *P, const float *bias_u, const float *bias_v, uint16_t *Os, uint32_t Lmax,
                                  uint32_t H, uint32_t dh, uint32_t D, float scale);
int nk_dwconv_ln_silu_rows(gpu_t *g, const float *din_base, const int *rows, uint32_t M, const float *W,
                           const float *gamma, const float *beta, float *Y, uint32_t D, uint32_t taps, float eps);
/* Same, output as split rows (row stride 2D) to Ys (Y NULL) or f32 to Y (Ys NULL). */
int nk_dwconv_ln_silu_rows_split(gpu_t *g, const float *din_base, const int *rows, uint32_t M, const float *W,
                                 const float *gamma, const float *beta, float *Y, uint16_t *Ys, uint32_t D, uint32_t taps,
                                 float eps);
int nk_conv2d_c1_s2_relu(gpu_t *g, const float *X, const float *W, const float *bias, float *Y, uint32_t T,
                         uint32_t F, uint32_t T1, uint32_t F1, uint32_t C);
int nk_dwconv2d_s2(gpu_t *g, const float *X, const float *W, const float *bias, float *Y, uint32_t T, uint32_t F,
                   uint32_t T1, uint32_t F1, uint32_t C);
int nk_flatten_cf(gpu_t *g, const float *X, float *Y, uint32_t T, uint32_t F, uint32_t C);
/* The same three over `batch` windows of one size stored back to back (batched streams). */
int nk_conv2d_c1_s2_relu_b(gpu_t *g, const float *X, const float *W, const float *bias, float *Y, uint32_t T,
                           uint32_t F, uint32_t T1, uint32_t F1, uint32_t C, uint32_t batch);
int nk_dwconv2d_s2_b(gpu_t *g, const float *X, const float *W, const float *bias, float *Y, uint32_t T, uint32_t F,
                     uint32_t T1, uint32_t F1, uint32_t C, uint32_t batch);
int nk_flatten_cf_b(gpu_t *g, const float *X, float *Y, uint32_t T, uint32_t F, uint32_t C, uint32_t batch);
/* conv 0 + ReLU and conv 2 in one pass (src/encoder.c:124-130, kernels.metal:411-454): X [T][F]
   -> Y [T2][F2][C] per window, equal to nk_conv2d_c1_s2_relu_b then nk_dwconv2d_s2_b without
   conv 0's [T1][F1][C] output.  F <= 256. */
int nk_conv2d_c1_dw_s2_b(gpu_t *g, const float *X, const float *W0, const float *b0, const float *W2,
                         const float *b2, float *Y, uint32_t T, uint32_t F, uint32_t T1, uint32_t F1, uint32_t T2,
                         uint32_t F2, uint32_t C, uint32_t batch);
/* dst[m] = src[map[m]] for m < rows (cols floats per row) */
int nk_gather_rows(gpu_t *g, const float *src, uint32_t src_ld, const int *map, float *dst, uint32_t dst_ld,
                   uint32_t rows, uint32_t cols);
/* dst row map[m] = src row m, m < rows (distinct targets). */
int nk_scatter_rows(gpu_t *g, const float *src, uint32_t src_ld, const int *map, float *dst, uint32_t dst_ld,
                    uint32_t rows, uint32_t cols);
/* Log-mel rows of F frames (all pointers device): frame f reads the 512 pre-emphasised samples
 * span[tab[2f] ..] and writes row tab[2f+1] of out (rows of 128 floats); tables as the host front
 * end's (window [512], filterbank [128][257], filter bin ranges, double twiddles [256], bit reversal
 * [512]).  The power spectrum equals the host front end's (same double arithmetic, no contraction);
 * the log may differ by rounding. */
int nk_mel_frames(gpu_t *g, const float *span, const int *tab, uint32_t F, const float *win, const float *fb,
                  const int *fb_lo, const int *fb_hi, const double *tw_re, const double *tw_im, const uint16_t *rev,
                  float *out);
int nk_copy(gpu_t *g, const float *src, float *dst, uint32_t n);
int nk_copy2d(gpu_t *g, const float *src, uint32_t src_ld, float *dst, uint32_t dst_ld, uint32_t rows, uint32_t cols);
int nk_fill(gpu_t *g, float *dst, uint32_t n, float value);
int nk_compact(gpu_t *g, float *base, uint64_t stride, uint32_t nbuf, uint32_t rows, uint32_t cols,
               uint32_t src_row, uint32_t dst_row);

/* ---- RNNT decoder ------------------------------------------------------------------------------ */
/* Batched decoder pieces (rows of many streams; see kernel_params.h for the layouts):
 * LSTM input rows [x | h], the LSTM cell on rows, joint input rows relu(enc + pred), row argmax. */
int nk_lstm_input_rows(gpu_t *g, const uint16_t *embed, const int *tok, const float *xsrc, const float *hc,
                       const int *hrow, float *A, uint32_t n, uint32_t P, uint32_t blank);
int nk_lstm_cell_rows(gpu_t *g, const float *gates, float *hc, const int *crow_in, const int *crow_out,
                      const int *hrow_out, float *hout, uint32_t n, uint32_t P);
int nk_joint_in_rows(gpu_t *g, const float *enc, const float *pred, const int *erow, const int *prow, float *jin,
                     uint32_t rows, uint32_t J);
int nk_argmax_rows(gpu_t *g, const float *logits, uint32_t ld, uint32_t rows, uint32_t V, int *out);

/* ---- dispatches of the reference that this library's own path fuses away -------------------------
 * Served for hosts driving include/nemo_gpu.h (reference kernels glu, lstm_cell, joint_partial,
 * argmax_reduce: src/kernels.metal:349-356, :474-550; dispatch sites src/decoder.c:71-73, :79-90). */
int nk_glu(gpu_t *g, const float *X, float *Y, uint32_t M, uint32_t D);
int nk_lstm_cell(gpu_t *g, const float *gates, const float *c_in, float *c_out, float *h_out, uint32_t H);
/* per row r < rows: slot s < 8 groups keeps the best of n = s, s + 8 groups, ... < V of
 * W[n] . relu(enc[enc_row + r] + pred) + bias[n] in part_v / part_i[r][s] */
int nk_joint_partial(gpu_t *g, const float *enc, const float *pred, const uint16_t *W, const float *bias,
                     float *part_v, int *part_i, uint32_t V, uint32_t H, uint32_t enc_row, uint32_t enc_ld,
                     uint32_t groups, uint32_t rows);
/* out[2 r], out[2 r + 1] = index and value bits of the best of row r's n partials (lowest index on ties) */
int nk_argmax_reduce(gpu_t *g, const float *part_v, const int *part_i, int *out, uint32_t n, uint32_t rows);

#ifdef __cplusplus
}
#endif
#endif
