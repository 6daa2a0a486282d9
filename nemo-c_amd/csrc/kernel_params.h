/* Kernel argument blocks shared by the C host and the gfx950 HIP kernels.
 *
 * Every kernel takes exactly one of these structs by value; the host passes its bytes through
 * hipModuleLaunchKernel's argument buffer, so the struct layout is the kernel ABI.  Pointers are
 * device addresses.  This is a re-design of the reference's Metal parameter blocks
 * (src/kernel_params.h:22-32), which carried only scalars, with the buffers bound separately at
 * argument index i (src/gpu.m:98-101).  Here each struct carries the scalars of the reference's
 * block (same meaning) and the device pointers of its buffers:
 *   GemmParams   -> NkGemmArgs (+ row map, split-K scratch, LayerNorm prologue, argmax keys)
 *   LnParams     -> NkLnArgs (both outputs of the paired LayerNorm in one launch)
 *   AttnParams   -> NkAttnArgs (+ the chunk descriptor or per-row stream table), NkAttnChunksArgs,
 *                   NkAttnOutArgs (attention fused with the output projection)
 *   DwParams     -> NkDwArgs;  Conv2dParams / FlatParams -> the subsampling structs below
 *   GluParams    -> none (GLU is the GEMM epilogue, act 3, as in the reference's GEMMs)
 *   LstmParams, JointParams, CountParams, FillParams -> the decoder and copy structs below
 */
#ifndef NEMO_KERNEL_PARAMS_H
#define NEMO_KERNEL_PARAMS_H
#ifdef __HIPCC__
#include <hip/hip_runtime.h>
typedef unsigned int u32;
typedef unsigned short u16;
#else
#include <stdint.h>
typedef uint32_t u32;
typedef uint16_t u16;
#endif

/* Row and chunk limits.  One wavefront is 64 lanes on CDNA4. */
#define NK_WAVE 64
#define NK_MX_KS_SPLIT 64       /* K step of the many-row kernels on split-row A (K % this == 0)  */
#define NK_FEW_ROWS 16          /* GEMMs with M <= 16 use the weight-streaming kernels            */
#define NK_ATT_MAX_L 128        /* attention window limit (reference ATT_MAX_L 80; 56 + 16 + 2)    */
#define NK_DEC_MAX_BATCH 16     /* joint rows per decoder round trip (reference DEC_MAX_BATCH)    */
#define NK_JOINT_MAX_H 1024     /* joint hidden size limit (16 floats per lane of a wavefront)     */
#define NK_CACHE_EPOCH_CHUNKS 8 /* K/V and conv caches compacted once per this many chunks         */
#define NK_LN_THREADS 256
#define NK_ROW_MAX 4096         /* row width limit of the per-row kernels (4 float4 per thread)    */
#define NK_CONV_TAPS 9          /* causal depthwise conv kernel size                               */
#define NK_FR_MAX_KC 1024       /* few-row MFMA GEMM: K columns of A staged per workgroup          */

enum { NK_ACT_NONE = 0, NK_ACT_SILU = 1, NK_ACT_RELU = 2, NK_ACT_GLU = 3 };

/* C[row(m)][n] (= or +=) alpha * act(sum_k A[m][k] * W[n][k] + bias[n]); act GLU: N is the
 * weight height and the output has N/2 columns, column j = a_j * sigmoid(b_{j+N/2}).
 * crow, when set, maps output row m to row crow[m] of C (scatter into a cache). */
typedef struct {
    const float *A;
    const u16 *W;
    const float *bias;
    float *C;
    const int *crow;
    float *ws;      /* split-K residual updates: partial rows [split][M][nout], folded by resid_fold */
    u32 M, N, K, lda, ldw, ldc;
    u32 act, accumulate, splits, group_m; /* group_m: row tiles per group of the many-row tile order */
    float alpha;
    /* many-row residual updates: K is summed in kblocks equal blocks, each block from zero, the
     * block sums added in order; splits is 1 or kblocks (one block per workgroup) and gives the same
     * bits either way; the sums go to partial rows at ws (NkFoldArgs) */
    u32 kblocks;
    /* LayerNorm prologue on A (weight-streaming GEMV): ln_mode 0 none, 1 LN(g1,b1),
     * 2 LN(LN(g1,b1); g2,b2); ln_out (optional) receives LN(A; g1,b1), rows of lda floats */
    const float *ln_g1, *ln_b1, *ln_g2, *ln_b2;
    float *ln_out;
    u32 ln_mode;
    float ln_eps;
    /* argmax epilogue of the many-row kernel (joint scores): per row, the best (score, lowest
     * column) of each wavefront's columns < keys_n as a packed key, keys[row * keys_ld + part] */
    unsigned long long *keys;
    u32 keys_ld, keys_n;
    /* many-row kernel: with mrows set, only the first min(M, *mrows * mrows_mul) rows are computed
     * (a row count known on the device only; the grid covers M) */
    const int *mrows;
    u32 mrows_mul, pad2;
    /* split activations (many-row kernels): a row of K values is stored as K bf16 hi = RNE(a) then
     * K bf16 lo = RNE(a - hi), lda / ldc in bf16 elements.  A2 set: A is read from A2 (split by its
     * producer, the same hi / lo the kernel would form itself); C2 set: the outputs are written as
     * split rows of nout values to C2 instead of f32 to C (no accumulate, no row map). */
    const u16 *A2;
    u16 *C2;
    /* weight-streaming GEMV with a LayerNorm prologue: with fold set, a pending residual update is
     * applied to A first, x = A + fold_alpha * (((0 + P[0]) + P[1]) + ...) (fold_n parts of M rows of
     * K floats, part stride M * K), by every workgroup into LDS; workgroup 0 also writes x to
     * fold_out (rows of lda floats), the residual stream after the update */
    const float *fold;
    float *fold_out;
    u32 fold_n;
    float fold_alpha;
} NkGemmArgs;

typedef struct {
    const float *X;
    const float *g1, *b1, *g2, *b2;
    float *Y1, *Y2; /* Y2 only for the paired LayerNorm */
    u32 M, D;
    float eps;
    u32 pad;
    /* set: the LayerNorm that feeds the next GEMM (Y2 when paired, else Y1) is written as split
     * rows (D bf16 hi, D bf16 lo; row stride 2D) here instead (see NkGemmArgs.A2) */
    u16 *Ys;
    /* set: a pending residual update is applied to X first (and X written back):
     * X[r] = X[r] + palpha * (((0 + P[0][r]) + P[1][r]) + ...), nparts rows of D floats per part
     * (part stride M * D) */
    const float *P;
    u32 nparts;
    float palpha;
} NkLnArgs;

/* C[r][n] = C[r][n] + alpha * (((0 + P[0][r][n]) + P[1][r][n]) + ...): a pending residual update
 * of the many-row GEMM (parts of M rows of N floats, part stride M * N) applied to C. */
typedef struct {
    float *C;
    const float *P;
    u32 M, N, ldc, nparts;
    float alpha;
    u32 pad;
} NkFoldArgs;

/* Chunk descriptor in device memory, written by the host before each chunk so that a captured
 * graph can replay a chunk at any cache position:
 *   [0] pos        first cache row of this chunk in the per-layer K/V and conv buffers
 *   [1] cache_len  cached attention rows in front of pos
 *   [2] L          attention window = cache_len + c
 *   [3] c          rows of the chunk
 *   [4 + i]        pos + i, the cache row of chunk row i (GEMM output row map)
 *   [4 + 16]       epoch, a per-chunk number that never repeats on consecutive chunks (the
 *                  tag base of the single-row chain's hand-offs) */
#define NK_DESC_POS 0
#define NK_DESC_CACHE 1
#define NK_DESC_L 2
#define NK_DESC_C 3
#define NK_DESC_ROWS 4
#define NK_DESC_EPOCH (NK_DESC_ROWS + NK_FEW_ROWS)
#define NK_DESC_INTS (NK_DESC_EPOCH + 1)

/* Relative-position attention for one chunk of one stream.
 * Q: [c][ldq]; K, V: [L][ldk] (the window: cached rows then the chunk's rows);
 * P: [2*Lmax-1][D]; O: [c][D].
 * With desc set, Q/K/V are the cache bases (rows of ldq = ldk floats) and the window comes from
 * the descriptor: Q row pos + i, K/V rows pos - cache_len .. pos + c - 1, L = cache_len + c.
 * With rows set (batched streams), Q/K/V are the cache bases and output row m is described by
 * rows[4m .. 4m+3] = { cache row of the query, its index i in the stream's chunk, the chunk's
 * rows c, the stream's cached rows }; the window is the cache_len + c rows ending with the chunk. */
typedef struct {
    const float *Q, *K, *V, *P, *bu, *bv;
    float *O;
    const int *desc;
    const int *rows;
    u32 c, L, Lmax, H, dh, D, ldq, ldk;
    float scale;
    u32 pad;
} NkAttnArgs;

/* Relative-position attention of whole chunks (batched streams): one workgroup per (head, chunk)
 * stages the chunk's K/V window and position rows in LDS once for all its query rows.
 * chunks[4k..4k+3] = { cache row of the chunk's first row, its first output row, rows c, cached
 * rows }; L = cached + c <= NK_ATTC_MAX_L, c <= NK_ATTC_MAX_C. */
#define NK_ATTC_MAX_L 80
#define NK_ATTC_MAX_C 16
typedef struct {
    const float *kv; /* q | k | v rows of ld floats */
    const float *P, *bu, *bv;
    float *O;
    const int *chunks;
    u32 H, dh, D, ld, Lmax;
    float scale;
    u16 *Os; /* set: O written as split rows (row stride 2D) here instead */
} NkAttnChunkArgs;

/* Causal depthwise conv + LN + SiLU. din: [(taps-1) + c][D]; W: [D][taps].
 * With desc set, din is the conv cache base and the rows start at pos - (taps-1).
 * With rows set (batched streams, same table as the attention), din is the conv cache base and
 * output row m convolves cache rows rows[4m] - (taps-1) .. rows[4m]. */
typedef struct {
    const float *din, *W, *g, *b;
    float *Y;
    const int *desc;
    const int *rows;
    u32 c, D, taps;
    float eps;
    u16 *Ys; /* set: Y written as split rows (row stride 2D) here instead */
} NkDwArgs;

/* Attention fused with its output projection (single stream, window from the descriptor):
 * C[row] += alpha * O[row] . Wo^T with O the attention output of `at` (at.O unused); Wo [D][ldw]. */
typedef struct {
    NkAttnArgs at;
    const u16 *Wo;
    float *C;
    float *ws;     /* per-head partial rows [head][row][D], folded into C by resid_fold */
    u32 ldw, ldc;
    float alpha;
    u32 pad;
} NkAttnOutArgs;

/* Depthwise conv + LN + SiLU (d, window from the descriptor; d.Y unused) as the prologue of the
 * GEMV g that consumes it (g.A unused, g.K = d.D). */
typedef struct {
    NkGemmArgs g;
    NkDwArgs d;
} NkGemvDwArgs;

/* Batched log-mel front end: frame f reads span[tab[2f] .. + 512) (pre-emphasised samples, edge
 * reflection already applied) and writes log-mel row tab[2f+1] of out ([*][128]).  Tables: window
 * [512], filterbank [128][257] with each filter's nonzero bins [fb_lo, fb_hi), twiddles
 * e^{-2 pi i k/512} for k < 256 (double), bit reversal [512]. */
typedef struct {
    const float *span;
    const int *tab;
    const float *win, *fb;
    const int *fb_lo, *fb_hi;
    const double *tw_re, *tw_im;
    const unsigned short *rev;
    float *out;
    u32 F, pad;
} NkMelArgs;

/* Subsampling convs. X [T][F] (conv 0) or [T][F][C]; Y [T1][F1][C].  grid.x = T1 * ceil(F1 / fb):
 * a workgroup computes fb consecutive output columns of one output row, its threads the channels;
 * grid.y runs over a batch of windows of the same size, xs / ys floats apart. */
typedef struct {
    const float *X, *W, *bias;
    float *Y;
    u32 T, F, T1, F1, C, fb;
    u32 xs, ys;
} NkConvArgs;

/* conv 0 and conv 2 of the subsampling in one pass: X [T][F] -> Y [T2][F2][C], conv 0's
 * [T1][F1][C] output never stored.  grid.x = T2 * ceil(F2 / fb), grid.y = windows (xs / ys floats
 * apart); F <= NK_CONV02_FMAX. */
#define NK_CONV02_FMAX 256
typedef struct {
    const float *X, *W0, *b0, *W2, *b2;
    float *Y;
    u32 T, F, T1, F1, T2, F2, C, fb;
    u32 xs, ys;
} NkConv02Args;

typedef struct {
    const float *X;
    float *Y;
    u32 T, F, C, pad;
} NkFlatArgs;

typedef struct {
    const float *src;
    float *dst;
    u32 n, pad;
} NkCopyArgs;

typedef struct {
    float *dst;
    u32 n;
    float value;
} NkFillArgs;

/* rows x cols floats from src (row stride src_ld) to dst (row stride dst_ld) */
typedef struct {
    const float *src;
    float *dst;
    u32 rows, cols, src_ld, dst_ld;
} NkCopy2dArgs;

/* Moves `rows` rows of `cols` floats from row src_row to row dst_row in each of `nbuf`
 * buffers laid out `stride` floats apart (the per-layer caches). */
typedef struct {
    float *base;
    unsigned long long stride;
    u32 nbuf, rows, cols, src_row, dst_row, pad;
} NkCompactArgs;

/* ---- device-resident greedy RNNT loop -------------------------------------------------------- */
#define NK_DEC_MAX_TOKENS 256 /* tokens per chunk: at most 16 frames x max_symbols                  */
#define NK_DEC_GROUPS 40      /* joint workgroups per frame row, 32 vocabulary rows each (V <= 1280) */

/* State of the loop, kept on the device across chunks.  Two copies alternate by iteration parity:
 * iteration j reads copy j%2 and writes copy (j+1)%2.  The first six fields are reset by the host at
 * the start of every chunk. */
typedef struct {
    int frames, t, symbols, n_out, pending, joints; /* chunk fields                                 */
    int pred_valid, last_token, cur, done, need_pred; /* persistent: cur = committed LSTM state slot */
    int pad[5];
} NkDecState;

typedef struct {
    NkDecState *st;           /* [2]                                                              */
    unsigned long long *part; /* [2][NK_DEC_MAX_BATCH][NK_DEC_GROUPS] packed (score, index) keys   */
    int *tokens;              /* [NK_DEC_MAX_TOKENS] tokens emitted in the current chunk             */
    const float *enc;         /* joint.enc rows of the chunk, [frames][enc_ld]                       */
    const u16 *embed;         /* prediction embedding [blank + 1][P]                                 */
    const u16 *wx0, *wh0, *wx1, *wh1; /* LSTM [4P][P], gate order i, f, g, o                         */
    const float *b0, *b1;     /* [4P]                                                              */
    float *hc;                /* LSTM state [2 slots][h0, h1, c0, c1][P]                            */
    const u16 *wjp;           /* joint.pred [J][P]                                                  */
    const float *bjp;
    float *pred;              /* [J]                                                               */
    const u16 *wout;          /* joint output [V][J]                                                */
    const float *bout;        /* [V]                                                               */
    float *tx;                /* [blank + 1][4P] layer-0 input gates Wx0 . embed(v) + b0 (zero input
                                 for the blank row): read by dec_step, written by dec_tx_build     */
    float *pre0;              /* [2 slots][4P] Wh0 . h0 of each slot's layer-0 state (gate-major)   */
    u32 P, J, V, blank, max_symbols, parity, enc_ld, decide_only;
} NkDecArgs;

/* ---- batched streams ---------------------------------------------------------------------- */
/* dst[m][0:cols] = src[map[m]][0:cols] for m < rows */
typedef struct {
    const float *src;
    float *dst;
    const int *map;
    u32 rows, cols, src_ld, dst_ld;
} NkGatherArgs;

/* LSTM input rows of the batched decoder: A[n] = [x_n | h_n] (2P floats).  x_n is the bf16
 * embedding row tok[n] widened (zeros for blank) when tok is set, else row n of xsrc; h_n is
 * row hrow[n] of the state array hc (rows of P floats). */
typedef struct {
    const u16 *embed;
    const int *tok;
    const float *xsrc;
    const float *hc;
    const int *hrow;
    float *A;
    u32 n, P, blank, pad;
} NkLstmInArgs;

/* LSTM cell on rows: gates [n][4P] (order i, f, g, o); c = hc[crow_in[n]]; writes c' to
 * hc[crow_out[n]], h' to hc[hrow_out[n]] and to hout[n] (contiguous, for the next layer). */
typedef struct {
    const float *gates;
    float *hc;
    const int *crow_in, *crow_out, *hrow_out;
    float *hout;
    u32 n, P;
} NkLstmRowsArgs;

/* joint input rows: jin[r] = relu(enc[erow[r]] + pred[prow[r]]) (J floats) */
typedef struct {
    const float *enc, *pred;
    const int *erow, *prow;
    float *jin;
    u32 rows, J;
} NkJointInArgs;

/* per-row argmax over the first V of ld logits, lowest index on ties:
 * out[2r] = index, out[2r+1] = value bits */
typedef struct {
    const float *logits;
    int *out;
    u32 rows, V, ld, pad;
} NkArgmaxRowsArgs;

/* Device-resident greedy loop of many streams (kernels/nk_bdec.hip).  Per-stream state; the
 * first eight fields follow the reference's decoder (src/decoder.c:14-23, :92-127): frames of the
 * current chunk, next frame t, symbols emitted at frame t, whether the prediction is valid, the
 * committed LSTM slot set, the last token; then tokens emitted in this chunk, the chunk's first
 * joint.enc row, and whether this step recomputes the prediction. */
typedef struct {
    int frames, t, symbols, pred_valid, cur, last_token, n_out, erow0;
    int need, slot, joints, pad[5]; /* joints: decisions taken in the current chunk */
} NkBDecStream;

/* One row of a decoder step: the streams still inside their chunk, in the order their previous
 * decision (or the chunk's setup) appended them; the step's GEMM rows and joint-input rows follow
 * this order.  need: the prediction is recomputed (LSTM and joint.pred rows are used). */
typedef struct {
    int s, need, cur, tok, t, lim, erow, pad;
} NkBDecRow;

typedef struct {
    NkBDecStream *st;      /* [S]                                                        */
    const unsigned long long *keys; /* [S*W][nkeys] joint argmax partials (packed keys)     */
    u32 nkeys, pad2;
    const int *setup;      /* [S][2] frames, first joint.enc row of a new chunk (setup)    */
    int *tokens;           /* [S][tok_ld] tokens emitted in the current chunk              */
    const float *enc;      /* joint.enc rows [*][J]                                        */
    const float *tx;       /* [blank + 1][4P] embed . Wx0^T + b0, rows interleaved by unit */
    float *hc;             /* [S][2 slot sets][h0, c0, h1, c1][P]                          */
    float *pre0;           /* [S][2 slot sets][4P] Wh0 . h0 of each slot set's h0, interleaved
                              by unit like tx                                               */
    const u16 *wh0;        /* Wh0 rows interleaved by unit, row stride wh0_ld               */
    u32 wh0_ld, pad3;
    float *A1;             /* [S][2P] layer-1 input [h0' | h1], by row                     */
    float *hout;           /* [S][P] new layer-1 state, input of joint.pred, by row        */
    float *pred;           /* [S][J] current prediction                                    */
    float *jin;            /* [S*W][J] joint inputs relu(enc + pred), rows slot * W + k    */
    NkBDecRow *rows;       /* [S] the step's rows                                          */
    int *cnt;              /* [2] row counts by step parity: step par reads cnt[par ^ 1]    */
    u32 S, W, P, J, blank, max_symbols, tok_ld, par;
} NkBDecArgs;

/* Kernels of the reference-shaped dispatch (include/nemo_gpu.h) with no counterpart in this
 * library's own path: the standalone GLU, a one-vector LSTM cell with separate input and output
 * state buffers, and the two-stage joint argmax with the reference's partial-best layout
 * (src/kernels.metal:349-356, :474-550). */
typedef struct {
    const float *X; /* [M][2D]: value half then gate half */
    float *Y;       /* [M][D] */
    u32 M, D;
} NkGluArgs;
typedef struct {
    const float *gates; /* [4H] i, f, g, o */
    const float *c_in;
    float *c_out, *h_out;
    u32 H;
} NkLstmCellArgs;
typedef struct {
    const float *enc;   /* joint.enc rows; row enc_row + r of stride enc_ld */
    const float *pred;  /* [H] */
    const u16 *W;       /* [V][H] bf16 */
    const float *bias;  /* [V] */
    float *part_v;      /* [rows][groups * 8] best score per slot */
    int *part_i;        /* [rows][groups * 8] its index (lowest on ties) */
    u32 V, H, enc_row, enc_ld, groups;
} NkJointPartArgs;
typedef struct {
    const float *part_v;
    const int *part_i;
    int *out; /* [rows][2]: index, value bits */
    u32 n;    /* partials per row */
} NkArgmaxPartArgs;

/* The batched loop's GEMM kernels (bdec_lstm1_*, bdec_pred_*): the GEMM operands and the loop
 * state in one argument block, like every other kernel (one by-value struct per kernel). */
typedef struct {
    NkGemmArgs g;
    NkBDecArgs d;
} NkBDecGemmArgs;

/* Persistent encoder chain for one-row chunks (kernels/nk_chain.hip): all conformer blocks of a
 * chunk in one launch of NK_CHAIN_G resident workgroups that hand each block's intermediate rows
 * to one another through tagged entries, while one wavefront per workgroup streams that
 * workgroup's weight slices into an LDS ring.  Built for d_model 1024, d_ff 4096, 8 heads of 128
 * and a 9-tap depthwise conv; the host uses the per-kernel graph for any other shape. */
#define NK_CHAIN_G 256       /* workgroups, one per CU; every one must be resident at once      */
#define NK_CHAIN_THREADS 448 /* 4 compute, 2 hand-off and 1 weight-streaming wavefronts          */
#define NK_CHAIN_D 1024
#define NK_CHAIN_FF 4096
#define NK_CHAIN_HEADS 8
#define NK_CHAIN_PARTS 4     /* attention workgroups per head (each a quarter of the window)      */
#define NK_CHAIN_MAX_L 64    /* attention window (cached rows + the chunk's row)                 */
#define NK_CHAIN_SLOT 4160   /* hand-off entries per slot (4096 + the heads' 64 softmax terms)    */
#define NK_CHAIN_SLOTS 3     /* slots in rotation (hand-off i uses slot i mod 3)                 */
#define NK_CHAIN_PH 9        /* hand-offs per conformer block                                    */

/* device addresses of one block's weights (the layer's tensors in the model arenas) */
typedef struct {
    const u16 *ff1_w1, *ff1_w2, *wqkv, *wo, *pw1, *pw2, *ff2_w1, *ff2_w2;
    const float *ln_ff1_g, *ln_ff1_b, *ln_att_g, *ln_att_b, *ln_conv_g, *ln_conv_b, *ln_ff2_g, *ln_ff2_b;
    const float *ln_out_g, *ln_out_b, *bn_g, *bn_b, *dw_w, *bias_u, *bias_v, *ptab;
} NkChainLayer;

typedef struct {
    const NkChainLayer *L;          /* [n_layers] */
    const float *x_in;              /* block 0 input row [D] */
    float *x_out;                   /* last block's residual row [D], before its output norm */
    float *kv, *din;                /* layer 0's K/V and conv histories; layer l at + l * stride */
    unsigned long long *ll;         /* hand-off entries [NK_CHAIN_SLOTS][NK_CHAIN_SLOT]: {f32, tag} */
    u32 *abort_word;                /* epoch of a chunk that gave up waiting */
    int *err_word;                  /* host-visible: 1 + the hand-off that timed out */
    float *dump;                    /* optional [n_layers][D]: block outputs 0 .. n_layers-2 */
    const int *desc;                /* chunk descriptor (position, cache length, epoch) */
    unsigned long long kv_stride, din_stride; /* floats per layer */
    u32 n_layers, Lmax, spin_max;
    float eps, scale;
} NkChainArgs;

#endif
