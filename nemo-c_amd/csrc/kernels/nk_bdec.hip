/* Device-resident greedy RNNT loop of many streams at once (the batched decoder): the reference's
 * decoder_run (src/decoder.c:92-127) for every stream of a batch, one joint evaluation per step,
 * with no host round trip per step.  A step is five launches:
 *   bdec_lstm<0>  gates = Tx[last token] + h0 . Wh0^T for all S streams, where Tx = embed . Wx0^T + b0
 *                 is a table built once per model (the embedding half of layer 0's input is one of
 *                 V rows, so its product is looked up instead of recomputed), with the LSTM cell in
 *                 the epilogue (weight rows interleaved by unit: row 4u + q is gate q of unit u, so
 *                 a 16-column tile holds the four gates of four units); streams whose prediction is
 *                 stale write their provisional layer-0 state and the layer-1 input [h0' | h1];
 *   bdec_lstm<1>  gates = [h0' | h1] . [Wx1 | Wh1]^T + b1, the same cell; writes h1' (the joint.pred
 *                 input);
 *   bdec_pred     pred = h1' . Wjp^T + bjp for the streams that recomputed it, and their joint inputs
 *                 relu(enc[t + k] + pred) for the frames k of the chunk after the stream's t;
 *   gemm_mx64x64_argmax  joint scores with an argmax epilogue: per row, the best (score, lowest
 *                 index) of each wavefront's 32 columns as a packed key;
 *   bdec_decide   per stream: the best key of each scored frame, the greedy rule (first non-blank
 *                 frame wins: emit, commit the provisional LSTM state, the prediction becomes stale;
 *                 blank frames reset the symbol count; max_symbols moves past the frame), then the
 *                 next step's layer-0 input h0.
 * After a decision every stream still inside its chunk has emitted a token, so its prediction is
 * recomputed by the next step, which also writes its joint inputs; a prediction carried over from
 * the previous chunk gets its joint inputs from bdec_setup.  The GEMM rows of a step are the
 * streams still inside their chunk, compacted: each decision (or the chunk's setup) appends its
 * stream with an atomic slot counter (two counters by step parity; layer 0 clears the one the
 * step's decisions fill), and with more than 64 streams the workgroups of row blocks past the count
 * return at once, so a step costs what its live streams need.  A row's results do not depend on its
 * position.  LSTM states live in two slot sets per stream; committing a token flips the committed
 * set (the reference swaps its h/hp and c/cp buffers).
 *
 * bdec_lstm / bdec_pred are GEMMs over at most 64 rows per workgroup (grid.y = row blocks of 64):
 * a workgroup owns 16 columns; its W wavefronts split K (SPW steps of 32 each), issue every load
 * (activations of four 16-row tiles in the MFMA A layout, weights in the B layout) before the first
 * MFMA, multiply with A split into bf16 hi + lo, and leave their partial tiles in LDS; the epilogue
 * sums them with every thread working on its own (row, unit) cell or output. */
#include "nk_common.h"

__device__ __forceinline__ u32 hc_row(u32 s, u32 k, u32 which) { return (s * 2 + k) * 4 + which; }

__device__ __forceinline__ void ld8f(float (&d)[8], const float *p) {
    const floatx4 x = ((const floatx4 *)p)[0], y = ((const floatx4 *)p)[1];
    d[0] = x[0]; d[1] = x[1]; d[2] = x[2]; d[3] = x[3]; d[4] = y[0]; d[5] = y[1]; d[6] = y[2]; d[7] = y[3];
}

/* per-wavefront partial sums over its K range of one 64-row x 16-column tile, left in
 * sred[(wave * 4 + ti) * 64 + lane] in the MFMA D layout (row 16 ti + 4 (lane / 16) + e, column
 * lane % 16); ends with a barrier */
template <int W, int SPW>
__device__ __forceinline__ void fr64_partials(const float *A, u32 lda, const u16 *Wt, u32 M, u32 K, u32 r0,
                                              floatx4 *sred) {
    const u32 tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const u32 S = K >> 5, sb = wave * SPW, ns = sb < S ? min((u32)SPW, S - sb) : 0u;
    const u32 m = lane & 15, kq = 8 * (lane >> 4);
    uint4 fw[SPW];
#pragma unroll
    for (int s = 0; s < SPW; ++s) fw[s] = ld_nt16(Wt + (u64)(min(sb + s, S - 1) * 32 + kq));
    float x[SPW][4][8];
#pragma unroll
    for (int s = 0; s < SPW; ++s)
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) {
            const u32 r = min(r0 + 16 * ti + m, M - 1);
            ld8f(x[s][ti], A + (u64)r * lda + min(sb + s, S - 1) * 32 + kq);
        }
    floatx4 acc[4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) acc[ti] = (floatx4){ 0.f, 0.f, 0.f, 0.f };
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        if ((u32)s < ns) {
#pragma unroll
            for (int ti = 0; ti < 4; ++ti) {
                uint4 ah, al;
                split8(x[s][ti], ah, al);
                acc[ti] = mfma_bf16(ah, fw[s], acc[ti]);
                acc[ti] = mfma_bf16(al, fw[s], acc[ti]);
            }
        }
    }
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) sred[(wave * 4 + ti) * 64 + lane] = acc[ti];
    __syncthreads();
}

/* the tile's value at local row rl, column c: the W partials summed in wavefront order */
template <int W>
__device__ __forceinline__ float tile_at(const floatx4 *sred, u32 rl, u32 c) {
    const u32 ti = rl >> 4, ln = ((rl & 15) >> 2) * 16 + c, e = rl & 3;
    float v = ((const float *)&sred[ti * 64 + ln])[e];
#pragma unroll
    for (int w = 1; w < W; ++w) v += ((const float *)&sred[(w * 4 + ti) * 64 + ln])[e];
    return v;
}

/* rows of the current step (appended by the previous decision or the chunk's setup) */
__device__ __forceinline__ int step_rows(const NkBDecArgs &d) { return d.cnt[d.par ^ 1u]; }

/* the workgroup's 64 rows in LDS, staged before the GEMM phase (whose barrier publishes them):
 * stream, need, committed slot set, layer-0 table row, frame position, frames left to score (at
 * most W), first joint.enc row */
struct BDecStage {
    int s[64], need[64], cur[64], tok[64], t[64], lim[64], erow[64];
};

__device__ __forceinline__ void stage_state(const NkBDecArgs &d, u32 r0, BDecStage &ss) {
    if (threadIdx.x < 64) {
        const u32 i = threadIdx.x;
        const NkBDecRow p = d.rows[min(r0 + i, d.S - 1)];
        const bool ok = (int)(r0 + i) < step_rows(d);
        ss.s[i] = p.s;
        ss.need[i] = ok ? p.need : 0;
        ss.cur[i] = p.cur;
        ss.tok[i] = p.tok;
        ss.t[i] = p.t;
        ss.lim[i] = p.lim;
        ss.erow[i] = p.erow;
    }
}

/* the decision of a stream still inside its chunk appends it to the next step's rows */
__device__ __forceinline__ int append_row(const NkBDecArgs &d, u32 par, int s, int need, int cur, int last, int t,
                                          int frames, int erow) {
    const int slot = atomicAdd(d.cnt + par, 1);
    NkBDecRow r;
    r.s = s;
    r.need = need;
    r.cur = cur;
    r.tok = last >= 0 && last < (int)d.blank ? last : (int)d.blank;
    r.t = t;
    r.lim = min((int)d.W, frames - t);
    r.erow = erow;
    r.pad = 0;
    d.rows[slot] = r;
    return slot;
}

/* LSTM layer L (0 or 1) on all streams; grid (4P/16, ceil(S/64)), 64 W threads.  Layer 0: a.A = h0
 * [S][P], a.W = Wh0 rows interleaved by unit, gates start from the table row d.tx[tok] (bias
 * included); layer 1: a.A = [h0' | h1] [S][2P], a.W = [Wx1 | Wh1] interleaved, a.bias interleaved.
 * Epilogue: thread t < 256 runs the cell of row t / 4, unit 4 blockIdx.x + t % 4. */
template <int W, int SPW, int L>
__device__ __forceinline__ void bdec_lstm_impl(const NkGemmArgs &a, const NkBDecArgs &d, floatx4 *sred,
                                               BDecStage &ss) {
    static_assert(W >= 4, "the cell epilogue uses 256 threads");
    const u32 lane = threadIdx.x & 63, r0 = blockIdx.y * 64, col = blockIdx.x * 16 + (lane & 15);
    if (L == 0 && blockIdx.x == 0 && threadIdx.x == 0) d.cnt[d.par] = 0; /* this step's decisions append here */
    if (gridDim.y > 1 && (int)r0 >= step_rows(d)) return; /* no rows in this block */
    stage_state(d, r0, ss);
    fr64_partials<W, SPW>(a.A, a.lda, a.W + (u64)col * a.ldw, a.M, a.K, r0, sred);
    const u32 t = threadIdx.x;
    if (t >= 256) return;
    const u32 rl = t >> 2, j = t & 3, r = r0 + rl, P = d.P, u = blockIdx.x * 4 + j;
    if (!ss.need[rl]) return;
    const u32 s = (u32)ss.s[rl];
    const u32 kc = (u32)ss.cur[rl];
    constexpr u32 CI = L == 0 ? 1 : 3, HI = L == 0 ? 0 : 2;
    const float c_in = d.hc[(u64)hc_row(s, kc, CI) * P + u];
    const float h1c = L == 0 ? d.hc[(u64)hc_row(s, kc, 2) * P + u] : 0.0f;
    const floatx4 g0 = L == 0 ? *(const floatx4 *)(d.tx + (u64)ss.tok[rl] * 4 * P + 4 * u)
                              : *(const floatx4 *)(a.bias + 4 * u);
    float g[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) g[q] = g0[q] + tile_at<W>(sred, rl, 4 * j + q);
    const u32 kp = kc ^ 1u;
    const float c = sigmoid_f(g[1]) * c_in + sigmoid_f(g[0]) * tanhf(g[2]);
    const float h = sigmoid_f(g[3]) * tanhf(c);
    d.hc[(u64)hc_row(s, kp, CI) * P + u] = c;
    d.hc[(u64)hc_row(s, kp, HI) * P + u] = h;
    if (L == 0) {
        d.A1[(u64)r * 2 * P + u] = h;
        d.A1[(u64)r * 2 * P + P + u] = h1c;
    } else {
        d.hout[(u64)r * P + u] = h;
    }
}

/* joint inputs of step row r at column j: rows r W + k for the lim >= 1 frames after its t (loads
 * of clamped rows first, so that they are all in flight together) */
__device__ __forceinline__ void write_jin(const NkBDecArgs &d, u32 r, u32 j, float p, int t, int lim, int erow) {
    float e[NK_ATTC_MAX_C];
#pragma unroll
    for (int k = 0; k < NK_ATTC_MAX_C; ++k) e[k] = d.enc[(u64)(erow + t + min(k, lim - 1)) * d.J + j];
#pragma unroll
    for (int k = 0; k < NK_ATTC_MAX_C; ++k)
        if (k < lim) d.jin[(u64)(r * d.W + k) * d.J + j] = fmaxf(e[k] + p, 0.0f);
}

/* joint.pred for the streams that recompute their prediction, and their joint inputs; grid
 * (J/16, ceil(S/64)), 64 W threads; thread t handles column t % 16 of rows t / 16 + 16 i */
template <int W, int SPW>
__device__ __forceinline__ void bdec_pred_impl(const NkGemmArgs &a, const NkBDecArgs &d, floatx4 *sred,
                                               BDecStage &ss) {
    const u32 lane = threadIdx.x & 63, r0 = blockIdx.y * 64, col = blockIdx.x * 16 + (lane & 15);
    if (gridDim.y > 1 && (int)r0 >= step_rows(d)) return; /* no rows in this block */
    stage_state(d, r0, ss);
    fr64_partials<W, SPW>(a.A, a.lda, a.W + (u64)col * a.ldw, a.M, a.K, r0, sred);
    const u32 c = threadIdx.x & 15, j = blockIdx.x * 16 + c;
    const float bias = a.bias[j];
    for (u32 rl = threadIdx.x >> 4; rl < 64; rl += 4 * W) {
        if (!ss.need[rl]) continue;
        const u32 s = (u32)ss.s[rl];
        const float p = tile_at<W>(sred, rl, c) + bias;
        d.pred[(u64)s * d.J + j] = p;
        write_jin(d, r0 + rl, j, p, ss.t[rl], ss.lim[rl], ss.erow[rl]);
    }
}

#define BDEC_GEMM(NAME, IMPL, W, SPW)                                                                     \
    extern "C" __global__ __launch_bounds__(64 * W) void NAME(const NkGemmArgs a, const NkBDecArgs d) {   \
        __shared__ floatx4 sred[W * 4 * 64];                                                              \
        __shared__ BDecStage ss;                                                                          \
        IMPL(a, d, sred, ss);                                                                             \
    }
/* layer 0: K = P <= 640 (20 steps): 4 wavefronts x 5 steps; layer 1: K = 2P <= 1280: 8 x 5;
 * joint.pred: K = P: 4 x 5 */
BDEC_GEMM(bdec_lstm0_w4s5, (bdec_lstm_impl<4, 5, 0>), 4, 5)
BDEC_GEMM(bdec_lstm1_w8s5, (bdec_lstm_impl<8, 5, 1>), 8, 5)
BDEC_GEMM(bdec_pred_w4s5, (bdec_pred_impl<4, 5>), 4, 5)

/* next step's layer-0 input of stream s at step row r (one wavefront): its committed h0 (slot set
 * cur), P / 4 <= 192 float4 */
__device__ __forceinline__ void bdec_prepare(const NkBDecArgs &a, u32 r, u32 s, int cur) {
    const u32 n4 = a.P >> 2, lane = threadIdx.x;
    const floatx4 *h0 = (const floatx4 *)(a.hc + (u64)hc_row(s, (u32)cur, 0) * a.P);
    floatx4 *A = (floatx4 *)(a.A0 + (u64)r * a.P);
    floatx4 v[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) v[i] = h0[min(lane + 64 * i, n4 - 1)];
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (lane + 64 * i < n4) A[lane + 64 * i] = v[i];
}

/* new chunk: frames and first joint.enc row from the host, fresh frame position and counters; the
 * streams with frames become the first step's rows (row counter 1, zeroed by the host); a
 * prediction carried over from the previous chunk gets its joint inputs here.  grid S, 64 threads */
extern "C" __global__ __launch_bounds__(64) void bdec_setup(const NkBDecArgs a) {
    const u32 s = blockIdx.x;
    NkBDecStream *sp = a.st + s;
    const int frames = a.setup[2 * s], erow0 = a.setup[2 * s + 1], pred_valid = sp->pred_valid, cur = sp->cur;
    const int last = sp->last_token, need = 0 < frames && !pred_valid;
    int slot = 0;
    if (frames > 0 && threadIdx.x == 0) slot = append_row(a, 1u, (int)s, need, cur, last, 0, frames, erow0);
    slot = __shfl(slot, 0, 64);
    if (threadIdx.x == 0) {
        sp->frames = frames;
        sp->erow0 = erow0;
        sp->t = 0;
        sp->symbols = 0;
        sp->n_out = 0;
        sp->need = need;
        sp->slot = slot;
    }
    if (need) bdec_prepare(a, (u32)slot, s, cur);
    if (0 < frames && pred_valid) {
        const int lim = min((int)a.W, frames);
        for (u32 j = threadIdx.x; j < a.J; j += 64) write_jin(a, (u32)slot, j, a.pred[(u64)s * a.J + j], 0, lim, erow0);
    }
}

/* per stream (one wavefront): lane 4 r + p takes the maximum of keys p, p + 4, ... of scored frame r
 * (at most 16 frames, nkeys <= 64; the stream's key rows follow its step row), two exchanges finish
 * each frame's maximum, a ballot finds the first non-blank frame; then the greedy rule, and a
 * stream still inside its chunk is appended to the next step's rows with its layer-0 input. */
extern "C" __global__ __launch_bounds__(64) void bdec_decide(const NkBDecArgs a) {
    const u32 s = blockIdx.x, lane = threadIdx.x, row = lane >> 2, part = lane & 3;
    NkBDecStream *sp = a.st + s;
    const int frames = sp->frames, t = sp->t;
    if (t >= frames) return;
    int symbols = sp->symbols, cur = sp->cur, last = sp->last_token, n_out = sp->n_out, pred_valid = 1;
    const int rows = min(min((int)a.W, frames - t), NK_ATTC_MAX_C);
    const bool live = (int)row < rows;
    const unsigned long long *kr = a.keys + (u64)((u32)sp->slot * a.W + min((int)row, rows - 1)) * a.nkeys;
    unsigned long long kv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) kv[i] = kr[min(part + 4 * i, a.nkeys - 1)]; /* repeats change no maximum */
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) kv[i] = kv[i + w] > kv[i] ? kv[i + w] : kv[i];
    unsigned long long kb = kv[0];
#pragma unroll
    for (int msk = 1; msk < 4; msk <<= 1) {
        const unsigned long long o = shfl_xor_u64(kb, msk);
        kb = o > kb ? o : kb;
    }
    const int idx = (int)dec_key_index(kb);
    const unsigned long long nb = __ballot(part == 0 && live && idx != (int)a.blank);
    const int f = nb ? (__ffsll((long long)nb) - 1) >> 2 : rows; /* first non-blank frame */
    const int emitted = __shfl(idx, 4 * min(f, NK_ATTC_MAX_C - 1), 64);
    int k = f;
    if (f > 0) symbols = 0;
    if (f < rows) {
        if (lane == 0 && n_out < (int)a.tok_ld) a.tokens[(u64)s * a.tok_ld + (u32)n_out] = emitted;
        n_out++;
        last = emitted;
        cur ^= 1;
        pred_valid = 0;
        symbols++;
        if (symbols >= (int)a.max_symbols) { symbols = 0; k++; }
    }
    const int nt = t + k, need = nt < frames && !pred_valid;
    int slot = 0;
    if (nt < frames && lane == 0) slot = append_row(a, a.par, (int)s, need, cur, last, nt, frames, sp->erow0);
    slot = __shfl(slot, 0, 64);
    if (lane == 0) {
        sp->t = nt;
        sp->symbols = symbols;
        sp->pred_valid = pred_valid;
        sp->cur = cur;
        sp->last_token = last;
        sp->n_out = n_out;
        sp->need = need;
        sp->slot = slot;
    }
    if (need) bdec_prepare(a, (u32)slot, s, cur);
}
