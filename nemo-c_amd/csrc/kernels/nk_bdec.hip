/* Device-resident greedy RNNT loop of many streams at once (the batched decoder): the reference's
 * decoder_run (src/decoder.c:92-127) for every stream of a batch, one joint evaluation per step,
 * with no host round trip per step.  A step is four launches:
 *   bdec_lstm1    gates = [h0' | h1] . [Wx1 | Wh1]^T + b1 with the LSTM cell in the epilogue (weight
 *                 rows interleaved by unit: row 4u + q is gate q of unit u, so a 16-column tile
 *                 holds the four gates of four units); writes h1' (the joint.pred input);
 *   bdec_pred     pred = h1' . Wjp^T + bjp for the streams that recomputed it, and their joint inputs
 *                 relu(enc[t + k] + pred) for the frames k of the chunk after the stream's t.  A
 *                 second range of workgroups takes h0' . Wh0^T, the hidden half of layer 0's gates
 *                 for the step after, into pre0 of the provisional slot set (which the emitting
 *                 decision commits);
 *   gemm_mx64x64_argmax  joint scores with an argmax epilogue: per row, the best (score, lowest
 *                 index) of each wavefront's 32 columns as a packed key;
 *   bdec_decide   per stream (four wavefronts: the first decides): the best key of each scored
 *                 frame, the greedy rule (first non-blank
 *                 frame wins: emit, commit the provisional LSTM state, the prediction becomes stale;
 *                 blank frames reset the symbol count; max_symbols moves past the frame), then, for
 *                 a stream whose prediction must be recomputed, layer 0: gates = Tx[last token] +
 *                 pre0 of the committed slot set, where Tx = embed . Wx0^T + b0 is a table built
 *                 once per model (the embedding half of layer 0's input is one of V rows), and the
 *                 cell, which writes the provisional layer-0 state and the layer-1 input
 *                 [h0' | h1] of the stream's next step row.
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
 * bdec_lstm1 / bdec_pred are GEMMs over at most 64 rows per workgroup (grid.y = row blocks of 64):
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
    for (int s = 0; s < SPW; ++s) fw[s] = ld_c16(Wt + (u64)(min(sb + s, S - 1) * 32 + kq));
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

/* LSTM layer 1 on all streams; grid (4P/16, ceil(S/64)), 64 W threads: a.A = [h0' | h1] [S][2P],
 * a.W = [Wx1 | Wh1] interleaved, a.bias interleaved; epilogue: thread t < 256 runs the cell of row
 * t / 4, unit 4 blockIdx.x + t % 4. */
template <int W, int SPW>
__device__ __forceinline__ void bdec_lstm_impl(const NkGemmArgs &a, const NkBDecArgs &d, floatx4 *sred,
                                               BDecStage &ss) {
    static_assert(W >= 4, "the cell epilogue uses 256 threads");
    const u32 P = d.P, lane = threadIdx.x & 63, r0 = blockIdx.y * 64, col = blockIdx.x * 16 + (lane & 15);
    if (blockIdx.x == 0 && threadIdx.x == 0) d.cnt[d.par] = 0; /* this step's decisions append here */
    if (gridDim.y > 1 && (int)r0 >= step_rows(d)) return; /* no rows in this block */
    stage_state(d, r0, ss);
    fr64_partials<W, SPW>(a.A, a.lda, a.W + (u64)col * a.ldw, a.M, a.K, r0, sred);
    const u32 t = threadIdx.x;
    if (t >= 256) return;
    const u32 rl = t >> 2, j = t & 3, r = r0 + rl, u = blockIdx.x * 4 + j;
    if (!ss.need[rl]) return;
    const u32 s = (u32)ss.s[rl];
    const u32 kc = (u32)ss.cur[rl], kp = kc ^ 1u;
    const float c_in = d.hc[(u64)hc_row(s, kc, 3) * P + u];
    const floatx4 g0 = *(const floatx4 *)(a.bias + 4 * u);
    float g[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) g[q] = g0[q] + tile_at<W>(sred, rl, 4 * j + q);
    const float c = sigmoid_f(g[1]) * c_in + sigmoid_f(g[0]) * tanhf(g[2]);
    const float h = sigmoid_f(g[3]) * tanhf(c);
    d.hc[(u64)hc_row(s, kp, 3) * P + u] = c;
    d.hc[(u64)hc_row(s, kp, 2) * P + u] = h;
    d.hout[(u64)r * P + u] = h;
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
 * (J/16 + 4P/16, ceil(S/64)), 64 W threads.  Workgroups x < J/16: thread t handles column t % 16 of
 * rows t / 16 + 16 i.  Workgroups x >= J/16: h0' (the first P columns of the layer-1 input rows) .
 * Wh0^T for columns 16 (x - J/16) + [0, 16) into pre0 of the row's provisional slot set. */
template <int W, int SPW>
__device__ __forceinline__ void bdec_pred_impl(const NkGemmArgs &a, const NkBDecArgs &d, floatx4 *sred,
                                               BDecStage &ss) {
    const u32 nb = d.J / 16, hid = blockIdx.x >= nb, bx = hid ? blockIdx.x - nb : blockIdx.x;
    const u32 lane = threadIdx.x & 63, r0 = blockIdx.y * 64, col = bx * 16 + (lane & 15);
    if (gridDim.y > 1 && (int)r0 >= step_rows(d)) return; /* no rows in this block */
    stage_state(d, r0, ss);
    if (hid) {
        const u32 P = d.P;
        fr64_partials<W, SPW>(d.A1, 2 * P, d.wh0 + (u64)col * d.wh0_ld, a.M, P, r0, sred);
        for (u32 t = threadIdx.x; t < 256; t += 64 * W) {
            const u32 rl = t >> 2, j = t & 3, u = bx * 4 + j;
            if (!ss.need[rl]) continue;
            const u32 s = (u32)ss.s[rl], kp = (u32)ss.cur[rl] ^ 1u;
            floatx4 v;
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = tile_at<W>(sred, rl, 4 * j + q);
            *(floatx4 *)(d.pre0 + ((u64)s * 2 + kp) * 4 * P + 4 * u) = v;
        }
        return;
    }
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
    extern "C" __global__ __launch_bounds__(64 * W) void NAME(const NkBDecGemmArgs x) {                   \
        __shared__ floatx4 sred[W * 4 * 64];                                                              \
        __shared__ BDecStage ss;                                                                          \
        IMPL(x.g, x.d, sred, ss);                                                                         \
    }
/* layer 1: K = 2P <= 1280: 8 wavefronts x 5 steps; joint.pred and Wh0: K = P: 4 x 5 */
BDEC_GEMM(bdec_lstm1_w8s5, (bdec_lstm_impl<8, 5>), 8, 5)
BDEC_GEMM(bdec_pred_w4s5, (bdec_pred_impl<4, 5>), 4, 5)

/* layer 0 of stream s for its next step row r (NT threads, unit u = thread + NT i): gates =
 * Tx[tok] + pre0 of the committed slot set cur (the table row and the hidden product in that order,
 * as a GEMM epilogue adding its tile to the table row would), the cell, the provisional layer-0
 * state (slot set cur ^ 1) and the layer-1 input row [h0' | h1 of slot set cur].  P <= 640. */
template <int NT>
__device__ __forceinline__ void bdec_cell0(const NkBDecArgs &a, u32 r, u32 s, int cur, int tok) {
    const u32 P = a.P, lane = threadIdx.x, kc = (u32)cur, kp = kc ^ 1u;
    const float *tx = a.tx + (u64)(u32)tok * 4 * P;
    const float *pre = a.pre0 + ((u64)s * 2 + kc) * 4 * P;
    constexpr int UPL = (640 + NT - 1) / NT; /* units per thread */
    floatx4 tv[UPL], pv[UPL];
    float cv[UPL], h1[UPL];
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
        const u32 u = min(lane + NT * i, P - 1);
        tv[i] = *(const floatx4 *)(tx + 4 * u);
        pv[i] = *(const floatx4 *)(pre + 4 * u);
        cv[i] = a.hc[(u64)hc_row(s, kc, 1) * P + u];
        h1[i] = a.hc[(u64)hc_row(s, kc, 2) * P + u];
    }
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
        const u32 u = lane + NT * i;
        if (u >= P) break;
        float g[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) g[q] = tv[i][q] + pv[i][q];
        const float c = sigmoid_f(g[1]) * cv[i] + sigmoid_f(g[0]) * tanhf(g[2]);
        const float h = sigmoid_f(g[3]) * tanhf(c);
        a.hc[(u64)hc_row(s, kp, 1) * P + u] = c;
        a.hc[(u64)hc_row(s, kp, 0) * P + u] = h;
        a.A1[(u64)r * 2 * P + u] = h;
        a.A1[(u64)r * 2 * P + P + u] = h1[i];
    }
}

/* the layer-0 table row of a stream's last token (the blank's row, zero input, when none) */
__device__ __forceinline__ int tx_row_of(const NkBDecArgs &a, int last) {
    return last >= 0 && last < (int)a.blank ? last : (int)a.blank;
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
        sp->joints = 0;
    }
    if (need) bdec_cell0<64>(a, (u32)slot, s, cur, tx_row_of(a, last));
    if (0 < frames && pred_valid) {
        const int lim = min((int)a.W, frames);
        for (u32 j = threadIdx.x; j < a.J; j += 64) write_jin(a, (u32)slot, j, a.pred[(u64)s * a.J + j], 0, lim, erow0);
    }
}

/* per stream (one wavefront): lane 4 r + p takes the maximum of keys p, p + 4, ... of scored frame r
 * (at most 16 frames, nkeys <= 64; the stream's key rows follow its step row), two exchanges finish
 * each frame's maximum, a ballot finds the first non-blank frame; then the greedy rule, and a
 * stream still inside its chunk is appended to the next step's rows with its layer-0 input. */
extern "C" __global__ __launch_bounds__(256) void bdec_decide(const NkBDecArgs a) {
    __shared__ int dres[4]; /* need, slot, cur, last of the decision, for the four wavefronts */
    const u32 s = blockIdx.x, lane = threadIdx.x, row = lane >> 2, part = lane & 3;
    NkBDecStream *sp = a.st + s;
    const int frames = sp->frames, t = sp->t;
    if (t >= frames) return; /* the same for the whole workgroup */
    if (threadIdx.x < 64) {
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
            sp->joints = sp->joints + 1;
            dres[0] = need;
            dres[1] = slot;
            dres[2] = cur;
            dres[3] = last;
        }
    }
    __syncthreads();
    if (dres[0]) bdec_cell0<256>(a, (u32)dres[1], s, dres[2], tx_row_of(a, dres[3]));
}
