/* Device-resident greedy RNNT loop for gfx950: the reference's decoder_run (src/decoder.c:92-127)
 * without a host round trip per joint evaluation.
 *
 * One iteration of the loop is three launches, captured into a graph that holds a run of
 * iterations (the host replays it until the chunk is done):
 *   dec_step   every wavefront first takes the decision of the previous iteration's joint (the
 *              greedy rule of src/decoder.c:107-122: first non-blank row wins; blank rows reset
 *              the symbol count; max_symbols moves past the frame) from the packed per-workgroup
 *              argmax keys, workgroup 0 records it (next state copy, emitted token); then, when the
 *              prediction must be recomputed, both LSTM layers from embed(last token)
 *              (src/decoder.c:57-77; zeros for blank).  Layer 0's input half Wx0 . embed(v) + b0
 *              is a per-token table built once by dec_tx_build, and its hidden half Wh0 . h0 was
 *              taken by the launch that made h0, so layer 0 is a cell over stored gate sums and
 *              the launch streams Wx1, Wh1 and Wh0 (for the next step) once;
 *   dec_pred   joint.pred projection of the new hidden state;
 *   dec_joint  joint scores relu(enc[t + r] + pred) . W_out + b for up to 16 remaining frames
 *              with one prediction (speculating blank, src/decoder.c:79-90); each workgroup
 *              writes the best (score, lowest index) of its 32 vocabulary rows.
 * Kernels whose work is not needed return at once.  Every value is computed in the reference's
 * order of operations: gates = (Wx.x + b) + Wh.h; c' = f*c + i*g; h' = o*tanh(c'); the argmax keeps
 * the lowest index on ties.  The LSTM weights are streamed with the wave64 layout of the GEMV
 * (lane l reads the 16-byte chunks l and l + 64 of every row). */
#include "nk_common.h"

/* The previous joint's argmax keys this lane reduces: lane l takes groups l/16, l/16 + 4, ... of
 * row l % 16 (they do not depend on the state, so they load beside it) */
struct DecKeys {
    unsigned long long k[NK_DEC_GROUPS / 4];
};
__device__ __forceinline__ DecKeys dec_keys(const NkDecArgs &a) {
    const u32 lane = threadIdx.x & 63;
    const unsigned long long *pp = a.part + (u64)(a.parity ^ 1) * NK_DEC_MAX_BATCH * NK_DEC_GROUPS;
    DecKeys ks;
#pragma unroll
    for (int q = 0; q < NK_DEC_GROUPS / 4; ++q) ks.k[q] = pp[(lane & 15) * NK_DEC_GROUPS + (lane >> 4) + 4 * q];
    return ks;
}

/* The decision of the previous joint, taken by one wavefront (every wavefront gets the same
 * answer).  Returns the new state; *tok = emitted token or -1. */
__device__ __forceinline__ NkDecState dec_decide(const NkDecArgs &a, const NkDecState s, const DecKeys &ks, int *tok) {
    NkDecState d = s;
    *tok = -1;
    if (!s.pending) return d;
    const u32 lane = threadIdx.x & 63;
    const int rows = min(NK_DEC_MAX_BATCH, s.frames - s.t);
    /* lane l reduces its groups of row l % 16; then the four lanes of a row combine */
    const u32 r = lane & 15;
    unsigned long long best = 0;
#pragma unroll
    for (int q = 0; q < NK_DEC_GROUPS / 4; ++q) best = ks.k[q] > best ? ks.k[q] : best;
    unsigned long long o = shfl_xor_u64(best, 16);
    best = o > best ? o : best;
    o = shfl_xor_u64(best, 32);
    best = o > best ? o : best;
    const u32 idx = dec_key_index(best);
    const bool nonblank = (int)r < rows && idx != a.blank;
    const unsigned long long mask = __ballot(nonblank);
    d.pending = 0;
    d.joints = s.joints + 1;
    if (!mask) { /* every scored frame decodes to blank: frames done, prediction kept */
        d.t = s.t + rows;
        d.symbols = 0;
        return d;
    }
    const int first = __builtin_ctzll(mask);
    const u32 t_idx = (u32)__shfl((int)idx, first, 64);
    *tok = (int)t_idx;
    d.last_token = (int)t_idx;
    d.cur = s.cur ^ 1; /* commit the provisional LSTM state */
    d.pred_valid = 0;
    d.n_out = s.n_out + 1;
    d.symbols = (first > 0 ? 0 : s.symbols) + 1;
    if (d.symbols >= (int)a.max_symbols) { d.symbols = 0; d.t = s.t + first + 1; }
    else d.t = s.t + first;
    return d;
}

/* lane l's 16-byte chunks l and l + 64 of a row of P floats (or bf16), zero past the row */
__device__ __forceinline__ void dec_row_chunks(float (&x)[2][8], const float *x_f32, const u16 *x_bf16, bool zero,
                                               u32 lane, u32 nch) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const u32 k = 8 * min(lane + 64 * q, nch - 1);
        if (x_bf16) {
            const uint4 w = *(const uint4 *)(x_bf16 + k);
            x[q][0] = bf_lo(w.x); x[q][1] = bf_hi(w.x); x[q][2] = bf_lo(w.y); x[q][3] = bf_hi(w.y);
            x[q][4] = bf_lo(w.z); x[q][5] = bf_hi(w.z); x[q][6] = bf_lo(w.w); x[q][7] = bf_hi(w.w);
        } else {
            const floatx4 p0 = *(const floatx4 *)(x_f32 + k), p1 = *(const floatx4 *)(x_f32 + k + 4);
            x[q][0] = p0[0]; x[q][1] = p0[1]; x[q][2] = p0[2]; x[q][3] = p0[3];
            x[q][4] = p1[0]; x[q][5] = p1[1]; x[q][6] = p1[2]; x[q][7] = p1[3];
        }
    }
}

/* wavefront sums of the four gate rows g*P + j of W against the lane's chunks of x */
__device__ __forceinline__ void dec_gate_dots(float (&out)[4], float (&x)[2][8], const uint4 (&w)[4][2]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        float sx = 0.0f;
#pragma unroll
        for (int q = 0; q < 2; ++q) sx = dot8(x[q], w[g][q], sx);
        out[g] = wsum(sx);
    }
}

/* the layer-0 input table: row v = Wx0 . embed(v) + b0 (the blank row: b0), gate-major [4P], in
 * dec_step's lane layout and summation order.  grid = ceil(P/4) x (blank + 1), block 256. */
extern "C" __global__ __launch_bounds__(256) void dec_tx_build(const NkDecArgs a) {
    const u32 j = blockIdx.x * 4 + (threadIdx.x >> 6), v = blockIdx.y, lane = threadIdx.x & 63, P = a.P, nch = P >> 3;
    if (j >= P) return;
    const bool zero = v == a.blank;
    float x[2][8];
    dec_row_chunks(x, nullptr, a.embed + (u64)(zero ? 0u : v) * P, zero, lane, nch);
    uint4 wx[4][2];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < 2; ++q) wx[g][q] = ld_c16(a.wx0 + (u64)(g * P + j) * P + 8 * min(lane + 64 * q, nch - 1));
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const bool ok = lane + 64 * q < nch;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[q][e] = ok && !zero ? x[q][e] : 0.0f;
    }
    float sx[4];
    dec_gate_dots(sx, x, wx);
    if (lane != 0) return;
#pragma unroll
    for (int g = 0; g < 4; ++g) a.tx[(u64)v * 4 * P + g * P + j] = sx[g] + a.b0[g * P + j];
}

/* One step of the loop up to the new hidden state, in one launch: the decision of the previous
 * joint, the layer-0 cell, LSTM layer 1, and layer 0's hidden product for the step after.
 * Layer 0's gates are tx[last token] + Wh0 . h0 with h0 the committed layer-0 state.  That state is
 * always the provisional state of the last launch that ran the cell (the decision that emits commits
 * it), so Wh0 . h0 is taken by that launch, against the h0 it has just made, and kept per state
 * slot in pre0: then the cell needs no GEMV of its own and a step is one dependent phase shorter.
 * grid = ceil(P/4), block 256.  Every workgroup takes the decision (the same answer) and computes
 * the whole layer-0 cell into LDS from pre0 and the table row; wavefront j then runs layer-1 unit j
 * and the four Wh0 rows of unit j against the new h0.  Workgroup 0 writes the state, the token and
 * the new layer-0 state. */
extern "C" __global__ __launch_bounds__(256) void dec_step(const NkDecArgs a) {
    __shared__ float h0s[1024];
    const u32 tid = threadIdx.x, lane = tid & 63, j = blockIdx.x * 4 + (tid >> 6), P = a.P;
    /* loaded together: the state, the joint's keys, and the layer-0 gate sums and cell states of
     * both slots (the decision picks the slot) for this thread's units tid, tid + 256, ... */
    const NkDecState s = a.st[a.parity];
    const DecKeys ks = dec_keys(a);
    constexpr int UPT = 4; /* units per thread: P <= 1024 */
    float pre2[2][UPT][4], c02[2][UPT];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            const u32 u = min(tid + 256 * i, P - 1);
#pragma unroll
            for (int g = 0; g < 4; ++g) pre2[sl][i][g] = a.pre0[(u64)sl * 4 * P + g * P + u];
            c02[sl][i] = a.hc[(u64)sl * 4 * P + 2 * P + u];
        }
    int tok;
    NkDecState d = dec_decide(a, s, ks, &tok);
    d.done = d.t >= d.frames;
    d.need_pred = !d.done && !d.pred_valid && !a.decide_only;
    if (blockIdx.x == 0 && tid == 0) {
        NkDecState ns = d;
        if (d.need_pred) ns.pred_valid = 1;
        ns.pending = !d.done && !a.decide_only;
        a.st[a.parity ^ 1] = ns;
        if (tok >= 0 && d.n_out <= NK_DEC_MAX_TOKENS) a.tokens[d.n_out - 1] = tok;
    }
    if (!d.need_pred) return; /* the same for every thread of the grid */
    const u32 nch = P >> 3, cm = (u32)d.cur, pv = cm ^ 1u, jj = min(j, P - 1);
    const float *hc_c = a.hc + (u64)cm * 4 * P;
    float *hc_p = a.hc + (u64)pv * 4 * P;
    /* this wavefront's weight rows first (they do not wait for the cell), then its state operands */
    uint4 wx[4][2], wh[4][2], w0[4][2];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const u64 off = (u64)(g * P + jj) * P + 8 * min(lane + 64 * q, nch - 1);
            wx[g][q] = ld_c16(a.wx1 + off);
            wh[g][q] = ld_c16(a.wh1 + off);
            w0[g][q] = ld_c16(a.wh0 + off);
        }
    float h1[2][8];
    dec_row_chunks(h1, hc_c + P, nullptr, false, lane, nch);
    float b1[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) b1[g] = a.b1[g * P + jj];
    const float c1 = hc_c[3 * P + jj];
    /* the layer-0 cell of every unit: gates = tx[last token] + Wh0 . h0 (input zero for blank) */
    const bool blank = d.last_token == (int)a.blank || d.last_token < 0;
    const float *tx_row = a.tx + (u64)(blank ? a.blank : (u32)d.last_token) * 4 * P;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
        const u32 u = tid + 256 * i;
        if (u >= P) break;
        float gate[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) gate[g] = tx_row[g * P + u] + (cm ? pre2[1][i][g] : pre2[0][i][g]);
        const float ig = sigmoid_f(gate[0]), fg = sigmoid_f(gate[1]), gg = tanhf(gate[2]), og = sigmoid_f(gate[3]);
        const float c = fg * (cm ? c02[1][i] : c02[0][i]) + ig * gg;
        const float h = og * tanhf(c);
        h0s[u] = h;
        if (blockIdx.x == 0) {
            hc_p[u] = h;
            hc_p[2 * P + u] = c;
        }
    }
    __syncthreads();
    if (j >= P) return;
    float x[2][8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const bool ok = lane + 64 * q < nch;
        const u32 k = 8 * min(lane + 64 * q, nch - 1);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            x[q][e] = ok ? h0s[k + e] : 0.0f;
            h1[q][e] = ok ? h1[q][e] : 0.0f;
        }
    }
    float sx[4], sh[4], s0[4];
    dec_gate_dots(sx, x, wx);
    dec_gate_dots(sh, h1, wh);
    dec_gate_dots(s0, x, w0);
    if (lane != 0) return;
    float gate[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) gate[g] = (sx[g] + b1[g]) + sh[g];
    const float ig = sigmoid_f(gate[0]), fg = sigmoid_f(gate[1]), gg = tanhf(gate[2]), og = sigmoid_f(gate[3]);
    const float c = fg * c1 + ig * gg;
    hc_p[3 * P + j] = c;
    hc_p[P + j] = og * tanhf(c);
    float *pre_p = a.pre0 + (u64)pv * 4 * P;
#pragma unroll
    for (int g = 0; g < 4; ++g) pre_p[g * P + j] = s0[g];
}

/* pred = joint.pred . h1' + b; one output per wavefront (K = P <= 1024) */
extern "C" __global__ __launch_bounds__(256) void dec_pred(const NkDecArgs a) {
    const NkDecState s = a.st[a.parity ^ 1];
    const u32 j = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (!s.need_pred || j >= a.J) return;
    const u32 P = a.P, nch = P >> 3;
    const float *h = a.hc + (u64)(s.cur ^ 1) * 4 * P + P;
    float x[2][8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const u32 k = 8 * min(lane + 64 * q, nch - 1);
        const floatx4 p0 = *(const floatx4 *)(h + k), p1 = *(const floatx4 *)(h + k + 4);
        x[q][0] = p0[0]; x[q][1] = p0[1]; x[q][2] = p0[2]; x[q][3] = p0[3];
        x[q][4] = p1[0]; x[q][5] = p1[1]; x[q][6] = p1[2]; x[q][7] = p1[3];
    }
    const float b = a.bjp[j];
    __builtin_amdgcn_sched_barrier(0);
    uint4 w[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) w[q] = ld_c16(a.wjp + (u64)j * P + 8 * min(lane + 64 * q, nch - 1));
    __builtin_amdgcn_sched_barrier(0);
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const bool ok = lane + 64 * q < nch;
        float xm[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) xm[e] = ok ? x[q][e] : 0.0f;
        acc = dot8(xm, w[q], acc);
    }
    const float v = wsum(acc) + b;
    if (lane == 0) a.pred[j] = v;
}

/* joint scores of frame t + blockIdx.y over vocabulary rows [32*blockIdx.x, +32): wavefront w
 * scores rows 32*g + 8*w + i (i < 8); the workgroup's best key goes to part[parity][row][g].
 * grid = (NK_DEC_GROUPS, NK_DEC_MAX_BATCH), block 256.  J <= 1024. */
extern "C" __global__ __launch_bounds__(256) void dec_joint(const NkDecArgs a) {
    __shared__ unsigned long long wbest[4];
    const NkDecState s = a.st[a.parity ^ 1];
    const int r = (int)blockIdx.y;
    if (!s.pending || r >= min(NK_DEC_MAX_BATCH, s.frames - s.t)) return;
    const u32 lane = threadIdx.x & 63, wave = threadIdx.x >> 6, J = a.J, nch = J >> 3;
    const u32 n0 = blockIdx.x * 32 + wave * 8;
    const float *e = a.enc + (u64)(s.t + r) * a.enc_ld;
    float x[2][8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const u32 k = 8 * min(lane + 64 * q, nch - 1);
        const floatx4 e0 = *(const floatx4 *)(e + k), e1 = *(const floatx4 *)(e + k + 4);
        const floatx4 p0 = *(const floatx4 *)(a.pred + k), p1 = *(const floatx4 *)(a.pred + k + 4);
        x[q][0] = e0[0] + p0[0]; x[q][1] = e0[1] + p0[1]; x[q][2] = e0[2] + p0[2]; x[q][3] = e0[3] + p0[3];
        x[q][4] = e1[0] + p1[0]; x[q][5] = e1[1] + p1[1]; x[q][6] = e1[2] + p1[2]; x[q][7] = e1[3] + p1[3];
    }
    float bias[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) bias[i] = a.bout[min(n0 + i, a.V - 1)];
    __builtin_amdgcn_sched_barrier(0);
    uint4 w[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int q = 0; q < 2; ++q) w[i][q] = ld_c16(a.wout + (u64)min(n0 + i, a.V - 1) * J + 8 * min(lane + 64 * q, nch - 1));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const bool ok = lane + 64 * q < nch;
#pragma unroll
        for (int k = 0; k < 8; ++k) x[q][k] = ok ? fmaxf(x[q][k], 0.0f) : 0.0f;
    }
    unsigned long long best = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < 2; ++q) acc = dot8(x[q], w[i][q], acc);
        const float v = wsum(acc) + bias[i];
        const unsigned long long k = n0 + i < a.V ? dec_key(v, n0 + i) : 0ull;
        best = k > best ? k : best;
    }
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = wbest[0];
#pragma unroll
        for (int w2 = 1; w2 < 4; ++w2) b = wbest[w2] > b ? wbest[w2] : b;
        a.part[((u64)a.parity * NK_DEC_MAX_BATCH + r) * NK_DEC_GROUPS + blockIdx.x] = b;
    }
}
