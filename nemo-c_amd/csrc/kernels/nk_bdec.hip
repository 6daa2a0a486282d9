/* Device-resident greedy RNNT loop of many streams at once (the batched decoder): the reference's
 * decoder_run (src/decoder.c:92-127) for every stream of a batch, one joint evaluation per step,
 * with no host round trip per step.  A step is six launches:
 *   bdec_lstm<0>  gates = [x | h0] . [Wx0 | Wh0]^T + b0 for all S streams, with the LSTM cell in the
 *                 epilogue (weight rows interleaved by unit: row 4u + q is gate q of unit u, so a
 *                 16-column tile holds the four gates of four units); streams whose prediction is
 *                 stale write their provisional layer-0 state and the layer-1 input [h0' | h1];
 *   bdec_lstm<1>  the same for layer 1; writes h1' (the joint.pred input);
 *   bdec_pred     pred = h1' . Wjp^T + bjp, stored for the streams that recomputed it;
 *   bdec_joint_in the joint inputs relu(enc[t + k] + pred) of the W frames after each stream's t;
 *   gemm_mx64x64_argmax  joint scores with an argmax epilogue: per row, the best (score, lowest
 *                 index) of each wavefront's 32 columns as a packed key;
 *   bdec_decide   per stream: the best key of each scored frame, the greedy rule (first non-blank
 *                 frame wins: emit, commit the provisional LSTM state, the prediction becomes stale;
 *                 blank frames reset the symbol count; max_symbols moves past the frame), then the
 *                 next step's layer-0 input [embed(last token) | h0].
 * Streams whose prediction is valid or whose chunk is done keep stale rows in the GEMM inputs;
 * their results are never stored.  LSTM states live in two slot sets per stream; committing a token
 * flips the committed set (the reference swaps its h/hp and c/cp buffers).
 *
 * bdec_lstm / bdec_pred are GEMMs over at most 64 rows per workgroup (grid.y = row blocks of 64):
 * a workgroup owns 16 columns; its W wavefronts split K (SPW steps of 32 each), issue every load
 * (activations of four 16-row tiles in the MFMA A layout, weights in the B layout) before the first
 * MFMA, multiply with A split into bf16 hi + lo, and sum their partial tiles in wavefront order
 * through LDS; wavefront 0 applies the epilogue. */
#include "nk_common.h"

__device__ __forceinline__ u32 hc_row(u32 s, u32 k, u32 which) { return (s * 2 + k) * 4 + which; }

__device__ __forceinline__ void ld8f(float (&d)[8], const float *p) {
    const floatx4 x = ((const floatx4 *)p)[0], y = ((const floatx4 *)p)[1];
    d[0] = x[0]; d[1] = x[1]; d[2] = x[2]; d[3] = x[3]; d[4] = y[0]; d[5] = y[1]; d[6] = y[2]; d[7] = y[3];
}

/* sum over K of one 64-row x 16-column tile: wavefront 0 returns tot[ti] (rows 16 ti + 4 (l/16) + e,
 * column l % 16); other wavefronts return false */
template <int W, int SPW>
__device__ __forceinline__ bool fr64_tile(const float *A, u32 lda, const u16 *Wt, u32 ldw, u32 M, u32 K, u32 r0,
                                          floatx4 *sred, floatx4 (&tot)[4]) {
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
    if (wave != 0) return false;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
        floatx4 t = sred[ti * 64 + lane];
#pragma unroll
        for (int w = 1; w < W; ++w) t += sred[(w * 4 + ti) * 64 + lane];
        tot[ti] = t;
    }
    return true;
}

/* need / committed slot set of the workgroup's 64 streams, staged in LDS before the GEMM phase
 * (fr64_tile's barrier publishes them) */
__device__ __forceinline__ void stage_state(const NkBDecArgs &d, u32 r0, int *sneed, int *scur) {
    if (threadIdx.x < 64) {
        const u32 s = min(r0 + threadIdx.x, d.S - 1);
        const NkBDecStream *p = d.st + s;
        sneed[threadIdx.x] = r0 + threadIdx.x < d.S ? p->need : 0;
        scur[threadIdx.x] = p->cur;
    }
}

/* LSTM layer L (0 or 1) on all streams; grid (4P/16, ceil(S/64)); a.W: [Wx | Wh] with rows
 * interleaved by unit, a.bias interleaved the same way.  Epilogue: the four gates of a unit sit in
 * four consecutive lanes; the first lane of each quad runs the cell for its 16 rows, all cell-state
 * loads issued before the first use. */
template <int W, int SPW, int L>
__device__ __forceinline__ void bdec_lstm_impl(const NkGemmArgs &a, const NkBDecArgs &d, floatx4 *sred, int *sneed,
                                               int *scur) {
    const u32 lane = threadIdx.x & 63, n0 = blockIdx.x * 16, r0 = blockIdx.y * 64, col = n0 + (lane & 15);
    stage_state(d, r0, sneed, scur);
    floatx4 tot[4];
    if (!fr64_tile<W, SPW>(a.A, a.lda, a.W + (u64)col * a.ldw, a.ldw, a.M, a.K, r0, sred, tot)) return;
    const float bias = a.bias[col];
    const u32 P = d.P, u = col >> 2, base = lane & ~3u;
    const bool leader = (lane & 3) == 0;
    constexpr u32 CI = L == 0 ? 1 : 3, HI = L == 0 ? 0 : 2;
    float c_in[4][4], h1c[4][4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const u32 rl = 16 * ti + 4 * (lane >> 4) + e, s = min(r0 + rl, d.S - 1), kc = (u32)scur[rl];
            c_in[ti][e] = d.hc[(u64)hc_row(s, kc, CI) * P + u];
            h1c[ti][e] = L == 0 ? d.hc[(u64)hc_row(s, kc, 2) * P + u] : 0.0f;
        }
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = tot[ti][e] + bias;
            const float gi = __shfl(v, (int)base, 64), gf = __shfl(v, (int)base + 1, 64);
            const float gg = __shfl(v, (int)base + 2, 64), go = __shfl(v, (int)base + 3, 64);
            const u32 rl = 16 * ti + 4 * (lane >> 4) + e, s = r0 + rl;
            if (!leader || s >= d.S || !sneed[rl]) continue;
            const u32 kp = (u32)scur[rl] ^ 1u;
            const float c = sigmoid_f(gf) * c_in[ti][e] + sigmoid_f(gi) * tanhf(gg);
            const float h = sigmoid_f(go) * tanhf(c);
            d.hc[(u64)hc_row(s, kp, CI) * P + u] = c;
            d.hc[(u64)hc_row(s, kp, HI) * P + u] = h;
            if (L == 0) {
                d.A1[(u64)s * 2 * P + u] = h;
                d.A1[(u64)s * 2 * P + P + u] = h1c[ti][e];
            } else {
                d.hout[(u64)s * P + u] = h;
            }
        }
}

/* joint.pred for the streams that recompute their prediction; grid (J/16, ceil(S/64)) */
template <int W, int SPW>
__device__ __forceinline__ void bdec_pred_impl(const NkGemmArgs &a, const NkBDecArgs &d, floatx4 *sred, int *sneed,
                                               int *scur) {
    const u32 lane = threadIdx.x & 63, n0 = blockIdx.x * 16, r0 = blockIdx.y * 64, j = n0 + (lane & 15);
    stage_state(d, r0, sneed, scur);
    floatx4 tot[4];
    if (!fr64_tile<W, SPW>(a.A, a.lda, a.W + (u64)j * a.ldw, a.ldw, a.M, a.K, r0, sred, tot)) return;
    const float bias = a.bias[j];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const u32 rl = 16 * ti + 4 * (lane >> 4) + e, s = r0 + rl;
            if (s < d.S && sneed[rl]) d.pred[(u64)s * d.J + j] = tot[ti][e] + bias;
        }
}

#define BDEC_GEMM(NAME, IMPL, W, SPW)                                                                     \
    extern "C" __global__ __launch_bounds__(64 * W) void NAME(const NkGemmArgs a, const NkBDecArgs d) {   \
        __shared__ floatx4 sred[W * 4 * 64];                                                              \
        __shared__ int sneed[64], scur[64];                                                               \
        IMPL(a, d, sred, sneed, scur);                                                                    \
    }
/* K = 2P = 1280 (40 steps): 8 wavefronts x 5 steps; K = P = 640: 4 x 5; tiny models fit both */
BDEC_GEMM(bdec_lstm0_w8s5, (bdec_lstm_impl<8, 5, 0>), 8, 5)
BDEC_GEMM(bdec_lstm1_w8s5, (bdec_lstm_impl<8, 5, 1>), 8, 5)
BDEC_GEMM(bdec_pred_w4s5, (bdec_pred_impl<4, 5>), 4, 5)

/* joint input rows: row s*W + k is frame t + k of stream s (rows past the chunk are left as they
 * are: their scores are never read); grid (ceil(J/256), S*W) */
extern "C" __global__ __launch_bounds__(256) void bdec_joint_in(const NkBDecArgs a) {
    const u32 r = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.J) return;
    const u32 s = r / a.W, k = r % a.W;
    const NkBDecStream *p = a.st + s;
    const int t = p->t, frames = p->frames;
    if (t >= frames || t + (int)k >= frames) return;
    a.jin[(u64)r * a.J + i] = fmaxf(a.enc[(u64)(p->erow0 + t + (int)k) * a.J + i] + a.pred[(u64)s * a.J + i], 0.0f);
}

/* next step's layer-0 input for stream s (all threads of the workgroup): [embed(last) | h0] */
__device__ __forceinline__ void bdec_prepare(const NkBDecArgs &a, u32 s, const NkBDecStream &st) {
    if (!(st.t < st.frames && !st.pred_valid)) return;
    const u32 P = a.P;
    float *A = a.A0 + (u64)s * 2 * P;
    const bool emb = st.last_token >= 0 && (u32)st.last_token != a.blank;
    const float *h0 = a.hc + (u64)hc_row(s, (u32)st.cur, 0) * P;
    for (u32 j = threadIdx.x; j < P; j += blockDim.x) {
        A[j] = emb ? bf2f(a.embed[(u64)st.last_token * P + j]) : 0.0f;
        A[P + j] = h0[j];
    }
}

/* new chunk: frames and first joint.enc row from the host, fresh frame position and counters */
extern "C" __global__ __launch_bounds__(64) void bdec_setup(const NkBDecArgs a) {
    const u32 s = blockIdx.x;
    NkBDecStream x = a.st[s];
    x.frames = a.setup[2 * s];
    x.erow0 = a.setup[2 * s + 1];
    x.t = 0;
    x.symbols = 0;
    x.n_out = 0;
    x.need = x.t < x.frames && !x.pred_valid;
    if (threadIdx.x == 0) a.st[s] = x;
    bdec_prepare(a, s, x);
}

/* per stream (one wavefront): best key of each scored frame, the greedy rule, next step's input.
 * All keys of the scored frames (at most 16 x 64) are loaded before the first reduction. */
extern "C" __global__ __launch_bounds__(64) void bdec_decide(const NkBDecArgs a) {
    const u32 s = blockIdx.x, lane = threadIdx.x;
    NkBDecStream x = a.st[s];
    if (x.t >= x.frames) return;
    const int rows = min(min((int)a.W, x.frames - x.t), NK_ATTC_MAX_C);
    unsigned long long kv[NK_ATTC_MAX_C];
#pragma unroll
    for (int k = 0; k < NK_ATTC_MAX_C; ++k) {
        const bool ok = k < rows && lane < a.nkeys;
        const u32 kk = ok ? (u32)k : 0u, q = ok ? lane : 0u;
        const unsigned long long v = a.keys[(u64)(s * a.W + kk) * a.nkeys + q];
        kv[k] = ok ? v : 0ull;
    }
    int best_idx[NK_ATTC_MAX_C];
#pragma unroll
    for (int k = 0; k < NK_ATTC_MAX_C; ++k) {
        unsigned long long kb = kv[k];
#pragma unroll
        for (int msk = 1; msk < 64; msk <<= 1) {
            const unsigned long long o = shfl_xor_u64(kb, msk);
            kb = o > kb ? o : kb;
        }
        best_idx[k] = (int)dec_key_index(kb);
    }
    x.pred_valid = 1;
    int k = 0;
    int emitted = -1;
#pragma unroll
    for (int q = 0; q < NK_ATTC_MAX_C; ++q) {
        if (q >= rows || emitted >= 0) continue;
        const int p = best_idx[q];
        k = q + 1;
        if (p == (int)a.blank) { x.symbols = 0; continue; }
        emitted = p;
        k = q;
    }
    if (emitted >= 0) {
        if (lane == 0 && x.n_out < (int)a.tok_ld) a.tokens[(u64)s * a.tok_ld + (u32)x.n_out] = emitted;
        x.n_out++;
        x.last_token = emitted;
        x.cur ^= 1;
        x.pred_valid = 0;
        x.symbols++;
        if (x.symbols >= (int)a.max_symbols) { x.symbols = 0; k++; }
    }
    x.t += k;
    x.need = x.t < x.frames && !x.pred_valid;
    if (lane == 0) a.st[s] = x;
    bdec_prepare(a, s, x);
}
