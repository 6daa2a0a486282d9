/* Device-resident greedy RNNT loop of many streams at once (the batched decoder): the reference's
 * decoder_run (src/decoder.c:92-127) for every stream of a batch, one joint evaluation per step,
 * with no host round trip per step.  A step is
 *   GEMM   gates0 += [x | h0] . [Wx0 | Wh0]^T          (rows: all streams; gates0 preset to b0)
 *   bdec_cell0   LSTM layer 0 cell for the streams that recompute their prediction; builds the
 *                layer-1 inputs [h0' | h1] and presets gates1 = b1
 *   GEMM   gates1 += [h0' | h1] . [Wx1 | Wh1]^T
 *   bdec_cell1   LSTM layer 1 cell; presets the prediction accumulator to the joint.pred bias
 *   GEMM   predtmp += h1' . Wjp^T
 *   bdec_joint_in  relu(enc[t + k] + pred) for the W frames after each stream's t
 *   GEMM   logits = jin . Wout^T + bout
 *   bdec_decide  per stream: argmax of each scored frame (lowest index on ties), then the greedy
 *                rule (first non-blank frame wins: emit, commit the provisional LSTM state, the
 *                prediction becomes stale; blank frames reset the symbol count; max_symbols moves
 *                past the frame), then the inputs of the next step.
 * Streams whose prediction is valid or whose chunk is done pass through the GEMMs as zero rows and
 * are masked in the cells.  LSTM states live in two slot sets per stream; committing a token flips
 * the committed set (the reference swaps its h/hp and c/cp buffers). */
#include "nk_common.h"

__device__ __forceinline__ u32 hc_row(u32 s, u32 k, u32 which) { return (s * 2 + k) * 4 + which; }

/* next step's layer-0 input and gate preset for stream s (all threads of the workgroup) */
__device__ __forceinline__ void bdec_prepare(const NkBDecArgs &a, u32 s, const NkBDecStream &st) {
    const bool need = st.t < st.frames && !st.pred_valid;
    const u32 P = a.P;
    float *A = a.A0 + (u64)s * 2 * P;
    const bool emb = need && st.last_token >= 0 && (u32)st.last_token != a.blank;
    const float *h0 = a.hc + (u64)hc_row(s, (u32)st.cur, 0) * P;
    for (u32 j = threadIdx.x; j < P; j += blockDim.x) {
        A[j] = emb ? bf2f(a.embed[(u64)st.last_token * P + j]) : 0.0f;
        A[P + j] = need ? h0[j] : 0.0f;
    }
    float *g = a.g0 + (u64)s * 4 * P;
    for (u32 j = threadIdx.x; j < 4 * P; j += blockDim.x) g[j] = a.b0[j];
}

/* new chunk: frames and first joint.enc row from the host, fresh frame position and counters */
extern "C" __global__ __launch_bounds__(256) void bdec_setup(const NkBDecArgs a) {
    const u32 s = blockIdx.x;
    __shared__ NkBDecStream st;
    if (threadIdx.x == 0) {
        NkBDecStream x = a.st[s];
        x.frames = a.setup[2 * s];
        x.erow0 = a.setup[2 * s + 1];
        x.t = 0;
        x.symbols = 0;
        x.n_out = 0;
        x.need = x.t < x.frames && !x.pred_valid;
        a.st[s] = x;
        st = x;
    }
    __syncthreads();
    bdec_prepare(a, s, st);
}

/* LSTM cell c' = f*c + i*g, h' = o*tanh(c') (reference src/kernels.metal:474-486), gate order
 * i, f, g, o, on the provisional slot set of the streams that recompute their prediction */
__device__ __forceinline__ void bdec_cell(const float *gt, const float *c_in, float *c_out, float *h_out, u32 P, u32 j,
                                          float &h) {
    const float ig = sigmoid_f(gt[j]), fg = sigmoid_f(gt[P + j]), gg = tanhf(gt[2 * P + j]), og = sigmoid_f(gt[3 * P + j]);
    const float c = fg * c_in[j] + ig * gg;
    h = og * tanhf(c);
    c_out[j] = c;
    h_out[j] = h;
}

extern "C" __global__ __launch_bounds__(256) void bdec_cell0(const NkBDecArgs a) {
    const u32 s = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x, P = a.P;
    if (j >= P) return;
    const NkBDecStream st = a.st[s];
    const u32 kc = (u32)st.cur, kp = kc ^ 1u;
    float *A = a.A1 + (u64)s * 2 * P;
    if (st.need) {
        float h;
        bdec_cell(a.g0 + (u64)s * 4 * P, a.hc + (u64)hc_row(s, kc, 1) * P, a.hc + (u64)hc_row(s, kp, 1) * P,
                  a.hc + (u64)hc_row(s, kp, 0) * P, P, j, h);
        A[j] = h;
        A[P + j] = a.hc[(u64)hc_row(s, kc, 2) * P + j];
    } else {
        A[j] = 0.0f;
        A[P + j] = 0.0f;
    }
    float *g = a.g1 + (u64)s * 4 * P;
#pragma unroll
    for (int q = 0; q < 4; ++q) g[q * P + j] = a.b1[q * P + j];
}

extern "C" __global__ __launch_bounds__(256) void bdec_cell1(const NkBDecArgs a) {
    const u32 s = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x, P = a.P;
    if (j >= P) return;
    const NkBDecStream st = a.st[s];
    const u32 kc = (u32)st.cur, kp = kc ^ 1u;
    float h = 0.0f;
    if (st.need)
        bdec_cell(a.g1 + (u64)s * 4 * P, a.hc + (u64)hc_row(s, kc, 3) * P, a.hc + (u64)hc_row(s, kp, 3) * P,
                  a.hc + (u64)hc_row(s, kp, 2) * P, P, j, h);
    a.hout[(u64)s * P + j] = h;
    for (u32 k = j; k < a.J; k += P) a.predtmp[(u64)s * a.J + k] = a.bjp[k];
}

/* joint input rows: row s*W + k is frame t + k of stream s (zeros past the chunk) */
extern "C" __global__ __launch_bounds__(256) void bdec_joint_in(const NkBDecArgs a) {
    const u32 r = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.J) return;
    const u32 s = r / a.W, k = r % a.W;
    const NkBDecStream st = a.st[s];
    const int frame = st.t + (int)k;
    float v = 0.0f;
    if (st.t < st.frames && frame < st.frames) {
        const float p = st.need ? a.predtmp[(u64)s * a.J + i] : a.pred[(u64)s * a.J + i];
        v = fmaxf(a.enc[(u64)(st.erow0 + frame) * a.J + i] + p, 0.0f);
    }
    a.jin[(u64)r * a.J + i] = v;
}

/* per stream: argmax of its scored frames, the greedy rule, the next step's inputs */
extern "C" __global__ __launch_bounds__(256) void bdec_decide(const NkBDecArgs a) {
    const u32 s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ NkBDecStream st;
    __shared__ int best[64];
    if (tid == 0) st = a.st[s];
    __syncthreads();
    const bool active = st.t < st.frames;
    const int rows = active ? min((int)a.W, st.frames - st.t) : 0;
    for (int k = (int)wave; k < rows; k += 4) {
        const float *x = a.logits + (u64)(s * a.W + (u32)k) * a.ldl;
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (u32 n = lane; n < a.V; n += 64) {
            const float v = x[n];
            if (v > bv || (v == bv && (int)n < bi)) { bv = v; bi = (int)n; }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m, 64);
            const int oi = __shfl_xor(bi, m, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) best[k] = bi;
    }
    if (active && st.need)
        for (u32 i = tid; i < a.J; i += 256) a.pred[(u64)s * a.J + i] = a.predtmp[(u64)s * a.J + i];
    __syncthreads();
    if (tid == 0 && active) {
        NkBDecStream x = st;
        x.pred_valid = 1;
        int k = 0;
        for (; k < rows; ++k) {
            const int p = best[k];
            if (p == (int)a.blank) { x.symbols = 0; continue; }
            if (x.n_out < (int)a.tok_ld) a.tokens[(u64)s * a.tok_ld + (u32)x.n_out] = p;
            x.n_out++;
            x.last_token = p;
            x.cur ^= 1;
            x.pred_valid = 0;
            x.symbols++;
            if (x.symbols >= (int)a.max_symbols) { x.symbols = 0; k++; }
            break;
        }
        x.t += k;
        x.need = x.t < x.frames && !x.pred_valid;
        st = x;
        a.st[s] = x;
    } else if (tid == 0) {
        st.need = 0;
        a.st[s].need = 0;
    }
    __syncthreads();
    bdec_prepare(a, s, st);
}
