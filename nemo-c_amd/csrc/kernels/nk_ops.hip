/* Non-GEMM kernels of the streaming chunk for gfx950: LayerNorm (single and paired),
 * relative-position attention, causal depthwise conv + LN + SiLU, the subsampling convs, and the
 * RNNT decoder's LSTM cell and joint argmax.  Each states the reference kernel it replaces. */
#include "nk_common.h"

/* Block-wide sum over 256 threads (4 wavefronts), combined in wavefront order. */
__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

/* LayerNorm of one row held in registers (reference src/kernels.metal:257-288):
 * mean = sum/D, var = sum((x-mean)^2)/D, inv = 1/sqrt(var + eps), y = (x-mean)*inv*g + b. */
__device__ __forceinline__ void ln_regs(float *v, int per, u32 D, float eps, const float *g, const float *b, float *red) {
    const u32 tid = threadIdx.x;
    float s = 0.0f;
    for (int k = 0; k < per; ++k)
        if (tid + k * NK_LN_THREADS < D) s += v[k];
    const float mean = block_sum256(s, red) / (float)D;
    float q = 0.0f;
    for (int k = 0; k < per; ++k)
        if (tid + k * NK_LN_THREADS < D) { const float d = v[k] - mean; q += d * d; }
    const float var = block_sum256(q, red);
    const float inv = 1.0f / sqrtf(var / (float)D + eps);
    for (int k = 0; k < per; ++k) {
        const u32 i = tid + k * NK_LN_THREADS;
        if (i < D) v[k] = (v[k] - mean) * inv * g[i] + b[i];
    }
}

/* One workgroup per row. Y1 = LN(X; g1,b1); with Y2 set, also Y2 = LN(Y1; g2,b2)
 * (the paired norm_out + next norm_feed_forward1 of reference src/kernels.metal:210-255). */
extern "C" __global__ __launch_bounds__(256) void layernorm(const NkLnArgs a) {
    __shared__ float red[4];
    const u32 row = blockIdx.x, tid = threadIdx.x;
    const int per = (int)((a.D + NK_LN_THREADS - 1) / NK_LN_THREADS);
    const float *x = a.X + (u64)row * a.D;
    float v[NK_LN_MAX_PER];
    for (int k = 0; k < per; ++k) {
        const u32 i = tid + k * NK_LN_THREADS;
        v[k] = i < a.D ? x[i] : 0.0f;
    }
    ln_regs(v, per, a.D, a.eps, a.g1, a.b1, red);
    for (int k = 0; k < per; ++k) {
        const u32 i = tid + k * NK_LN_THREADS;
        if (i < a.D) a.Y1[(u64)row * a.D + i] = v[k];
    }
    if (!a.Y2) return;
    ln_regs(v, per, a.D, a.eps, a.g2, a.b2, red);
    for (int k = 0; k < per; ++k) {
        const u32 i = tid + k * NK_LN_THREADS;
        if (i < a.D) a.Y2[(u64)row * a.D + i] = v[k];
    }
}

/* Relative-position attention, one workgroup (2 wavefronts, dh = 128 threads) per (head, query):
 * reference src/kernels.metal:290-348.  Scores: each wavefront takes every other key and its 64
 * lanes cover two head dims each; softmax over the whole window (no mask inside the chunk);
 * output: thread d sums the softmax-weighted V column d. */
extern "C" __global__ __launch_bounds__(128) void attention_rel(const NkAttnArgs a) {
    __shared__ float qu[128], qv[128], s[NK_ATT_MAX_L], red[2];
    const u32 h = blockIdx.x, i = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const u32 off = h * a.dh;
    const float *Q = a.Q, *Kp = a.K, *Vp = a.V;
    u32 L = a.L;
    if (a.desc) {
        const u32 pos = (u32)a.desc[NK_DESC_POS], cl = (u32)a.desc[NK_DESC_CACHE];
        Q += (u64)pos * a.ldq;
        Kp += (u64)(pos - cl) * a.ldk;
        Vp += (u64)(pos - cl) * a.ldk;
        L = cl + a.c;
    }
    {
        const float q = Q[(u64)i * a.ldq + off + tid];
        qu[tid] = q + a.bu[off + tid];
        qv[tid] = q + a.bv[off + tid];
    }
    __syncthreads();
    const u32 d0 = 2 * lane;
    const float2 u2 = make_float2(qu[d0], qu[d0 + 1]), v2 = make_float2(qv[d0], qv[d0 + 1]);
    for (u32 j = wave; j < L; j += 2) {
        const u32 prow = (a.Lmax - L) + (a.c - 1 - i + j); /* relative position (L-c+i) - j */
        const float2 k2 = *(const float2 *)(Kp + (u64)j * a.ldk + off + d0);
        const float2 p2 = *(const float2 *)(a.P + (u64)prow * a.D + off + d0);
        float part = u2.x * k2.x + u2.y * k2.y + v2.x * p2.x + v2.y * p2.y;
        part = wave_sum(part);
        if (lane == 0) s[j] = part * a.scale;
    }
    __syncthreads();
    const float sv = tid < L ? s[tid] : -INFINITY;
    float mx = wave_max(sv);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(red[0], red[1]);
    __syncthreads();
    const float ev = tid < L ? expf(sv - mx) : 0.0f;
    float sum = wave_sum(ev);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = red[0] + red[1];
    if (tid < L) s[tid] = ev / sum;
    __syncthreads();
    float acc = 0.0f;
    for (u32 j = 0; j < L; ++j) acc += s[j] * Vp[(u64)j * a.ldk + off + tid];
    a.O[(u64)i * a.D + off + tid] = acc;
}

/* Causal depthwise conv (taps rows: taps-1 history rows + the row itself, no bias) + LN + SiLU,
 * one workgroup per output row: reference src/kernels.metal:359-409. */
extern "C" __global__ __launch_bounds__(256) void dwconv_ln_silu(const NkDwArgs a) {
    __shared__ float red[4];
    const u32 t = blockIdx.x, tid = threadIdx.x;
    const int per = (int)((a.D + NK_LN_THREADS - 1) / NK_LN_THREADS);
    const float *din = a.din;
    if (a.desc) din += (u64)((u32)a.desc[NK_DESC_POS] - (a.taps - 1)) * a.D;
    float v[NK_LN_MAX_PER];
    for (int k = 0; k < per; ++k) {
        const u32 ch = tid + k * NK_LN_THREADS;
        float acc = 0.0f;
        if (ch < a.D)
            for (u32 tap = 0; tap < a.taps; ++tap) acc += a.W[ch * a.taps + tap] * din[(u64)(t + tap) * a.D + ch];
        v[k] = acc;
    }
    ln_regs(v, per, a.D, a.eps, a.g, a.b, red);
    for (int k = 0; k < per; ++k) {
        const u32 ch = tid + k * NK_LN_THREADS;
        if (ch < a.D) a.Y[(u64)t * a.D + ch] = silu_f(v[k]);
    }
}

/* Subsampling conv 0: 1 -> C channels, 3x3, stride 2, causal padding (2 before, 1 after) on
 * time and frequency, + bias, ReLU.  X [T][F] -> Y [T1][F1][C].  One thread per output, channel
 * fastest.  Reference src/kernels.metal:411-432. */
extern "C" __global__ __launch_bounds__(256) void conv2d_c1_s2_relu(const NkConvArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    const u64 total = (u64)a.T1 * a.F1 * a.C;
    if (idx >= total) return;
    const u32 o = (u32)(idx % a.C), f1 = (u32)((idx / a.C) % a.F1), t1 = (u32)(idx / ((u64)a.C * a.F1));
    float acc = a.bias[o];
    for (u32 kh = 0; kh < 3; ++kh) {
        const int ti = (int)(2 * t1 + kh) - 2;
        if (ti < 0 || ti >= (int)a.T) continue;
        for (u32 kw = 0; kw < 3; ++kw) {
            const int fi = (int)(2 * f1 + kw) - 2;
            if (fi < 0 || fi >= (int)a.F) continue;
            acc += a.W[o * 9 + kh * 3 + kw] * a.X[(u64)ti * a.F + fi];
        }
    }
    a.Y[idx] = fmaxf(acc, 0.0f);
}

/* Depthwise 3x3 stride-2 conv, same causal padding, + bias, no activation:
 * reference src/kernels.metal:434-454.  X [T][F][C] -> Y [T1][F1][C]. */
extern "C" __global__ __launch_bounds__(256) void dwconv2d_s2(const NkConvArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    const u64 total = (u64)a.T1 * a.F1 * a.C;
    if (idx >= total) return;
    const u32 c = (u32)(idx % a.C), f1 = (u32)((idx / a.C) % a.F1), t1 = (u32)(idx / ((u64)a.C * a.F1));
    float acc = a.bias[c];
    for (u32 kh = 0; kh < 3; ++kh) {
        const int ti = (int)(2 * t1 + kh) - 2;
        if (ti < 0 || ti >= (int)a.T) continue;
        for (u32 kw = 0; kw < 3; ++kw) {
            const int fi = (int)(2 * f1 + kw) - 2;
            if (fi < 0 || fi >= (int)a.F) continue;
            acc += a.W[c * 9 + kh * 3 + kw] * a.X[((u64)ti * a.F + fi) * a.C + c];
        }
    }
    a.Y[idx] = acc;
}

/* [T][F][C] -> [T][C*F] channel-major flatten: reference src/kernels.metal:456-462.
 * One thread per output element (reads gather, writes are coalesced). */
extern "C" __global__ __launch_bounds__(256) void flatten_cf(const NkFlatArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    const u64 total = (u64)a.T * a.C * a.F;
    if (idx >= total) return;
    const u32 f = (u32)(idx % a.F), c = (u32)((idx / a.F) % a.C), t = (u32)(idx / ((u64)a.F * a.C));
    a.Y[idx] = a.X[((u64)t * a.F + f) * a.C + c];
}

extern "C" __global__ __launch_bounds__(256) void copy_f32(const NkCopyArgs a) {
    const u32 i = blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.dst[i] = a.src[i];
}

extern "C" __global__ __launch_bounds__(256) void fill_f32(const NkFillArgs a) {
    const u32 i = blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.dst[i] = a.value;
}

/* Epoch compaction of the per-layer caches in one launch (reference src/encoder.c:230-240 issues
 * one copy per layer and cache).  grid = (ceil(rows*cols/256), nbuf).  Source and destination rows
 * never overlap (the host checks src_row >= dst_row + rows). */
extern "C" __global__ __launch_bounds__(256) void compact_rows(const NkCompactArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (u64)a.rows * a.cols) return;
    float *b = a.base + (u64)blockIdx.y * a.stride;
    b[(u64)a.dst_row * a.cols + idx] = b[(u64)a.src_row * a.cols + idx];
}

/* LSTM cell, gates [4H] in order i, f, g, o: reference src/kernels.metal:474-486. */
extern "C" __global__ __launch_bounds__(256) void lstm_cell(const NkLstmArgs a) {
    const u32 i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.H) return;
    const float ig = sigmoid_f(a.gates[i]);
    const float fg = sigmoid_f(a.gates[a.H + i]);
    const float gg = tanhf(a.gates[2 * a.H + i]);
    const float og = sigmoid_f(a.gates[3 * a.H + i]);
    const float c = fg * a.c_in[i] + ig * gg;
    a.c_out[i] = c;
    a.h_out[i] = og * tanhf(c);
}

/* RNNT joint, stage 1 (reference src/kernels.metal:488-519): r = relu(enc[row] + pred) in LDS;
 * wavefront w of workgroup g scores vocabulary rows n = g*4 + w (mod G*4) and keeps the best,
 * lowest index on ties.  grid = (NK_JOINT_GROUPS, rows), block = 256. */
extern "C" __global__ __launch_bounds__(256) void joint_partial(const NkJointArgs a) {
    __shared__ float r[NK_JOINT_MAX_H];
    const u32 g = blockIdx.x, G = gridDim.x, row = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const float *e = a.enc + (u64)(a.enc_row + row) * a.enc_ld;
    for (u32 i = tid; i < a.H; i += 256) r[i] = fmaxf(e[i] + a.pred[i], 0.0f);
    __syncthreads();
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    const u32 npair = a.H >> 1;
    for (u32 n = g * NK_JOINT_WAVES + wave; n < a.V; n += G * NK_JOINT_WAVES) {
        const u32 *w2 = (const u32 *)(a.W + (u64)n * a.H);
        float acc = 0.0f;
        for (u32 k = lane; k < npair; k += 64) {
            const u32 w = w2[k];
            acc += r[2 * k] * bf_lo(w);
            acc += r[2 * k + 1] * bf_hi(w);
        }
        acc = wave_sum(acc) + a.bias[n];
        if (acc > bv || (acc == bv && (int)n < bi)) { bv = acc; bi = (int)n; }
    }
    if (lane == 0) {
        const u32 slot = row * G * NK_JOINT_WAVES + g * NK_JOINT_WAVES + wave;
        a.part_v[slot] = bv;
        a.part_i[slot] = bi;
    }
}

/* RNNT joint, stage 2 (reference src/kernels.metal:521-550): reduce n partial bests of one row,
 * same tie rule; out[2*row] = index, out[2*row+1] = value bits.  grid = rows, block = 256. */
extern "C" __global__ __launch_bounds__(256) void argmax_reduce(const NkArgmaxArgs a) {
    __shared__ float bestv[256];
    __shared__ int besti[256];
    const u32 row = blockIdx.x, tid = threadIdx.x;
    const float *pv = a.part_v + (u64)row * a.n;
    const int *pi = a.part_i + (u64)row * a.n;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (u32 i = tid; i < a.n; i += 256)
        if (pv[i] > bv || (pv[i] == bv && pi[i] < bi)) { bv = pv[i]; bi = pi[i]; }
    bestv[tid] = bv;
    besti[tid] = bi;
    __syncthreads();
    for (u32 st = 128; st > 0; st >>= 1) {
        if (tid < st) {
            const float ov = bestv[tid + st];
            const int oi = besti[tid + st];
            if (ov > bestv[tid] || (ov == bestv[tid] && oi < besti[tid])) { bestv[tid] = ov; besti[tid] = oi; }
        }
        __syncthreads();
    }
    if (tid == 0) {
        a.out[2 * row] = besti[0];
        a.out[2 * row + 1] = __float_as_int(bestv[0]);
    }
}

/* Strided row copy: rows x cols floats from src (row stride src_ld) to dst (row stride dst_ld).
 * Used for the row select of the subsampled window and for activation dumps. */
extern "C" __global__ __launch_bounds__(256) void copy2d_f32(const NkCopy2dArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (u64)a.rows * a.cols) return;
    const u32 r = (u32)(idx / a.cols), c = (u32)(idx % a.cols);
    a.dst[(u64)r * a.dst_ld + c] = a.src[(u64)r * a.src_ld + c];
}
