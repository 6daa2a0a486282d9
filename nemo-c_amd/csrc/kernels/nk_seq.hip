/* Latency-bound per-row kernels of the chunk for gfx950: LayerNorm (single and paired),
 * relative-position attention and causal depthwise conv + LN + SiLU.  Each kernel issues every
 * global load it needs before its first use (activations, gammas, betas, conv taps, K/V/P rows),
 * so a launch costs about one memory round trip plus its reductions. */
#include "nk_common.h"

/* Block-wide sum over 256 threads (4 wavefronts), combined in wavefront order.  `red` holds 4
 * floats; the leading barrier protects it from the previous call's readers. */
__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

#define LN_VEC 4 /* float4 per thread: D <= 4096 */

/* LayerNorm of a row held as float4s (reference src/kernels.metal:257-288):
 * mean = sum/D, var = sum((x-mean)^2)/D, inv = 1/sqrt(var + eps), y = (x-mean)*inv*g + b. */
__device__ __forceinline__ void ln_vec(float4 *v, const float4 *g, const float4 *b, u32 D4, u32 D, float eps, float *red) {
    const u32 tid = threadIdx.x;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < LN_VEC; ++k)
        if (tid + k * 256 < D4) s += ((v[k].x + v[k].y) + v[k].z) + v[k].w;
    const float mean = block_sum256(s, red) / (float)D;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < LN_VEC; ++k)
        if (tid + k * 256 < D4) {
            const float dx = v[k].x - mean, dy = v[k].y - mean, dz = v[k].z - mean, dw = v[k].w - mean;
            q += ((dx * dx + dy * dy) + dz * dz) + dw * dw;
        }
    const float var = block_sum256(q, red);
    const float inv = 1.0f / sqrtf(var / (float)D + eps);
#pragma unroll
    for (int k = 0; k < LN_VEC; ++k) {
        v[k].x = (v[k].x - mean) * inv * g[k].x + b[k].x;
        v[k].y = (v[k].y - mean) * inv * g[k].y + b[k].y;
        v[k].z = (v[k].z - mean) * inv * g[k].z + b[k].z;
        v[k].w = (v[k].w - mean) * inv * g[k].w + b[k].w;
    }
}

/* One workgroup per row. Y1 = LN(X; g1,b1); with Y2 set, also Y2 = LN(Y1; g2,b2)
 * (norm_out of a block paired with norm_feed_forward1 of the next, src/kernels.metal:210-255). */
extern "C" __global__ __launch_bounds__(256) void layernorm(const NkLnArgs a) {
    __shared__ float red[4];
    const u32 row = blockIdx.x, tid = threadIdx.x, D4 = a.D >> 2;
    const float4 *x = (const float4 *)(a.X + (u64)row * a.D);
    float4 v[LN_VEC], g1[LN_VEC], b1[LN_VEC], g2[LN_VEC], b2[LN_VEC];
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < LN_VEC; ++k) {
        const u32 i = tid + k * 256;
        const bool ok = i < D4;
        v[k] = ok ? x[i] : z;
        g1[k] = ok ? ((const float4 *)a.g1)[i] : z;
        b1[k] = ok ? ((const float4 *)a.b1)[i] : z;
        g2[k] = ok && a.Y2 ? ((const float4 *)a.g2)[i] : z;
        b2[k] = ok && a.Y2 ? ((const float4 *)a.b2)[i] : z;
    }
    ln_vec(v, g1, b1, D4, a.D, a.eps, red);
    float4 *y1 = (float4 *)(a.Y1 + (u64)row * a.D);
#pragma unroll
    for (int k = 0; k < LN_VEC; ++k)
        if (tid + k * 256 < D4) y1[tid + k * 256] = v[k];
    if (!a.Y2) return;
    ln_vec(v, g2, b2, D4, a.D, a.eps, red);
    float4 *y2 = (float4 *)(a.Y2 + (u64)row * a.D);
#pragma unroll
    for (int k = 0; k < LN_VEC; ++k)
        if (tid + k * 256 < D4) y2[tid + k * 256] = v[k];
}

/* Relative-position attention, one workgroup of 256 threads per (head, query):
 * reference src/kernels.metal:290-348.  Four threads share a key (32 head dims each), 64 keys per
 * pass, at most two passes (L <= 128).  Every K, P and V element the workgroup needs is loaded
 * before the first score is formed: V is preloaded per output dim (thread d sums keys of one
 * parity), the scores go through LDS, and the two parities are added at the end.
 *   score_j = ((q + u) . K_j + (q + v) . P[(Lmax - L) + (c - 1 - i + j)]) * scale
 *   O_i = sum_j softmax(score)_j V_j  (no mask inside the chunk) */
extern "C" __global__ __launch_bounds__(256) void attention_rel(const NkAttnArgs a) {
    __shared__ float s[NK_ATT_MAX_L], red[8], half_out[128];
    const u32 h = blockIdx.x, i = blockIdx.y, tid = threadIdx.x;
    const u32 off = h * 128;
    const float *Q = a.Q, *Kp = a.K, *Vp = a.V;
    u32 L = a.L;
    if (a.desc) {
        const u32 pos = (u32)a.desc[NK_DESC_POS], cl = (u32)a.desc[NK_DESC_CACHE];
        Q += (u64)pos * a.ldq;
        Kp += (u64)(pos - cl) * a.ldk;
        Vp += (u64)(pos - cl) * a.ldk;
        L = cl + a.c;
    }
    const u32 ks = tid >> 2, part = tid & 3, dofs = off + part * 32;
    /* V preload: output dim d = tid & 127, keys of parity tid >> 7 */
    const u32 d = tid & 127, par = tid >> 7;
    float vv[NK_ATT_MAX_L / 2];
#pragma unroll
    for (int t = 0; t < NK_ATT_MAX_L / 2; ++t) {
        const u32 j = par + 2 * t;
        vv[t] = j < L ? Vp[(u64)j * a.ldk + off + d] : 0.0f;
    }
    /* K and P rows of this thread's keys */
    float4 kr[2][8], pr[2][8];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const u32 j = ks + 64 * p;
        const bool ok = j < L;
        const u32 prow = (a.Lmax - L) + (a.c - 1 - i + j);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            kr[p][q] = ok ? *(const float4 *)(Kp + (u64)j * a.ldk + dofs + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
            pr[p][q] = ok ? *(const float4 *)(a.P + (u64)prow * a.D + dofs + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float4 qu[8], qv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float4 x = *(const float4 *)(Q + (u64)i * a.ldq + dofs + 4 * q);
        const float4 u = *(const float4 *)(a.bu + dofs + 4 * q), w = *(const float4 *)(a.bv + dofs + 4 * q);
        qu[q] = make_float4(x.x + u.x, x.y + u.y, x.z + u.z, x.w + u.w);
        qv[q] = make_float4(x.x + w.x, x.y + w.y, x.z + w.z, x.w + w.w);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            acc += qu[q].x * kr[p][q].x + qu[q].y * kr[p][q].y + qu[q].z * kr[p][q].z + qu[q].w * kr[p][q].w;
            acc += qv[q].x * pr[p][q].x + qv[q].y * pr[p][q].y + qv[q].z * pr[p][q].z + qv[q].w * pr[p][q].w;
        }
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        const u32 j = ks + 64 * p;
        if (part == 0 && j < L) s[j] = acc * a.scale;
    }
    __syncthreads();
    /* softmax over the window */
    const int lane = tid & 63, wave = tid >> 6;
    const float sv = tid < L ? s[tid] : -INFINITY;
    float mx = wave_max(sv);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float ev = tid < L ? expf(sv - mx) : 0.0f;
    float sum = wave_sum(ev);
    if (lane == 0) red[4 + wave] = sum;
    __syncthreads();
    sum = ((red[4] + red[5]) + red[6]) + red[7];
    if (tid < L) s[tid] = ev / sum;
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < NK_ATT_MAX_L / 2; ++t) {
        const u32 j = par + 2 * t;
        if (j < L) acc += s[j] * vv[t];
    }
    if (par == 1) half_out[d] = acc;
    __syncthreads();
    if (par == 0) a.O[(u64)i * a.D + off + d] = acc + half_out[d];
}

/* Causal depthwise conv (9 taps: 8 history rows + the row itself, no bias) + LN + SiLU, one
 * workgroup per output row: reference src/kernels.metal:359-409.  Thread t owns channels
 * 4t..4t+3 (+1024k); all 9 input rows and the 4x9 taps are loaded up front. */
#define DW_TAPS 9
extern "C" __global__ __launch_bounds__(256) void dwconv_ln_silu(const NkDwArgs a) {
    __shared__ float red[4];
    const u32 t = blockIdx.x, tid = threadIdx.x, D4 = a.D >> 2;
    const float *din = a.din;
    if (a.desc) din += (u64)((u32)a.desc[NK_DESC_POS] - (DW_TAPS - 1)) * a.D;
    float4 v[LN_VEC], g[LN_VEC], b[LN_VEC];
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < LN_VEC; ++k) {
        const u32 c4 = tid + k * 256;
        if (c4 >= D4) { v[k] = g[k] = b[k] = z; continue; }
        float4 x[DW_TAPS], w[DW_TAPS];
#pragma unroll
        for (int tap = 0; tap < DW_TAPS; ++tap) {
            x[tap] = *(const float4 *)(din + (u64)(t + tap) * a.D + 4 * c4);
            w[tap] = *(const float4 *)(a.W + (u64)c4 * 4 * DW_TAPS + 4 * tap); /* taps of channels 4c4.. */
        }
        g[k] = ((const float4 *)a.g)[c4];
        b[k] = ((const float4 *)a.b)[c4];
        /* w holds W[4c4 .. 4c4+3][0..8] flattened: channel e, tap q is element 9e + q */
        const float *wf = (const float *)w;
        float acc[4] = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
        for (int tap = 0; tap < DW_TAPS; ++tap) {
            acc[0] += wf[0 * DW_TAPS + tap] * x[tap].x;
            acc[1] += wf[1 * DW_TAPS + tap] * x[tap].y;
            acc[2] += wf[2 * DW_TAPS + tap] * x[tap].z;
            acc[3] += wf[3 * DW_TAPS + tap] * x[tap].w;
        }
        v[k] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
    ln_vec(v, g, b, D4, a.D, a.eps, red);
    float4 *y = (float4 *)(a.Y + (u64)t * a.D);
#pragma unroll
    for (int k = 0; k < LN_VEC; ++k)
        if (tid + k * 256 < D4)
            y[tid + k * 256] = make_float4(silu_f(v[k].x), silu_f(v[k].y), silu_f(v[k].z), silu_f(v[k].w));
}
