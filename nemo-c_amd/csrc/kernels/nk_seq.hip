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

/* Relative-position attention of one (head h, query row orow) on a workgroup of 512 threads:
 * reference src/kernels.metal:290-348.
 *   score_j = ((q + u) . K_j + (q + v) . P[(Lmax - L) + (c - 1 - i + j)]) * scale
 *   O_i = sum_j softmax(score)_j V_j  (no mask inside the chunk)
 * Scores: four threads per key (32 head dims each), one key per thread quad (L <= 128).
 * Output: thread (g = tid / 32, d4 = tid % 32) accumulates dims 4*d4..4*d4+3 over the keys
 * j = g (mod 16); the 16 key groups are summed in order through LDS.  Every K, P and V load is
 * issued at the start (indices past the window clamped to a valid row and masked at use), then
 * after_loads() (a fused caller's own loads, so that the waits for K, P and V never wait for
 * them); the barriers wait for LDS only, so the V loads stay in flight through the score phase.
 * Returns dims 4 tid .. 4 tid + 3 of the head's output row on threads tid < 32. */
struct AttnShared {
    floatx4 qu4[32], qv4[32];
    float s[NK_ATT_MAX_L], red[16];
    floatx4 part[16][32];
};

template <class F>
__device__ __forceinline__ floatx4 attn_rel_core(const NkAttnArgs &a, u32 h, u32 orow, AttnShared &sh, F &&after_loads) {
    const u32 tid = threadIdx.x;
    const u32 off = h * 128;
    const float *Q = a.Q, *Kp = a.K, *Vp = a.V;
    u32 L = a.L, i = orow, c = a.c;
    if (a.rows) { /* batched streams: this row's stream window */
        const u32 qrow = (u32)a.rows[4 * orow], cl = (u32)a.rows[4 * orow + 3];
        i = (u32)a.rows[4 * orow + 1];
        c = (u32)a.rows[4 * orow + 2];
        Q += (u64)(qrow - i) * a.ldq;
        Kp += (u64)(qrow - i - cl) * a.ldk;
        Vp += (u64)(qrow - i - cl) * a.ldk;
        L = cl + c;
    } else if (a.desc) {
        const u32 pos = (u32)a.desc[NK_DESC_POS], cl = (u32)a.desc[NK_DESC_CACHE];
        Q += (u64)pos * a.ldq;
        Kp += (u64)(pos - cl) * a.ldk;
        Vp += (u64)(pos - cl) * a.ldk;
        L = cl + a.c;
    }
    /* q + u, q + v for this head */
    floatx4 qx = { 0.f, 0.f, 0.f, 0.f }, ux = qx, vx = qx;
    if (tid < 32) {
        qx = *(const floatx4 *)(Q + (u64)i * a.ldq + off + 4 * tid);
        ux = *(const floatx4 *)(a.bu + off + 4 * tid);
        vx = *(const floatx4 *)(a.bv + off + 4 * tid);
    }
    /* K and P rows of this thread's key: key ks = tid / 4, dims part4*32 .. +32; lanes past the
     * window issue no load (their values are never used) */
    const u32 ks = tid >> 2, part4 = tid & 3, dofs = off + part4 * 32;
    const bool kin = ks < L;
    const u32 prow = (a.Lmax - L) + (c - 1 - i + ks);
    floatx4 kr[8], pr[8];
    if (kin) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            kr[q] = *(const floatx4 *)(Kp + (u64)ks * a.ldk + dofs + 4 * q);
            pr[q] = *(const floatx4 *)(a.P + (u64)prow * a.D + dofs + 4 * q);
        }
    }
    /* V rows for the output phase: group vg = tid / 32 takes keys vg, vg + 16, ... */
    const u32 vg = tid >> 5, d4 = tid & 31;
    floatx4 vv[NK_ATT_MAX_L / 16];
#pragma unroll
    for (int t = 0; t < NK_ATT_MAX_L / 16; ++t)
        if (vg + 16 * t < L) vv[t] = *(const floatx4 *)(Vp + (u64)(vg + 16 * t) * a.ldk + off + 4 * d4);
    __builtin_amdgcn_sched_barrier(0);
    after_loads();
    __builtin_amdgcn_sched_barrier(0);
    if (tid < 32) {
        sh.qu4[tid] = qx + ux;
        sh.qv4[tid] = qx + vx;
    }
    lds_barrier();
    float acc = 0.0f;
    if (kin) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const floatx4 u = sh.qu4[part4 * 8 + q], w = sh.qv4[part4 * 8 + q];
            acc += u[0] * kr[q][0] + u[1] * kr[q][1] + u[2] * kr[q][2] + u[3] * kr[q][3];
            acc += w[0] * pr[q][0] + w[1] * pr[q][1] + w[2] * pr[q][2] + w[3] * pr[q][3];
        }
    }
    acc += dpp_f<DPP_QUAD_1032>(acc);
    acc += dpp_f<DPP_QUAD_2301>(acc);
    if (part4 == 0 && kin) sh.s[ks] = acc * a.scale;
    lds_barrier();
    /* softmax over the window (threads 0..127 hold one score each) */
    const int lane = tid & 63, wave = tid >> 6;
    const float sv = tid < L ? sh.s[tid] : -INFINITY;
    float mx = wmax(sv);
    if (wave < 2 && lane == 0) sh.red[wave] = mx;
    lds_barrier();
    mx = fmaxf(sh.red[0], sh.red[1]);
    const float ev = tid < L ? expf(sv - mx) : 0.0f;
    float sum = wsum(ev);
    if (wave < 2 && lane == 0) sh.red[2 + wave] = sum;
    lds_barrier();
    sum = sh.red[2] + sh.red[3];
    if (tid < L) sh.s[tid] = ev / sum;
    lds_barrier();
    floatx4 o = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
    for (int t = 0; t < NK_ATT_MAX_L / 16; ++t) {
        const u32 j = vg + 16 * t;
        if (j < L) o += sh.s[j] * vv[t];
    }
    sh.part[vg][d4] = o;
    lds_barrier();
    floatx4 r = { 0.f, 0.f, 0.f, 0.f };
    if (tid < 32) {
        r = sh.part[0][tid];
#pragma unroll
        for (int g = 1; g < 16; ++g) r += sh.part[g][tid];
    }
    return r;
}

/* one workgroup of 512 threads per (head, query row) */
extern "C" __global__ __launch_bounds__(512) void attention_rel(const NkAttnArgs a) {
    __shared__ AttnShared sh;
    const floatx4 r = attn_rel_core(a, blockIdx.x, blockIdx.y, sh, [] {});
    if (threadIdx.x < 32) *(floatx4 *)(a.O + (u64)blockIdx.y * a.D + blockIdx.x * 128 + 4 * threadIdx.x) = r;
}

/* Relative-position attention of whole chunks (batched streams), the math of attention_rel above
 * (reference src/kernels.metal:290-348).  One workgroup per (head, chunk): the chunk's L = cached
 * + c keys and values and its L + c - 1 position rows are brought into LDS by direct global -> LDS
 * loads (16 bytes per lane, granule g of row r stored at slot g ^ (r % 16), so the row-parallel
 * 16-byte reads below, 16 lanes per cycle, are conflict-free), then every query row of the chunk is scored against
 * them: wavefront w takes rows w, w+4, ...; lane l takes keys l and l+64; softmax by wavefront
 * reductions; output lane l accumulates dims 2l, 2l+1 over the keys in order. */
extern "C" __global__ __launch_bounds__(256) void attention_rel_chunks(const NkAttnChunkArgs a) {
    __shared__ floatx4 Ks[NK_ATTC_MAX_L * 32], Vs[NK_ATTC_MAX_L * 32];
    __shared__ floatx4 Ps[(NK_ATTC_MAX_L + NK_ATTC_MAX_C) * 32];
    __shared__ floatx4 qu[NK_ATTC_MAX_C * 32], qv[NK_ATTC_MAX_C * 32];
    __shared__ float sc[NK_ATTC_MAX_C][NK_ATTC_MAX_L];
    const u32 h = blockIdx.x, ch = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int *cd = a.chunks + 4 * ch;
    const u32 qrow0 = (u32)cd[0], m0 = (u32)cd[1], c = (u32)cd[2], cl = (u32)cd[3];
    const u32 L = cl + c, NP = L + c - 1;
    if (c == 0 || c > NK_ATTC_MAX_C || L > NK_ATTC_MAX_L || L > a.Lmax) return; /* host-checked */
    const u32 off = h * 128;
    const float *Kg = a.kv + a.D + (u64)(qrow0 - cl) * a.ld + off;
    const float *Vg = a.kv + 2 * a.D + (u64)(qrow0 - cl) * a.ld + off;
    const float *Pg = a.P + (u64)(a.Lmax - L) * a.D + off;
    /* LDS granule p = 32 r + s of a table holds granule s ^ (r % 8) of row r; one DMA instruction
     * fills 64 granules (two rows); rows past the end re-read the last row (never used) */
    for (u32 blk = wave; blk < (L + 1) / 2; blk += 4) {
        const u32 p = blk * 64 + lane, r = p >> 5, g = (p & 31) ^ (r & 15), rr = min(r, L - 1);
        dma16(Kg + (u64)rr * a.ld + 4 * g, (lds_char_t *)&Ks[blk * 64]);
        dma16(Vg + (u64)rr * a.ld + 4 * g, (lds_char_t *)&Vs[blk * 64]);
    }
    for (u32 blk = wave; blk < (NP + 1) / 2; blk += 4) {
        const u32 p = blk * 64 + lane, r = p >> 5, g = (p & 31) ^ (r & 15), rr = min(r, NP - 1);
        dma16(Pg + (u64)rr * a.D + 4 * g, (lds_char_t *)&Ps[blk * 64]);
    }
    for (u32 idx = tid; idx < c * 32; idx += 256) {
        const u32 i = idx >> 5, g = idx & 31;
        const floatx4 q = *(const floatx4 *)(a.kv + (u64)(qrow0 + i) * a.ld + off + 4 * g);
        qu[idx] = q + *(const floatx4 *)(a.bu + off + 4 * g);
        qv[idx] = q + *(const floatx4 *)(a.bv + off + 4 * g);
    }
    wait_vm_lgkm<0>();
    barrier_mem();
    const u32 j0 = lane, j1 = lane + 64;
    for (u32 i = wave; i < c; i += 4) {
        /* position row of (i, j): (Lmax - L) + (c - 1 - i + j), i.e. row c - 1 - i + j of Ps */
        const u32 p0 = c - 1 - i + j0, p1 = c - 1 - i + j1;
        float s0 = 0.0f, s1 = 0.0f;
        if (j0 < L) {
#pragma unroll 8
            for (u32 g = 0; g < 32; ++g) {
                const floatx4 u = qu[i * 32 + g], w = qv[i * 32 + g];
                const floatx4 k = Ks[j0 * 32 + (g ^ (j0 & 15))], pp = Ps[p0 * 32 + (g ^ (p0 & 15))];
                s0 += u[0] * k[0] + u[1] * k[1] + u[2] * k[2] + u[3] * k[3];
                s0 += w[0] * pp[0] + w[1] * pp[1] + w[2] * pp[2] + w[3] * pp[3];
            }
        }
        if (j1 < L) {
#pragma unroll 8
            for (u32 g = 0; g < 32; ++g) {
                const floatx4 u = qu[i * 32 + g], w = qv[i * 32 + g];
                const floatx4 k = Ks[j1 * 32 + (g ^ (j1 & 15))], pp = Ps[p1 * 32 + (g ^ (p1 & 15))];
                s1 += u[0] * k[0] + u[1] * k[1] + u[2] * k[2] + u[3] * k[3];
                s1 += w[0] * pp[0] + w[1] * pp[1] + w[2] * pp[2] + w[3] * pp[3];
            }
        }
        s0 = j0 < L ? s0 * a.scale : -INFINITY;
        s1 = j1 < L ? s1 * a.scale : -INFINITY;
        const float mx = wave_max(fmaxf(s0, s1));
        const float e0 = j0 < L ? expf(s0 - mx) : 0.0f, e1 = j1 < L ? expf(s1 - mx) : 0.0f;
        const float sum = wave_sum(e0 + e1);
        if (j0 < L) sc[i][j0] = e0 / sum;
        if (j1 < L) sc[i][j1] = e1 / sum;
    }
    lds_barrier();
    const u32 gq = lane >> 1, hf = (lane & 1) * 2;
    for (u32 i = wave; i < c; i += 4) {
        float o0 = 0.0f, o1 = 0.0f;
        for (u32 j = 0; j < L; ++j) {
            const float pj = sc[i][j];
            const floatx4 v = Vs[j * 32 + (gq ^ (j & 15))];
            o0 += pj * v[hf];
            o1 += pj * v[hf + 1];
        }
        *(floatx2 *)(a.O + (u64)(m0 + i) * a.D + off + 2 * lane) = (floatx2){ o0, o1 };
    }
}

/* Causal depthwise conv (9 taps: 8 history rows + the row itself, no bias) + LN + SiLU, one
 * workgroup per output row: reference src/kernels.metal:359-409.  Thread t owns channels
 * 4t..4t+3 (+1024k); all 9 input rows and the 4x9 taps are loaded up front. */
#define DW_TAPS 9
extern "C" __global__ __launch_bounds__(256) void dwconv_ln_silu(const NkDwArgs a) {
    __shared__ float red[4];
    const u32 t = blockIdx.x, tid = threadIdx.x, D4 = a.D >> 2;
    const float *din = a.din;
    if (a.rows) din += ((long long)a.rows[4 * t] - (DW_TAPS - 1) - (long long)t) * (long long)a.D;
    else if (a.desc) din += (u64)((u32)a.desc[NK_DESC_POS] - (DW_TAPS - 1)) * a.D;
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
