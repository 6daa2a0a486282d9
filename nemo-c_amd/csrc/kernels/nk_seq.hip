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
#ifndef LN_PARTS_AHEAD
#define LN_PARTS_AHEAD 4 /* pending parts whose loads layernorm_rows issues together */
#endif

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
        v[k] = ld4z(x, i, D4);
        g1[k] = ld4z((const float4 *)a.g1, i, D4);
        b1[k] = ld4z((const float4 *)a.b1, i, D4);
        g2[k] = a.Y2 ? ld4z((const float4 *)a.g2, i, D4) : z;
        b2[k] = a.Y2 ? ld4z((const float4 *)a.b2, i, D4) : z;
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

/* One row per wavefront (D <= 1024: lane l holds float4s l, l+64, l+128, l+192), four rows per
 * workgroup: the same LayerNorm (two-pass mean and variance) with wavefront reductions and no
 * barriers, for the batched path's many rows.  Y2 as in layernorm. */
__device__ __forceinline__ void ln_row64(float4 (&v)[4], const float4 (&g)[4], const float4 (&b)[4], u32 lane, u32 D4,
                                         u32 D, float eps) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) s += ((v[k].x + v[k].y) + v[k].z) + v[k].w;
    const float mean = wsum(s) / (float)D;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (lane + 64 * k < D4) {
            const float dx = v[k].x - mean, dy = v[k].y - mean, dz = v[k].z - mean, dw = v[k].w - mean;
            q += ((dx * dx + dy * dy) + dz * dz) + dw * dw;
        }
    const float inv = 1.0f / sqrtf(wsum(q) / (float)D + eps);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        v[k].x = (v[k].x - mean) * inv * g[k].x + b[k].x;
        v[k].y = (v[k].y - mean) * inv * g[k].y + b[k].y;
        v[k].z = (v[k].z - mean) * inv * g[k].z + b[k].z;
        v[k].w = (v[k].w - mean) * inv * g[k].w + b[k].w;
    }
}

/* R consecutive rows per wavefront (the rows' loads issued together, the LayerNorm parameters
 * loaded once for all R); each row's arithmetic is ln_row64's, so every R gives the same bits.
 * Only R = 1 is launched: with the guarded per-lane loads of an earlier form, 2 and 4 rows per
 * wavefront paid at thousands of rows, but with the full-width loads below one row per wavefront
 * is fastest at every size (3584 rows x 1024, graph-replayed: 7.6 / 8.1 / 8.3 us for R = 1 / 2 / 4
 * with no pending update, 12.6 / 13.5 / 15.6 with one part, 20.5 / 21.6 / 23.1 with four).
 * FULL: D = 1024, every lane holds four float4s of the row, so no load or store needs a per-lane
 * guard (a guarded 16-byte load costs a branch, and a guarded use lets the compiler move the load
 * behind that branch, after the previous loads have been waited for).
 * A pending update's first LN_PARTS_AHEAD parts are loaded before any of them is summed (one
 * memory round trip instead of one per part): part min(b, nparts - 1) is loaded for every b, and
 * the parts past nparts add +0, which leaves the sum's bits unchanged (the running sum starts at
 * +0 and, as a sum of at least two terms one of which is +0, is never -0). */
template <int R, bool FULL>
__device__ __forceinline__ void layernorm_rows_impl(const NkLnArgs &a) {
    const u32 lane = threadIdx.x & 63, D4 = FULL ? 256 : a.D >> 2;
    const u32 r0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (r0 >= a.M) return; /* uniform per wavefront; no barriers */
    float4 v[R][4], g1[4], b1[4], g2[4], b2[4];
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    auto ld = [&](const float4 *p, u32 i) { return FULL ? p[i] : ld4z(p, i, D4); };
    auto in_row = [&](u32 i) { return FULL || i < D4; };
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float4 *x = (const float4 *)(a.X + (u64)min(r0 + r, a.M - 1) * a.D);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[r][k] = ld(x, lane + 64 * k);
    }
    if (a.P) {
        /* pending residual update: x + palpha * (((0 + p0) + p1) + ...), written back to X (this
         * wavefront owns its rows); the host sets P only with nparts >= 1 */
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const u32 row = min(r0 + r, a.M - 1);
            float4 t[4] = { z, z, z, z };
            float4 q[LN_PARTS_AHEAD][4];
#pragma unroll
            for (u32 b = 0; b < LN_PARTS_AHEAD; ++b) {
                const float4 *p = (const float4 *)(a.P + ((u64)min(b, a.nparts - 1) * a.M + row) * a.D);
#pragma unroll
                for (int k = 0; k < 4; ++k) q[b][k] = ld(p, lane + 64 * k);
            }
#pragma unroll
            for (u32 b = 0; b < LN_PARTS_AHEAD; ++b) {
                const bool use = b < a.nparts;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    t[k].x += use ? q[b][k].x : 0.0f;
                    t[k].y += use ? q[b][k].y : 0.0f;
                    t[k].z += use ? q[b][k].z : 0.0f;
                    t[k].w += use ? q[b][k].w : 0.0f;
                }
            }
            for (u32 b = LN_PARTS_AHEAD; b < a.nparts; ++b) {
                const float4 *p = (const float4 *)(a.P + ((u64)b * a.M + row) * a.D);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 w = ld(p, lane + 64 * k);
                    t[k].x += w.x; t[k].y += w.y; t[k].z += w.z; t[k].w += w.w;
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[r][k].x = v[r][k].x + t[k].x * a.palpha;
                v[r][k].y = v[r][k].y + t[k].y * a.palpha;
                v[r][k].z = v[r][k].z + t[k].z * a.palpha;
                v[r][k].w = v[r][k].w + t[k].w * a.palpha;
            }
            if (r0 + r < a.M) {
                float4 *x = (float4 *)(a.X + (u64)row * a.D);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (in_row(lane + 64 * k)) x[lane + 64 * k] = v[r][k];
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const u32 i = lane + 64 * k;
        g1[k] = ld((const float4 *)a.g1, i);
        b1[k] = ld((const float4 *)a.b1, i);
        g2[k] = a.Y2 ? ld((const float4 *)a.g2, i) : z;
        b2[k] = a.Y2 ? ld((const float4 *)a.b2, i) : z;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const u32 row = r0 + r;
        if (row >= a.M) break;
        ln_row64(v[r], g1, b1, lane, D4, a.D, a.eps);
        u16 *ys = a.Ys ? a.Ys + (u64)row * 2 * a.D : nullptr;
        if (!a.Y2 && ys) {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (in_row(lane + 64 * k)) store_split4(ys, a.D, 4 * (lane + 64 * k), v[r][k]);
            continue;
        }
        float4 *y1 = (float4 *)(a.Y1 + (u64)row * a.D);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (in_row(lane + 64 * k)) y1[lane + 64 * k] = v[r][k];
        if (!a.Y2) continue;
        ln_row64(v[r], g2, b2, lane, D4, a.D, a.eps);
        if (ys) {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (in_row(lane + 64 * k)) store_split4(ys, a.D, 4 * (lane + 64 * k), v[r][k]);
            continue;
        }
        float4 *y2 = (float4 *)(a.Y2 + (u64)row * a.D);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (in_row(lane + 64 * k)) y2[lane + 64 * k] = v[r][k];
    }
}
template <int R> __device__ __forceinline__ void layernorm_rows_any(const NkLnArgs &a) {
    if (a.D == 1024) layernorm_rows_impl<R, true>(a);
    else layernorm_rows_impl<R, false>(a);
}
extern "C" __global__ __launch_bounds__(256) void layernorm_rows(const NkLnArgs a) { layernorm_rows_any<1>(a); }

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
 * (reference src/kernels.metal:290-348), on fp32 matrix cores (v_mfma_f32_16x16x4f32: fp32
 * products and sums, so results equal the vector-unit ones up to summation order).  One workgroup
 * per (head, chunk); the chunk's c <= 16 query rows are one 16-row tile:
 *   S1 = (Q + u) K^T   [16][80]  five 16-column tiles over the L <= 80 keys
 *   S2 = (Q + v) P^T   [16][96]  six tiles over the chunk's L + c - 1 position rows
 *   score(i, j) = (S1[i][j] + S2[i][c - 1 - i + j]) * scale,  softmax over j < L
 *   O = softmax . V    [16][128] eight tiles
 * The eleven score tiles are spread over the four wavefronts; a lane reads its K or P row (32
 * consecutive dims of the row) straight from global memory and holds its query row's matching 32
 * dims of q + u and q + v in registers (step s of the K loop is dim 32 (lane / 16) + s on both
 * operands).  V goes to LDS by direct loads (granule g of row r at slot g ^ (r % 16), so the
 * column reads of the P.V product are conflict-free); scores and probabilities go through LDS. */
#define ATC_SLD 97 /* score row stride in floats: 96 position columns + 1 */
extern "C" __global__ __launch_bounds__(256) void attention_rel_chunks(const NkAttnChunkArgs a) {
    __shared__ floatx4 Vs[NK_ATTC_MAX_L * 32];
    __shared__ float S1[16 * ATC_SLD], S2[16 * ATC_SLD];
    static_assert(NK_ATTC_MAX_L == 80 && NK_ATTC_MAX_C <= 16, "tile counts assume 80 keys, 16 query rows");
    const u32 h = blockIdx.x, ch = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int *cd = a.chunks + 4 * ch;
    const u32 qrow0 = (u32)cd[0], m0 = (u32)cd[1], c = (u32)cd[2], cl = (u32)cd[3];
    const u32 L = cl + c, NP = L + c - 1;
    if (c == 0 || c > NK_ATTC_MAX_C || L > NK_ATTC_MAX_L || L > a.Lmax) return; /* host-checked */
    const u32 off = h * 128;
    const float *Kg = a.kv + a.D + (u64)(qrow0 - cl) * a.ld + off;
    const float *Vg = a.kv + 2 * a.D + (u64)(qrow0 - cl) * a.ld + off;
    const float *Pg = a.P + (u64)(a.Lmax - L) * a.D + off;
    /* V rows 0 .. 79 into LDS, two rows per direct-load instruction (rows past L re-read row L - 1:
     * finite values, weighted by zero probabilities) */
    for (u32 blk = wave; blk < NK_ATTC_MAX_L / 2; blk += 4) {
        const u32 p = blk * 64 + lane, r = p >> 5, g = (p & 31) ^ (r & 15), rr = min(r, L - 1);
        dma16(Vg + (u64)rr * a.ld + 4 * g, (lds_char_t *)&Vs[blk * 64]);
    }
    /* query row qi = lane % 16 (zero past c), dims 32 kq .. 32 kq + 31 */
    const u32 qi = lane & 15, kq = lane >> 4;
    float qu[32], qv[32];
    {
        const bool ok = qi < c;
        const floatx4 *qp = (const floatx4 *)(a.kv + (u64)(qrow0 + min(qi, c - 1)) * a.ld + off + 32 * kq);
        const floatx4 *up = (const floatx4 *)(a.bu + off + 32 * kq), *vp = (const floatx4 *)(a.bv + off + 32 * kq);
#pragma unroll
        for (int v4 = 0; v4 < 8; ++v4) {
            const floatx4 q = qp[v4], u = up[v4], w = vp[v4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qu[4 * v4 + e] = ok ? q[e] + u[e] : 0.0f;
                qv[4 * v4 + e] = ok ? q[e] + w[e] : 0.0f;
            }
        }
    }
    /* score tiles: T < 5 content (K rows 16 T ..), T >= 5 position (P rows 16 (T - 5) ..) */
    for (u32 T = wave; T < 11; T += 4) {
        const bool pos = T >= 5;
        const u32 col0 = (pos ? T - 5 : T) * 16, row = col0 + qi;
        const floatx4 *src = (const floatx4 *)((pos ? Pg + (u64)min(row, NP - 1) * a.D : Kg + (u64)min(row, L - 1) * a.ld) +
                                               32 * kq);
        float b[32];
#pragma unroll
        for (int v4 = 0; v4 < 8; ++v4) {
            const floatx4 x = src[v4];
#pragma unroll
            for (int e = 0; e < 4; ++e) b[4 * v4 + e] = x[e];
        }
        floatx4 acc = { 0.f, 0.f, 0.f, 0.f };
        if (pos) {
#pragma unroll
            for (int k = 0; k < 32; ++k) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[k], b[k], acc, 0, 0, 0);
        } else {
#pragma unroll
            for (int k = 0; k < 32; ++k) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qu[k], b[k], acc, 0, 0, 0);
        }
        float *S = pos ? S2 : S1;
#pragma unroll
        for (int r = 0; r < 4; ++r) S[(4 * kq + r) * ATC_SLD + col0 + qi] = acc[r];
    }
    wait_vm_lgkm<0>();
    barrier_mem();
    /* scores and softmax: wavefront w takes rows w, w + 4, ...; lane takes keys lane, lane + 64;
     * the probabilities replace S1 (zero for rows past c and keys past L) */
    for (u32 i = wave; i < 16; i += 4) {
        const u32 j0 = lane, j1 = lane + 64;
        if (i < c) {
            const bool v0 = j0 < L, v1 = j1 < L;
            const float s0 = v0 ? (S1[i * ATC_SLD + j0] + S2[i * ATC_SLD + (c - 1 - i + j0)]) * a.scale : -INFINITY;
            const float s1 = v1 ? (S1[i * ATC_SLD + j1] + S2[i * ATC_SLD + (v1 ? c - 1 - i + j1 : 0)]) * a.scale : -INFINITY;
            const float mx = wave_max(fmaxf(s0, s1));
            const float e0 = v0 ? expf(s0 - mx) : 0.0f, e1 = v1 ? expf(s1 - mx) : 0.0f;
            const float sum = wave_sum(e0 + e1);
            S1[i * ATC_SLD + j0] = e0 / sum;
            if (j1 < NK_ATTC_MAX_L) S1[i * ATC_SLD + j1] = e1 / sum;
        } else {
            S1[i * ATC_SLD + j0] = 0.0f;
            if (j1 < NK_ATTC_MAX_L) S1[i * ATC_SLD + j1] = 0.0f;
        }
    }
    lds_barrier();
    /* O = P V: wavefront w takes output column tiles w and w + 4; step s of the K loop is key
     * 20 (lane / 16) + s on both operands */
    for (u32 dt = wave; dt < 8; dt += 4) {
        const u32 d = dt * 16 + qi, gq = d >> 2, e = d & 3;
        floatx4 acc = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
        for (u32 k = 0; k < NK_ATTC_MAX_L / 4; ++k) {
            const u32 j = (NK_ATTC_MAX_L / 4) * kq + k;
            const float pa = S1[qi * ATC_SLD + j];
            const float vb = ((const float *)&Vs[j * 32 + (gq ^ (j & 15))])[e];
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vb, acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const u32 i = 4 * kq + r;
            if (i < c) {
                if (a.Os) store_split1(a.Os + (u64)(m0 + i) * 2 * a.D, a.D, off + d, acc[r]);
                else a.O[(u64)(m0 + i) * a.D + off + d] = acc[r];
            }
        }
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
        if (tid + k * 256 < D4) {
            const float4 o = make_float4(silu_f(v[k].x), silu_f(v[k].y), silu_f(v[k].z), silu_f(v[k].w));
            if (a.Ys) store_split4(a.Ys + (u64)t * 2 * a.D, a.D, 4 * (tid + k * 256), o);
            else y[tid + k * 256] = o;
        }
}
