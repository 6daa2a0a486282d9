/* bf16-weight GEMMs for gfx950 with the fused epilogue of the reference
 * (bias, SiLU / ReLU, GLU pairing, alpha scale, accumulate into C).
 *
 *   gemm_fr_*: 5 <= M <= 16 rows (M <= 4 uses the GEMV of nk_gemv.hip).
 *       v_mfma_f32_16x16x32_bf16 with the activations split into bf16 hi + lo (two MFMAs per
 *       step; hi + lo keeps 16 significant bits, so the product error stays near f32 summation
 *       error).  Weights go straight from HBM into the B operand (16 bytes per lane); the
 *       wavefronts of a workgroup split K and sum in a fixed order.  Replaces gemm_mma
 *       (reference src/kernels.metal:120-208).
 *   gemm_mr: M > 16 rows (subsampling 1x1 convs, position table).  64x64 output tiles, both
 *       operands staged through LDS per 32-wide K step, same hi/lo split.
 */
#include "nk_common.h"

/* ---- few-row MFMA GEMM ---------------------------------------------------------------------
 * grid = ceil(nout / 16) workgroups of W wavefronts; a workgroup owns 16 output columns (GLU: 16
 * output pairs; the LayerNorm-fused GLU kernels 8 pairs, grid ceil(nout / 8)) and all of K.  Wavefront w takes the K steps [S*w/W, S*(w+1)/W) of the S = K/32
 * steps (at most FR_SPW).  Order of work:
 *   1. every weight load of the wavefront is issued (16 bytes per lane per step, straight into the
 *      B operand layout);
 *   2. activations: rows < M are read into the A operand layout, from LDS after a workgroup
 *      LayerNorm (the _ln kernels, K <= 1024) or straight from global memory;
 *   3. per step two MFMAs, A = hi + lo bf16 split of the f32 activations (16 significant bits);
 *   4. the W partial tiles are summed in wavefront order through LDS; wavefront 0 applies the
 *      epilogue (or, with K split over workgroups, writes its share's partial rows).
 * MFMA 16x16x32 bf16 lane layouts (lane l, element i):
 *   A: row l % 16, k 8*(l/16) + i;  B: k 8*(l/16) + i, column l % 16;
 *   D: row 4*(l/16) + i, column l % 16. */

/* LayerNorm of one row of 1024 floats held by a wavefront as four float4 per lane (float4 index
 * lane + 64 j): mean = sum/D; var = sum((x-mean)^2)/D; y = (x-mean) * (1/sqrt(var+eps)) * g + b. */
__device__ __forceinline__ void ln_wave4(floatx4 (&v)[4], const floatx4 (&g)[4], const floatx4 (&b)[4], float D,
                                         float eps) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) s += ((v[j][0] + v[j][1]) + v[j][2]) + v[j][3];
    const float mean = wsum(s) / D;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const floatx4 d = v[j] - mean;
        q += ((d[0] * d[0] + d[1] * d[1]) + d[2] * d[2]) + d[3] * d[3];
    }
    const float inv = 1.0f / sqrtf(wsum(q) / D + eps);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[j][e] = (v[j][e] - mean) * inv * g[j][e] + b[j][e];
}

/* grid = (ceil(nout/16), KS): workgroup (tile, ks) takes the K steps [ks*S/KS, (ks+1)*S/KS) of the
 * S = K/32 steps, wavefront w the SPW steps from w*SPW within them.  With KS > 1 (the host uses it
 * only for residual updates: accumulate, no bias, no activation, identity rows) every workgroup
 * writes its share as partial rows, which are added to C in share order afterwards (by resid_fold,
 * or by the LayerNorm prologue of the GEMM that reads C next), so no result depends on which
 * workgroup finishes first.
 * FOLD (with LNA): the activation rows are A plus a pending residual update,
 * A + alpha * (((0 + p0) + p1) + ...) with at most FR_FOLD_PARTS partial rows, formed by each
 * wavefront for the rows it normalises (the order and form of resid_fold); workgroup (0, 0) writes
 * them to fold_out when it is set.  The LayerNorm parameters pass through LDS (sP) in every LNA
 * variant, so that they load with the rows (and the parts) without holding registers through the
 * fold. */
#define FR_FOLD_PARTS 4
/* PK (GLU only): a workgroup owns 8 output pairs, whose value and gate weight rows share one
 * 16-column B operand (columns 0-7 values, 8-15 gates), so there is one MFMA pair per step and
 * twice the workgroups; the epilogue takes each gate sum from lane ^ 8.  Every output's value and
 * gate sums are the same expressions in the same order as with 16 pairs in two operands. */
template <int W, int SPW, bool LNA, bool GLU, bool FOLD = false, bool PK = false>
__device__ __forceinline__ void fr_impl(const NkGemmArgs &a, float *sA, floatx4 *sred, floatx4 *sP = nullptr) {
    static_assert(!FOLD || LNA, "the fold feeds the LayerNorm prologue");
    static_assert(!PK || GLU, "packed pairs are a GLU layout");
    constexpr bool G2 = GLU && !PK; /* value and gate rows in two B operands */
    constexpr int RPW = 16 / W; /* LayerNorm rows per wavefront: wave, wave + W, ... */
    const u32 tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const u32 nout = GLU ? a.N / 2 : a.N;
    const u32 n0 = blockIdx.x * (PK ? 8 : 16);
    const u32 S = a.K >> 5, M = a.M, KS = gridDim.y;
    const u32 Sw = S / KS, s0 = blockIdx.y * Sw;
    /* this wavefront's K steps: [sb, sb + ns), ns <= SPW (wave-uniform) */
    const u32 sb = s0 + wave * SPW;
    const u32 ns = wave * SPW < Sw ? min((u32)SPW, Sw - wave * SPW) : 0u;
    const u32 m = lane & 15, kq = 8 * (lane >> 4);
    const bool mrow = m < M;

    /* LayerNorm variant: wavefront w normalises rows w, w + W, ... (those below M).  Its parameters
     * are loaded once per workgroup and pass through LDS (sP): loaded by every wavefront they were
     * 128 KB of cache reads per workgroup queued ahead of its weights (0.4 us per launch) */
    floatx4 v[LNA ? RPW : 1][4], g1[4], b1[4], g2[4], b2[4];
    floatx4 fp[FOLD ? RPW : 1][FOLD ? FR_FOLD_PARTS : 1][4];
    if constexpr (LNA) {
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const u32 r = min(wave + W * i, M - 1);
#pragma unroll
            for (int j = 0; j < 4; ++j) v[i][j] = ((const floatx4 *)(a.A + (u64)r * a.lda))[lane + 64 * j];
            if constexpr (FOLD) {
#pragma unroll
                for (int h = 0; h < FR_FOLD_PARTS; ++h)
                    if ((u32)h < a.fold_n)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            fp[i][h][j] = ((const floatx4 *)(a.fold + ((u64)h * M + r) * a.K))[lane + 64 * j];
            }
        }
    }
    /* this thread's float4 c = tid % 256 of two parameters: g1 and g2 (wavefronts 0-3) or b1 and b2
     * (wavefronts 4-7); the choice is per wavefront (a scalar branch) */
    floatx4 pq[LNA ? 2 : 1];
    if constexpr (LNA) {
        const u32 c = tid & 255;
        const bool two = a.ln_mode == 2;
        if (wave < 4) {
            pq[0] = ((const floatx4 *)a.ln_g1)[c];
            pq[1] = ((const floatx4 *)(two ? a.ln_g2 : a.ln_g1))[c];
        } else {
            pq[0] = ((const floatx4 *)a.ln_b1)[c];
            pq[1] = ((const floatx4 *)(two ? a.ln_b2 : a.ln_b1))[c];
        }
    }

    /* activations in the A layout (row m of lane l; lanes of rows past M load nothing and are
     * masked at use) */
    float x[LNA ? 1 : SPW][8];
    if constexpr (!LNA) {
        if (mrow) {
            const float *arow = a.A + (u64)m * a.lda + kq;
#pragma unroll
            for (int s = 0; s < SPW; ++s) {
                const u32 t = min(sb + s, S - 1);
                const floatx4 p = *(const floatx4 *)(arow + (u64)t * 32), q = *(const floatx4 *)(arow + (u64)t * 32 + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) { x[s][e] = p[e]; x[s][4 + e] = q[e]; }
            }
        }
    }

    /* epilogue operands (the host always passes bias and the row map), loaded by every
     * wavefront: lane l owns output rows 4*(l/16)+i, column n0 + l%16 */
    const u32 c16 = lane & 15;
    u32 col = n0 + (PK ? (c16 & 7) : c16);
    if (col >= nout) col = nout - 1;
    const bool gate_lane = PK && c16 >= 8;
    const u32 wrow = gate_lane ? col + a.N / 2 : col; /* this lane's B column's weight row */
    const float eba = a.bias[col];
    const float ebb = GLU ? a.bias[col + a.N / 2] : 0.0f;
    int erow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32 r = 4 * (lane >> 4) + i;
        erow[i] = a.crow[r < M ? r : 0];
    }
    __builtin_amdgcn_sched_barrier(0); /* keep the small loads ahead of the weight stream */

    /* 1. weights: every step of this wavefront (steps past K re-read the last one) */
    const u16 *wa = a.W + (u64)wrow * a.ldw + kq;
    const u16 *wb = G2 ? a.W + (u64)(col + a.N / 2) * a.ldw + kq : wa;
    uint4 fa[SPW], fb[G2 ? SPW : 1];
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        const u32 t = min(sb + s, S - 1);
        fa[s] = ld_nt16(wa + (u64)t * 32);
        if constexpr (G2) fb[s] = ld_nt16(wb + (u64)t * 32);
    }
    __builtin_amdgcn_sched_barrier(0);

    /* the C values to accumulate into */
    float ec[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ec[i] = a.C[(u64)(u32)erow[i] * a.ldc + col];

    /* 2. LayerNorm of the activation rows into LDS while the weights stream in */
    if constexpr (LNA) {
        static_assert(W == 8, "the parameter staging assumes 512 threads");
        /* sP: g1 [0, 256), b1 [256, 512), g2 [512, 768), b2 [768, 1024) */
        sP[tid] = pq[0];
        sP[(tid & 255) + (wave < 4 ? 512 : 768)] = pq[1];
        __syncthreads();
    }
    if constexpr (LNA) {
        const float D = (float)a.K;
        const bool write1 = a.ln_out && blockIdx.x == 0 && blockIdx.y == 0;
        if constexpr (FOLD) {
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                const u32 r = wave + W * i;
                if (r >= M) continue;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    floatx4 t = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
                    for (int h = 0; h < FR_FOLD_PARTS; ++h)
                        if ((u32)h < a.fold_n) {
                            t.x += fp[i][h][j].x; t.y += fp[i][h][j].y; t.z += fp[i][h][j].z; t.w += fp[i][h][j].w;
                        }
                    floatx4 x = v[i][j];
                    x.x = x.x + t.x * a.fold_alpha; x.y = x.y + t.y * a.fold_alpha;
                    x.z = x.z + t.z * a.fold_alpha; x.w = x.w + t.w * a.fold_alpha;
                    v[i][j] = x;
                }
                if (a.fold_out && blockIdx.x == 0 && blockIdx.y == 0)
#pragma unroll
                    for (int j = 0; j < 4; ++j) ((floatx4 *)(a.fold_out + (u64)r * a.lda))[lane + 64 * j] = v[i][j];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            g1[j] = sP[lane + 64 * j];
            b1[j] = sP[256 + lane + 64 * j];
            g2[j] = sP[512 + lane + 64 * j];
            b2[j] = sP[768 + lane + 64 * j];
        }
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const u32 r = wave + W * i;
            if (r < M) {
                ln_wave4(v[i], g1, b1, D, a.ln_eps);
                if (write1)
#pragma unroll
                    for (int j = 0; j < 4; ++j) ((floatx4 *)(a.ln_out + (u64)r * a.lda))[lane + 64 * j] = v[i][j];
                if (a.ln_mode == 2) ln_wave4(v[i], g2, b2, D, a.ln_eps);
#pragma unroll
                for (int j = 0; j < 4; ++j) ((floatx4 *)(sA + (u64)r * 1024))[lane + 64 * j] = v[i][j];
            }
        }
        lds_barrier();
    }

    /* 3. MFMAs: A = hi + lo */
    floatx4 acc_a = { 0.f, 0.f, 0.f, 0.f }, acc_b = acc_a;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        if ((u32)s < ns) {
            uint4 ah, al;
            if constexpr (LNA) {
                const float *sp = sA + (u64)m * 1024 + (sb + s) * 32 + kq;
                const floatx4 p = *(const floatx4 *)sp, q = *(const floatx4 *)(sp + 4);
                const float xs[8] = { p[0], p[1], p[2], p[3], q[0], q[1], q[2], q[3] };
                split8(xs, ah, al);
            } else {
                split8(x[s], ah, al);
            }
            if (!mrow) ah = al = make_uint4(0, 0, 0, 0);
            acc_a = mfma_bf16(ah, fa[s], acc_a);
            acc_a = mfma_bf16(al, fa[s], acc_a);
            if constexpr (G2) {
                acc_b = mfma_bf16(ah, fb[s], acc_b);
                acc_b = mfma_bf16(al, fb[s], acc_b);
            }
        }
    }

    /* 4. wavefront partials summed in order; epilogue on wavefront 0 */
    sred[wave * 64 + lane] = acc_a;
    if constexpr (G2) sred[(W + wave) * 64 + lane] = acc_b;
    __syncthreads();
    if (wave != 0) return;
    /* the gate sums: the second operand's partials, or (PK) lane ^ 8's column of the same ones */
    const u32 goff = PK ? (lane ^ 8u) : W * 64 + lane;
    floatx4 ta = sred[lane], tb = GLU ? sred[goff] : acc_b;
#pragma unroll
    for (int w = 1; w < W; ++w) {
        ta += sred[w * 64 + lane];
        if constexpr (GLU) tb += sred[w * 64 + goff];
    }
    if (KS > 1) {
        /* K split over workgroups (residual updates: no bias, no activation, identity rows): this
         * share's sums go to partial rows P[ks][row][n] (rows of nout floats); the host folds them
         * into C in ks order afterwards (resid_fold) */
        if (n0 + (lane & 15) >= nout) return;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32 r = 4 * (lane >> 4) + i;
            if (r < M) a.ws[((u64)blockIdx.y * M + r) * nout + col] = ta[i];
        }
        return;
    }
    if (gate_lane || n0 + (PK ? c16 : (lane & 15)) >= nout) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32 r = 4 * (lane >> 4) + i;
        if (r >= M) continue;
        float *dst = a.C + (u64)(u32)erow[i] * a.ldc + col;
        float v;
        if constexpr (GLU) {
            v = (ta[i] + eba) * sigmoid_f(tb[i] + ebb) * a.alpha;
        } else {
            v = ta[i] + eba;
            if (a.act == NK_ACT_SILU) v = silu_f(v);
            else if (a.act == NK_ACT_RELU) v = fmaxf(v, 0.0f);
            v *= a.alpha;
        }
        *dst = a.accumulate ? ec[i] + v : v;
    }
}

/* gemm_fr_w{W}s{SPW}: W wavefronts of SPW K steps each per workgroup */
#define GEMM_FR(NAME, W, SPW, GLU)                                                                       \
    extern "C" __global__ __launch_bounds__(64 * W) void NAME(const NkGemmArgs a) {                      \
        __shared__ floatx4 sred[2 * W * 64];                                                             \
        fr_impl<W, SPW, false, GLU>(a, nullptr, sred);                                                   \
    }
GEMM_FR(gemm_fr_w4s2, 4, 2, false)
GEMM_FR(gemm_fr_w4s8, 4, 8, false)
GEMM_FR(gemm_fr_w8s8, 8, 8, false)
GEMM_FR(gemm_fr_w16s8, 16, 8, false)
GEMM_FR(gemm_fr_w16s9, 16, 9, false)
GEMM_FR(gemm_fr_glu_w4s8, 4, 8, true)

/* LayerNorm prologue variants: K == 1024, M <= 16; 8 wavefronts (two rows each for the LayerNorm
 * and the fold), four K steps each; _glu8: GLU with packed pairs (8 outputs per workgroup); _f:
 * with the pending-update fold */
#define GEMM_FR_LN(NAME, GLU, FOLD)                                                                      \
    extern "C" __global__ __launch_bounds__(512) void NAME(const NkGemmArgs a) {                         \
        __shared__ float sA[16 * 1024];                                                                  \
        __shared__ floatx4 sred[8 * 64];                                                                 \
        __shared__ floatx4 sP[1024];                                                                     \
        fr_impl<8, 4, true, GLU, FOLD, GLU>(a, sA, sred, sP);                                            \
    }
GEMM_FR_LN(gemm_fr_ln_w8s4, false, false)
GEMM_FR_LN(gemm_fr_ln_glu8_w8s4, true, false)
GEMM_FR_LN(gemm_fr_ln_w8s4_f, false, true)
GEMM_FR_LN(gemm_fr_ln_glu8_w8s4_f, true, true)

/* ---- many-row MFMA GEMM ---------------------------------------------------------------------
 * grid = (ceil(N / 64), ceil(M / 64)), block = 256 (2 x 2 wavefronts, 32 x 32 outputs each).
 * act GLU is not supported here (the host checks). */
extern "C" __global__ __launch_bounds__(256) void gemm_mr(const NkGemmArgs a) {
    __shared__ uint4 sAh[64 * 4], sAl[64 * 4], sW[64 * 4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const u32 m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int wm = wave >> 1, wn = wave & 1;
    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (floatx4){ 0.f, 0.f, 0.f, 0.f };
    const u32 lr = tid >> 2, lu = tid & 3;
    const u32 am = m0 + lr;
    u32 wn_row = n0 + lr;
    if (wn_row >= a.N) wn_row = a.N - 1;
    const float *arow = a.A + (u64)(am < a.M ? am : 0) * a.lda + 8 * lu;
    const u16 *wrow = a.W + (u64)wn_row * a.ldw + 8 * lu;
    for (u32 k0 = 0; k0 < a.K; k0 += 32) {
        uint4 hi = make_uint4(0, 0, 0, 0), lo = hi;
        if (am < a.M) {
            const float4 *ap = (const float4 *)(arow + k0);
            const float4 x = ap[0], y = ap[1];
            const float v[8] = { x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w };
            u32 h[8], q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) split_bf16(v[i], h[i], q[i]);
            hi = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
            lo = make_uint4(q[0] | (q[1] << 16), q[2] | (q[3] << 16), q[4] | (q[5] << 16), q[6] | (q[7] << 16));
        }
        const uint4 w = *(const uint4 *)(wrow + k0);
        sAh[lr * 4 + lu] = hi;
        sAl[lr * 4 + lu] = lo;
        sW[lr * 4 + lu] = w;
        __syncthreads();
#pragma unroll
        for (int tm = 0; tm < 2; ++tm) {
            const u32 ar = wm * 32 + tm * 16 + (lane & 15);
            const uint4 ah = sAh[ar * 4 + (lane >> 4)], al = sAl[ar * 4 + (lane >> 4)];
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                const u32 br = wn * 32 + tn * 16 + (lane & 15);
                const uint4 b = sW[br * 4 + (lane >> 4)];
                acc[tm][tn] = mfma_bf16(ah, b, acc[tm][tn]);
                acc[tm][tn] = mfma_bf16(al, b, acc[tm][tn]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int tm = 0; tm < 2; ++tm)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const u32 col = n0 + wn * 32 + tn * 16 + (lane & 15);
            if (col >= a.N) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32 row = m0 + wm * 32 + tm * 16 + 4 * (lane >> 4) + i;
                if (row < a.M) epi_store(a, row, col, acc[tm][tn][i]);
            }
        }
}
