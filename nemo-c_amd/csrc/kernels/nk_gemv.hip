/* Weight-streaming GEMV for M <= 4 rows (the 80 ms single-stream path and the RNNT decoder):
 * C[crow[m]][n] (= or +=) alpha * act(sum_k A'[m][k] W[n][k] + bias[n]), act GLU pairs rows
 * n, n+N/2.  The host always passes bias and crow (zeros / identity rows when the call has none).
 *
 * A wavefront owns NC weight rows (GLU: NC/2 output pairs); lane l streams the 16-byte chunks l,
 * l+64, ... (KCH per row) of each row, so every load instruction of a wavefront reads 1 KB of
 * contiguous weights.  Memory operations are issued in this order, all unconditionally (indices
 * past the end are clamped to a valid address and their values masked at use), so that the
 * in-order load counter never makes a small load wait for the weight stream:
 *   1. the epilogue row map and bias;
 *   2. the lane's activation chunks of every row, and the LayerNorm parameters;
 *   3. every weight load of the wavefront;
 *   4. the C values to accumulate into.
 * The optional LayerNorm prologue (K <= 1024; ln_mode 1: A' = LN(A; g1,b1); 2: A' =
 * LN(LN(A; g1,b1); g2,b2)) runs on each wavefront from the chunks it holds while the weights are
 * in flight (two DPP reductions per LayerNorm, no barriers).  With ln_out set, wavefront 0 of
 * workgroup 0 also writes LN(A; g1,b1) there: the residual stream after a block's output norm
 * (reference src/encoder.c:180-187).  Dot products are finished with DPP row rotations plus four
 * lane reads, and lanes 0..M*outputs-1 each store one output.
 *
 * Instantiated for R <= 2 at every K up to 4608, for R = 3, 4 at K <= 1024, and for R = 5..8 with
 * one weight row per wavefront at K <= 1024 (the 1024-row matrices of 7-row chunks).
 * Replaces gemm_spec (reference src/kernels.metal:51-118) plus the layernorm / layernorm2
 * launches in front of it (src/encoder.c:155, :159, :169, :177, :180-186). */
#include "nk_common.h"

/* In-register LayerNorm of one row spread over the wavefront: v[q][e] is element 8*(lane+64q)+e,
 * zero for chunks past the row.  mean = sum/D; var = sum((x-mean)^2)/D;
 * y = (x-mean) * (1/sqrt(var+eps)) * g + b. */
template <int KCH>
__device__ __forceinline__ void ln_row_wave(float (&v)[KCH][8], const float (&g)[KCH][8], const float (&b)[KCH][8],
                                            u32 lane, u32 nch, u32 D, float eps) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < KCH; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[q][e];
    const float mean = wsum(s) / (float)D;
    float ss = 0.0f;
#pragma unroll
    for (int q = 0; q < KCH; ++q)
        if (lane + 64 * q < nch)
#pragma unroll
            for (int e = 0; e < 8; ++e) { const float d = v[q][e] - mean; ss += d * d; }
    const float inv = 1.0f / sqrtf(wsum(ss) / (float)D + eps);
#pragma unroll
    for (int q = 0; q < KCH; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[q][e] = (v[q][e] - mean) * inv * g[q][e] + b[q][e];
}

__device__ __forceinline__ void ld8(float (&d)[8], const float *p) {
    const floatx4 x = ((const floatx4 *)p)[0], y = ((const floatx4 *)p)[1];
    d[0] = x[0]; d[1] = x[1]; d[2] = x[2]; d[3] = x[3]; d[4] = y[0]; d[5] = y[1]; d[6] = y[2]; d[7] = y[3];
}

/* FOLD (K <= 1024, LayerNorm prologue): the activation rows are A plus a pending residual update,
 * formed by the workgroup in xs (R rows of K floats) before the LayerNorm; the partial rows are
 * loaded ahead of the weight stream, the sums finished after it is issued, one barrier. */
template <int R, int NC, int KCH, bool FOLD = false>
__device__ __forceinline__ void gemv_impl(const NkGemmArgs &a, float *xs = nullptr) {
    const u32 lane = threadIdx.x & 63;
    const u32 gw = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const bool glu = a.act == NK_ACT_GLU;
    const u32 nout = glu ? a.N / 2 : a.N;
    constexpr int NP = NC / 2 > 0 ? NC / 2 : 1; /* GLU output pairs per wavefront */
    const u32 per_wave = glu ? (u32)NP : (u32)NC;
    const u32 j0 = gw * per_wave;
    /* uniform per wavefront; without FOLD the kernel has no barriers, with it the wavefronts past
     * the end leave after the fold's barrier */
    const bool live = j0 < nout;
    if (!FOLD && !live) return;
    const u32 nch = a.K >> 3, M = a.M;

    /* 0. FOLD: this thread's float4 column c4 = tid (K <= 1024) of every row: A and the parts */
    constexpr int FP = 8; /* parts held in registers per pass */
    floatx4 fa[FOLD ? R : 1], fp[FOLD ? R : 1][FOLD ? FP : 1];
    const u32 c4 = threadIdx.x, k4 = a.K >> 2;
    if constexpr (FOLD) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const u32 rr = (u32)r < M ? r : 0, cc = c4 < k4 ? c4 : 0;
            fa[r] = ((const floatx4 *)(a.A + (u64)rr * a.lda))[cc];
#pragma unroll
            for (int h = 0; h < FP; ++h)
                fp[r][h] = (u32)h < a.fold_n ? ((const floatx4 *)(a.fold + ((u64)h * M + rr) * a.K))[cc]
                                            : (floatx4){ 0.f, 0.f, 0.f, 0.f };
        }
    }

    /* 1. epilogue row map and bias: lane e < M*outputs owns output (r = e / per_wave, column
     *    j0 + e % per_wave); other lanes read a clamped (valid) entry and store nothing */
    const u32 er = lane / per_wave, ecol = j0 + lane % per_wave;
    const bool e_ok = lane < (u32)R * per_wave && er < M && ecol < nout;
    const u32 er_c = e_ok ? er : 0, ecol_c = e_ok ? ecol : j0;
    const int e_row = a.crow[er_c];
    const float e_ba = a.bias[ecol_c];
    const float e_bb = glu ? a.bias[ecol_c + a.N / 2] : 0.0f;

    /* 2. activation chunks (rows past M read row 0) and LayerNorm parameters */
    float x[R][KCH][8];
    if constexpr (!FOLD) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int q = 0; q < KCH; ++q) {
                const u32 j = min(lane + 64 * q, nch - 1);
                ld8(x[r][q], a.A + (u64)((u32)r < M ? r : 0) * a.lda + 8 * j);
            }
    }
    float g1[KCH <= 2 ? KCH : 1][8], b1[KCH <= 2 ? KCH : 1][8], g2[KCH <= 2 ? KCH : 1][8], b2[KCH <= 2 ? KCH : 1][8];
    if constexpr (KCH <= 2) {
        if (a.ln_mode) {
#pragma unroll
            for (int q = 0; q < KCH; ++q) {
                const u32 j = min(lane + 64 * q, nch - 1);
                ld8(g1[q], a.ln_g1 + 8 * j);
                ld8(b1[q], a.ln_b1 + 8 * j);
                ld8(g2[q], (a.ln_mode == 2 ? a.ln_g2 : a.ln_g1) + 8 * j);
                ld8(b2[q], (a.ln_mode == 2 ? a.ln_b2 : a.ln_b1) + 8 * j);
            }
        }
    }

    __builtin_amdgcn_sched_barrier(0); /* keep the small loads ahead of the weight stream */

    /* 3. weight rows of this wavefront */
    uint4 w[NC][KCH];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (FOLD && !live) break;
        u32 row;
        if (glu) row = (c < NP) ? j0 + c : j0 + (c - NP) + a.N / 2;
        else row = j0 + c;
        if (glu ? (c < NP ? j0 + c >= nout : j0 + (c - NP) >= nout) : row >= a.N) row = glu ? j0 : a.N - 1;
        const u16 *wr = a.W + (u64)row * a.ldw;
#pragma unroll
        for (int q = 0; q < KCH; ++q) w[c][q] = ld_nt16(wr + 8 * (u64)min(lane + 64 * q, nch - 1));
    }

    __builtin_amdgcn_sched_barrier(0);

    /* 4. the C value to accumulate into */
    float *e_dst = a.C + (u64)(u32)e_row * a.ldc + ecol_c;
    const float e_c = a.accumulate && live ? *e_dst : 0.0f;

    if constexpr (FOLD) {
        /* x = A + alpha * (((0 + p0) + p1) + ...), the order and form of resid_fold; parts past
         * FP are read here (after the weight stream is issued) */
        if (c4 < k4) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if ((u32)r >= M) break;
                floatx4 t = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
                for (int h = 0; h < FP; ++h)
                    if ((u32)h < a.fold_n) { t.x += fp[r][h].x; t.y += fp[r][h].y; t.z += fp[r][h].z; t.w += fp[r][h].w; }
                for (u32 h = FP; h < a.fold_n; ++h) {
                    const floatx4 q = ((const floatx4 *)(a.fold + ((u64)h * M + r) * a.K))[c4];
                    t.x += q.x; t.y += q.y; t.z += q.z; t.w += q.w;
                }
                floatx4 v = fa[r];
                v.x = v.x + t.x * a.fold_alpha; v.y = v.y + t.y * a.fold_alpha;
                v.z = v.z + t.z * a.fold_alpha; v.w = v.w + t.w * a.fold_alpha;
                ((floatx4 *)(xs + r * 1024))[c4] = v;
                if (blockIdx.x == 0 && a.fold_out) ((floatx4 *)(a.fold_out + (u64)r * a.lda))[c4] = v;
            }
        }
        __syncthreads();
        if (!live) return;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int q = 0; q < KCH; ++q) {
                const u32 j = min(lane + 64 * q, nch - 1);
                ld8(x[r][q], xs + ((u32)r < M ? r : 0) * 1024 + 8 * j);
            }
    }

    /* chunks past the row contribute nothing (selects, so no register is rewritten while its
     * load is in flight) */
#pragma unroll
    for (int q = 0; q < KCH; ++q) {
        const bool ok = lane + 64 * q < nch;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int e = 0; e < 8; ++e) x[r][q][e] = ok ? x[r][q][e] : 0.0f;
    }

    if constexpr (KCH <= 2) {
        if (a.ln_mode) {
#pragma unroll
            for (int q = 0; q < KCH; ++q) {
                const bool ok = lane + 64 * q < nch;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    g1[q][e] = ok ? g1[q][e] : 0.0f;
                    b1[q][e] = ok ? b1[q][e] : 0.0f;
                    g2[q][e] = ok ? g2[q][e] : 0.0f;
                    b2[q][e] = ok ? b2[q][e] : 0.0f;
                }
            }
            const bool write1 = a.ln_out && gw == 0;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if ((u32)r >= M) break;
                ln_row_wave<KCH>(x[r], g1, b1, lane, nch, a.K, a.ln_eps);
                if (write1)
#pragma unroll
                    for (int q = 0; q < KCH; ++q) {
                        const u32 j = lane + 64 * q;
                        if (j < nch) {
                            floatx4 *o = (floatx4 *)(a.ln_out + (u64)r * a.lda + 8 * j);
                            o[0] = (floatx4){ x[r][q][0], x[r][q][1], x[r][q][2], x[r][q][3] };
                            o[1] = (floatx4){ x[r][q][4], x[r][q][5], x[r][q][6], x[r][q][7] };
                        }
                    }
                if (a.ln_mode == 2) ln_row_wave<KCH>(x[r], g2, b2, lane, nch, a.K, a.ln_eps);
            }
        }
    }

    /* 5. dot products */
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            float s = 0.0f;
#pragma unroll
            for (int q = 0; q < KCH; ++q) s = dot8(x[r][q], w[c][q], s);
            acc[r][c] = s;
        }

    /* 6. reductions and the fused epilogue */
    float mine_a = 0.0f, mine_b = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if ((u32)r >= M) break;
        if (glu) {
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const float sa = wsum(acc[r][p]);
                const float sb = wsum(acc[r][p + (NC > 1 ? NP : 0)]);
                if (lane == (u32)(r * NP + p)) { mine_a = sa; mine_b = sb; }
            }
        } else {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float s = wsum(acc[r][c]);
                if (lane == (u32)(r * NC + c)) mine_a = s;
            }
        }
    }
    if (!e_ok) return;
    float v;
    if (glu) {
        v = (mine_a + e_ba) * sigmoid_f(mine_b + e_bb) * a.alpha;
    } else {
        v = mine_a + e_ba;
        if (a.act == NK_ACT_SILU) v = silu_f(v);
        else if (a.act == NK_ACT_RELU) v = fmaxf(v, 0.0f);
        v *= a.alpha;
    }
    *e_dst = a.accumulate ? (e_c + v) : v;
}

#define GEMV2(R, NC, KCH) \
    extern "C" __global__ __launch_bounds__(256) void gemv_r##R##_n##NC##_k##KCH(const NkGemmArgs a) { gemv_impl<R, NC, KCH>(a); }
#define GEMV2_R(R)                                                                                             \
    GEMV2(R, 1, 1) GEMV2(R, 2, 1) GEMV2(R, 4, 1) GEMV2(R, 1, 2) GEMV2(R, 2, 2) GEMV2(R, 4, 2) GEMV2(R, 1, 4) \
    GEMV2(R, 2, 4) GEMV2(R, 4, 4) GEMV2(R, 1, 8) GEMV2(R, 2, 8) GEMV2(R, 1, 9) GEMV2(R, 2, 9)
#define GEMV2_SMALLK(R) GEMV2(R, 1, 1) GEMV2(R, 2, 1) GEMV2(R, 4, 1) GEMV2(R, 1, 2) GEMV2(R, 2, 2) GEMV2(R, 4, 2)
GEMV2_R(1)
GEMV2_R(2)
GEMV2_SMALLK(3)
GEMV2_SMALLK(4)
#define GEMV2_NARROW(R) GEMV2(R, 1, 1) GEMV2(R, 1, 2)
GEMV2_NARROW(5)
GEMV2_NARROW(6)
GEMV2_NARROW(7)
GEMV2_NARROW(8)

/* the FOLD variants (suffix _f): K <= 1024 with the LayerNorm prologue */
#define GEMV2F(R, NC, KCH)                                                                              \
    extern "C" __global__ __launch_bounds__(256) void gemv_r##R##_n##NC##_k##KCH##_f(const NkGemmArgs a) { \
        __shared__ float xs[R * 1024];                                                                  \
        gemv_impl<R, NC, KCH, true>(a, xs);                                                             \
    }
#define GEMV2F_R(R) GEMV2F(R, 1, 1) GEMV2F(R, 2, 1) GEMV2F(R, 4, 1) GEMV2F(R, 1, 2) GEMV2F(R, 2, 2) GEMV2F(R, 4, 2)
GEMV2F_R(1)
GEMV2F_R(2)
GEMV2F_R(3)
GEMV2F_R(4)
