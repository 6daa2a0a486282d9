/* Weight-streaming GEMV for M <= 4 rows (the 80 ms single-stream path and the RNNT decoder):
 * C[m][n] (= or +=) alpha * act(sum_k A'[m][k] W[n][k] + bias[n]), act GLU pairs rows n, n+N/2.
 *
 * Layout: a wavefront owns NC weight rows (GLU: NC/2 output pairs); lane l streams 16-byte chunks
 * l, l+64, ... (KCH per row) of each row, so every load instruction of a wavefront reads 1 KB of
 * contiguous weights.  Per lane, all NC*KCH weight loads, the activation chunks and the
 * epilogue operands (bias, the C values to accumulate into, the output row map) are issued
 * before the first FMA.  Dot products are finished with DPP row rotations plus four lane reads
 * (no LDS), and lanes 0..R*NC-1 each store one output.
 *
 * Instantiated for R <= 2 at every K up to 4608 and for R = 3, 4 at K <= 1024.
 *
 * Optional LayerNorm prologue (K <= 1024) (ln_mode 1: A' = LN(A; g1,b1); 2: A' = LN(LN(A; g1,b1); g2,b2)):
 * valid when K is the row width.  A lane's chunks cover its part of every row, so each
 * wavefront normalises the rows itself from the values it already holds (two DPP reductions per
 * LayerNorm).  With ln_out set, workgroup 0's first wavefront also writes LN(A; g1,b1) there: the
 * residual stream after a block's output norm (reference src/encoder.c:180-187).
 * Replaces gemm_spec (reference src/kernels.metal:51-118) plus the layernorm / layernorm2
 * launches in front of it (src/encoder.c:155, :159, :169, :177, :180-186). */
#include "nk_common.h"

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
#define DPP_QUAD_1032 0xB1 /* quad_perm(1,0,3,2) */
#define DPP_QUAD_2301 0x4E /* quad_perm(2,3,0,1) */
#define DPP_ROW_ROR4 0x124
#define DPP_ROW_ROR8 0x128

/* Sum over the 64 lanes of a wavefront, returned wave-uniform; fixed combination order. */
__device__ __forceinline__ float wsum(float v) {
    v += dpp_f<DPP_QUAD_1032>(v);
    v += dpp_f<DPP_QUAD_2301>(v);
    v += dpp_f<DPP_ROW_ROR4>(v);
    v += dpp_f<DPP_ROW_ROR8>(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

/* In-register LayerNorm of one row spread over the wavefront: v[q][e] is element 8*(lane+64q)+e,
 * valid for chunks j < nch.  mean = sum/D; var = sum((x-mean)^2)/D; y = (x-mean)*inv*g + b. */
template <int KCH>
__device__ __forceinline__ void ln_row_wave(float (&v)[KCH][8], const float (&g)[KCH][8], const float (&b)[KCH][8],
                                            u32 lane, u32 nch, u32 D, float eps) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < KCH; ++q)
        if (lane + 64 * q < nch)
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
    const float4 x = ((const float4 *)p)[0], y = ((const float4 *)p)[1];
    d[0] = x.x; d[1] = x.y; d[2] = x.z; d[3] = x.w; d[4] = y.x; d[5] = y.y; d[6] = y.z; d[7] = y.w;
}

template <int R, int NC, int KCH>
__device__ __forceinline__ void gemv_impl2(const NkGemmArgs &a) {
    const u32 lane = threadIdx.x & 63;
    const u32 gw = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const bool glu = a.act == NK_ACT_GLU;
    const u32 nout = glu ? a.N / 2 : a.N;
    constexpr int NP = NC / 2 > 0 ? NC / 2 : 1; /* GLU output pairs per wavefront */
    const u32 per_wave = glu ? (u32)NP : (u32)NC;
    const u32 j0 = gw * per_wave;
    if (j0 >= nout) return; /* uniform per wavefront */
    const u32 nch = a.K >> 3;

    /* 1. weight rows of this wavefront and their loads */
    const u16 *wr[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        u32 row;
        if (glu) row = (c < NP) ? j0 + c : j0 + (c - NP) + a.N / 2;
        else row = j0 + c;
        if (glu ? (c < NP ? j0 + c >= nout : j0 + (c - NP) >= nout) : row >= a.N) row = glu ? j0 : a.N - 1;
        wr[c] = a.W + (u64)row * a.ldw;
    }
    uint4 w[NC][KCH];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < KCH; ++q) {
            const u32 j = lane + 64 * q;
            w[c][q] = j < nch ? ld_nt16(wr[c] + 8 * (u64)j) : make_uint4(0, 0, 0, 0);
        }

    /* 2. epilogue operands: lane e < R*outputs owns output (r = e / per_wave, column j0 + e % per_wave) */
    const u32 outs = per_wave;
    const u32 er = lane / outs, ec = lane % outs, ecol = j0 + ec;
    const bool e_ok = lane < (u32)R * outs && er < a.M && ecol < nout;
    float e_ba = 0.0f, e_bb = 0.0f, e_c = 0.0f;
    float *e_dst = nullptr;
    if (e_ok) {
        if (a.bias) {
            e_ba = a.bias[ecol];
            if (glu) e_bb = a.bias[ecol + a.N / 2];
        }
        const u32 row = a.crow ? (u32)a.crow[er] : er;
        e_dst = a.C + (u64)row * a.ldc + ecol;
        if (a.accumulate) e_c = *e_dst;
    }

    /* 3. activation chunks (and LayerNorm parameters for the same indices) */
    float x[R][KCH][8];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < KCH; ++q) {
            const u32 j = lane + 64 * q;
            if (j < nch) ld8(x[r][q], a.A + (u64)r * a.lda + 8 * j);
            else
#pragma unroll
                for (int e = 0; e < 8; ++e) x[r][q][e] = 0.0f;
        }
    if constexpr (KCH <= 2) if (a.ln_mode) {
        float g1[KCH][8], b1[KCH][8], g2[KCH][8], b2[KCH][8];
#pragma unroll
        for (int q = 0; q < KCH; ++q) {
            const u32 j = lane + 64 * q;
            if (j < nch) {
                ld8(g1[q], a.ln_g1 + 8 * j);
                ld8(b1[q], a.ln_b1 + 8 * j);
                if (a.ln_mode == 2) { ld8(g2[q], a.ln_g2 + 8 * j); ld8(b2[q], a.ln_b2 + 8 * j); }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) { g1[q][e] = 0.0f; b1[q][e] = 0.0f; g2[q][e] = 0.0f; b2[q][e] = 0.0f; }
            }
        }
        const bool write1 = a.ln_out && blockIdx.x == 0 && (threadIdx.x >> 6) == 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if ((u32)r >= a.M) break;
            ln_row_wave<KCH>(x[r], g1, b1, lane, nch, a.K, a.ln_eps);
            if (write1)
#pragma unroll
                for (int q = 0; q < KCH; ++q) {
                    const u32 j = lane + 64 * q;
                    if (j < nch) {
                        float4 *o = (float4 *)(a.ln_out + (u64)r * a.lda + 8 * j);
                        o[0] = make_float4(x[r][q][0], x[r][q][1], x[r][q][2], x[r][q][3]);
                        o[1] = make_float4(x[r][q][4], x[r][q][5], x[r][q][6], x[r][q][7]);
                    }
                }
        }
        if (a.ln_mode == 2) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if ((u32)r >= a.M) break;
                ln_row_wave<KCH>(x[r], g2, b2, lane, nch, a.K, a.ln_eps);
            }
        }
    }

    /* 4. dot products */
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

    /* 5. reductions and the fused epilogue */
    float mine_a = 0.0f, mine_b = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if ((u32)r >= a.M) break;
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
    extern "C" __global__ __launch_bounds__(256) void gemv_r##R##_n##NC##_k##KCH(const NkGemmArgs a) { gemv_impl2<R, NC, KCH>(a); }
#define GEMV2_R(R)                                                                                                     \
    GEMV2(R, 1, 1) GEMV2(R, 2, 1) GEMV2(R, 4, 1) GEMV2(R, 1, 2) GEMV2(R, 2, 2) GEMV2(R, 4, 2) GEMV2(R, 1, 4)         \
    GEMV2(R, 2, 4) GEMV2(R, 4, 4) GEMV2(R, 1, 8) GEMV2(R, 2, 8) GEMV2(R, 1, 9) GEMV2(R, 2, 9)
#define GEMV2_SMALLK(R) GEMV2(R, 1, 1) GEMV2(R, 2, 1) GEMV2(R, 4, 1) GEMV2(R, 1, 2) GEMV2(R, 2, 2) GEMV2(R, 4, 2)
GEMV2_R(1)
GEMV2_R(2)
GEMV2_SMALLK(3)
GEMV2_SMALLK(4)
