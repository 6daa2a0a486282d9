/* bf16-weight GEMMs for gfx950 with the fused epilogue of the reference
 * (bias, SiLU / ReLU, GLU pairing, alpha scale, accumulate into C).
 *
 *   gemv_r{R}_c{NC}: M = R <= 4 rows.  Pure weight streaming on the VALU: each wavefront owns
 *       NC weight rows, every lane streams 16-byte chunks of those rows (a wavefront reads 1 KB of
 *       contiguous weights per row per pass), activations stay in registers for the pass, and a
 *       64-lane butterfly finishes each dot product.  Replaces gemm_spec
 *       (reference src/kernels.metal:51-118).
 *   gemm_fr: 5 <= M <= 16 rows.  v_mfma_f32_16x16x32_bf16 with the activations split into
 *       bf16 hi + lo (two MFMAs per step; hi + lo keeps 16 significant bits, so the product error
 *       stays near f32 summation error).  A is staged once per workgroup in LDS in fragment order;
 *       weights go straight from HBM into the B operand (16 bytes per lane).  Four wavefronts split
 *       the workgroup's K range; workgroups split K further with a deterministic fixup (the last
 *       arriving workgroup sums the partials in split order).  Replaces gemm_mma
 *       (reference src/kernels.metal:120-208).
 *   gemm_mr: M > 16 rows (subsampling 1x1 convs, position table).  64x64 output tiles, both
 *       operands staged through LDS per 32-wide K step, same hi/lo split.
 */
#include "nk_common.h"

template <int R, int NC, int SEG>
__device__ __forceinline__ void gemv_impl(const NkGemmArgs &a) {
    const int lane = threadIdx.x & 63;
    const u32 gw = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const bool glu = a.act == NK_ACT_GLU;
    const u32 nout = glu ? a.N / 2 : a.N;
    const u32 per_wave = glu ? 1u : (u32)NC;
    const u32 j0 = gw * per_wave;
    if (j0 >= nout) return; /* uniform per wavefront */
    const u16 *wr[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        u32 row = glu ? (c ? j0 + a.N / 2 : j0) : j0 + c;
        if (row >= a.N) row = a.N - 1;
        wr[c] = a.W + (u64)row * a.ldw;
    }
    const u32 nch = a.K >> 3; /* 8-element (16-byte) weight chunks per row */
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;
    for (u32 base = 0; base < nch; base += 64 * SEG) {
        uint4 wv[NC][SEG];
        float av[SEG][R][8];
#pragma unroll
        for (int s = 0; s < SEG; ++s) {
            const u32 j = base + s * 64 + lane;
            const bool ok = j < nch;
#pragma unroll
            for (int c = 0; c < NC; ++c)
                wv[c][s] = ok ? ld_nt16(wr[c] + 8 * (u64)j) : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float4 x = make_float4(0, 0, 0, 0), y = x;
                if (ok) {
                    const float4 *ap = (const float4 *)(a.A + (u64)r * a.lda + 8 * (u64)j);
                    x = ap[0];
                    y = ap[1];
                }
                av[s][r][0] = x.x; av[s][r][1] = x.y; av[s][r][2] = x.z; av[s][r][3] = x.w;
                av[s][r][4] = y.x; av[s][r][5] = y.y; av[s][r][6] = y.z; av[s][r][7] = y.w;
            }
        }
#pragma unroll
        for (int s = 0; s < SEG; ++s)
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][c] = dot8(av[s][r], wv[c][s], acc[r][c]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = wave_sum(acc[r][c]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if ((u32)r >= a.M) break;
            if (glu) {
                if constexpr (NC == 2) epi_store_glu(a, r, j0, acc[r][0], acc[r][1]);
            } else {
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    if (j0 + c < nout) epi_store(a, r, j0 + c, acc[r][c]);
            }
        }
    }
}

#define GEMV(R, NC, SEG) \
    extern "C" __global__ __launch_bounds__(256) void gemv_r##R##_c##NC(const NkGemmArgs a) { gemv_impl<R, NC, SEG>(a); }
GEMV(1, 1, 8)
GEMV(1, 2, 8)
GEMV(2, 1, 4)
GEMV(2, 2, 4)
GEMV(3, 1, 2)
GEMV(3, 2, 2)
GEMV(4, 1, 2)
GEMV(4, 2, 2)

/* ---- few-row MFMA GEMM ---------------------------------------------------------------------
 * grid = (ceil(nout / 16), splits), block = 256.  A workgroup owns 16 output columns and the
 * K steps [sb, se) of its split (se - sb <= NK_FR_MAX_KC / 32).
 * MFMA 16x16x32 bf16 lane layouts (lane l, element i):
 *   A: row l % 16, k 8*(l/16) + i;  B: k 8*(l/16) + i, column l % 16;
 *   D: row 4*(l/16) + i, column l % 16.
 */
#define FR_STEPS (NK_FR_MAX_KC / 32)

__device__ __forceinline__ void fr_epilogue(const NkGemmArgs &a, bool glu, u32 n0, u32 nout, int lane, floatx4 sa, floatx4 sb) {
    const u32 col = n0 + (lane & 15);
    if (col >= nout) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32 r = 4 * (lane >> 4) + i;
        if (r >= a.M) continue;
        if (glu) epi_store_glu(a, r, col, sa[i], sb[i]);
        else epi_store(a, r, col, sa[i]);
    }
}

extern "C" __global__ __launch_bounds__(256) void gemm_fr(const NkGemmArgs a) {
    __shared__ uint4 sA[2][FR_STEPS][64];
    __shared__ floatx4 sred[2][4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool glu = a.act == NK_ACT_GLU;
    const u32 nout = glu ? a.N / 2 : a.N;
    const u32 tile = blockIdx.x, n0 = tile * 16;
    const u32 S = a.splits, ks = blockIdx.y;
    const u32 KS = a.K >> 5;
    const u32 sb = (u32)(((u64)KS * ks) / S), se = (u32)(((u64)KS * (ks + 1)) / S);
    const u32 ns = se - sb;

    /* stage this split's A columns as hi/lo bf16 fragments */
    for (u32 idx = threadIdx.x; idx < ns * 64; idx += 256) {
        const u32 t = idx >> 6, l = idx & 63, m = l & 15;
        const u32 k = (sb + t) * 32 + 8 * (l >> 4);
        uint4 hi = make_uint4(0, 0, 0, 0), lo = hi;
        if (m < a.M) {
            const float4 *ap = (const float4 *)(a.A + (u64)m * a.lda + k);
            const float4 x = ap[0], y = ap[1];
            const float v[8] = { x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w };
            u32 h[8], q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) split_bf16(v[i], h[i], q[i]);
            hi = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
            lo = make_uint4(q[0] | (q[1] << 16), q[2] | (q[3] << 16), q[4] | (q[5] << 16), q[6] | (q[7] << 16));
        }
        sA[0][t][l] = hi;
        sA[1][t][l] = lo;
    }
    __syncthreads();

    u32 col = n0 + (lane & 15);
    if (col >= nout) col = nout - 1;
    const u16 *wa = a.W + (u64)col * a.ldw + 8 * (lane >> 4);
    const u16 *wb = glu ? a.W + (u64)(col + a.N / 2) * a.ldw + 8 * (lane >> 4) : wa;
    const u32 wbeg = ns * wave / 4, wend = ns * (wave + 1) / 4;
    floatx4 acc_a = { 0.f, 0.f, 0.f, 0.f }, acc_b = acc_a;
    uint4 fa[FR_STEPS / 4], fb[FR_STEPS / 4];
#pragma unroll
    for (int s = 0; s < FR_STEPS / 4; ++s) {
        const u32 t = wbeg + s;
        if (t < wend) {
            fa[s] = ld_nt16(wa + (u64)(sb + t) * 32);
            if (glu) fb[s] = ld_nt16(wb + (u64)(sb + t) * 32);
        }
    }
#pragma unroll
    for (int s = 0; s < FR_STEPS / 4; ++s) {
        const u32 t = wbeg + s;
        if (t < wend) {
            const uint4 ah = sA[0][t][lane], al = sA[1][t][lane];
            acc_a = mfma_bf16(ah, fa[s], acc_a);
            acc_a = mfma_bf16(al, fa[s], acc_a);
            if (glu) {
                acc_b = mfma_bf16(ah, fb[s], acc_b);
                acc_b = mfma_bf16(al, fb[s], acc_b);
            }
        }
    }
    sred[0][wave][lane] = acc_a;
    sred[1][wave][lane] = acc_b;
    __syncthreads();
    if (wave != 0) return;
    const floatx4 sa = ((sred[0][0][lane] + sred[0][1][lane]) + sred[0][2][lane]) + sred[0][3][lane];
    const floatx4 sbv = ((sred[1][0][lane] + sred[1][1][lane]) + sred[1][2][lane]) + sred[1][3][lane];
    if (S == 1) {
        fr_epilogue(a, glu, n0, nout, lane, sa, sbv);
        return;
    }
    /* split-K: publish this split's 16x16 partial, the last arriving split reduces in order */
    float *mine = a.ws + ((u64)tile * S + ks) * 512;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        __hip_atomic_store(mine + lane * 4 + i, sa[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(mine + 256 + lane * 4 + i, sbv[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __threadfence();
    u32 prev = 0;
    if (lane == 0) prev = atomicAdd(&a.counters[tile], 1u);
    prev = __shfl(prev, 0, 64);
    if (prev != S - 1) return;
    __threadfence();
    floatx4 ta = { 0.f, 0.f, 0.f, 0.f }, tb = ta;
    for (u32 q = 0; q < S; ++q) {
        const float *p = a.ws + ((u64)tile * S + q) * 512;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ta[i] += __hip_atomic_load(p + lane * 4 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            tb[i] += __hip_atomic_load(p + 256 + lane * 4 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (lane == 0) __hip_atomic_store(&a.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    fr_epilogue(a, glu, n0, nout, lane, ta, tb);
}

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
