/* Launch fusions of the single-stream chunk (few rows, every launch latency-bound): two pairs of
 * consecutive kernels of a conformer block become one launch each.
 *
 * attention_rel_out_c<CPW>: relative-position attention (attn_rel_core, the math of attention_rel)
 * fused with the output projection that follows it (reference src/encoder.c:163-166):
 *   C[row] += alpha * O[row] . Wo^T,  O[row] = [head 0 | ... | head H-1] attention outputs.
 * Workgroup (head h, column tile, row) computes its head's output (the heads' shares of the
 * product are independent: K of the projection is split by head) and multiplies it by its columns'
 * 128-wide slice of Wo, writing its head's partial row P[h][row][n]; the host folds the H partial
 * rows into C in head order with one more launch (resid_fold), so the sum does not depend on which
 * head finishes first.  Its Wo loads are issued with the attention's own loads.  CPW output columns
 * per wavefront, 8 wavefronts.
 *
 * gemv_dw_r<R>_n<NC>_k<KCH>: the causal depthwise conv + LayerNorm + SiLU of the convolution module
 * (the math of dwconv_ln_silu) as the prologue of the pointwise conv GEMV that consumes it
 * (reference src/encoder.c:171-175): every workgroup recomputes the R conv rows into LDS (they are
 * tiny next to the weight stream), then its wavefronts run the GEMV of gemv_impl on them.  The
 * per-thread conv, the LayerNorm reductions, the chunk mapping and the dot-product order are those
 * of the two separate kernels, so the results are identical to them. */
#include "nk_common.h"

template <int CPW>
__device__ __forceinline__ void attn_out_impl(const NkAttnOutArgs &p) {
    __shared__ AttnShared sh;
    __shared__ float oh[128];
    constexpr int LPC = 64 / CPW, DPL = 128 / LPC, LD = DPL / 8; /* lanes per column, dims per lane */
    const u32 h = blockIdx.x, orow = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const u32 n = blockIdx.y * (8 * CPW) + wave * CPW + lane / LPC, kq = (lane % LPC) * DPL;
    uint4 w[LD];
    const floatx4 r = attn_rel_core(p.at, h, orow, sh, [&] {
#pragma unroll
        for (int i = 0; i < LD; ++i) w[i] = ld_nt16(p.Wo + (u64)n * p.ldw + h * 128 + kq + 8 * i);
    });
    if (tid < 32) *(floatx4 *)&oh[4 * tid] = r;
    lds_barrier();
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < LD; ++i) acc = dot8(&oh[kq + 8 * i], w[i], acc);
#pragma unroll
    for (int m = 1; m < LPC; m <<= 1) acc += __shfl_xor(acc, m, 64);
    /* partial rows [head][row][D] */
    if (lane % LPC == 0) p.ws[((u64)h * gridDim.z + orow) * p.at.D + n] = acc;
}

extern "C" __global__ __launch_bounds__(512) void attention_rel_out_c16(const NkAttnOutArgs p) { attn_out_impl<16>(p); }
extern "C" __global__ __launch_bounds__(512) void attention_rel_out_c8(const NkAttnOutArgs p) { attn_out_impl<8>(p); }
extern "C" __global__ __launch_bounds__(512) void attention_rel_out_c4(const NkAttnOutArgs p) { attn_out_impl<4>(p); }

template <int R, int NC, int KCH>
__device__ __forceinline__ void gemv_dw_impl(const NkGemvDwArgs &p) {
    __shared__ float red[4];
    __shared__ float4 ys[R][256];
    const NkGemmArgs &a = p.g;
    const NkDwArgs &dw = p.d;
    const u32 tid = threadIdx.x, lane = tid & 63, gw = blockIdx.x * 4 + (tid >> 6);
    const u32 j0 = gw * NC, nch = a.K >> 3, M = a.M;
    const bool wave_ok = j0 < a.N; /* no early return: the prologue has barriers */

    /* 1. epilogue row map and bias (lane e < M * NC owns output (e / NC, j0 + e % NC)) */
    const u32 er = lane / NC, ecol = j0 + lane % NC;
    const bool e_ok = wave_ok && lane < (u32)R * NC && er < M && ecol < a.N;
    const u32 er_c = e_ok ? er : 0, ecol_c = e_ok ? ecol : 0;
    const int e_row = a.crow[er_c];
    const float e_ba = a.bias[ecol_c];

    /* 2. conv inputs: thread tid owns channels 4 tid .. 4 tid + 3 (D <= 1024) of every row */
    const u32 D4 = dw.D >> 2;
    const bool cok = tid < D4;
    const u32 c4 = cok ? tid : 0;
    const float *din = dw.din + (u64)((u32)dw.desc[NK_DESC_POS] - (DW_TAPS - 1)) * dw.D;
    float4 xin[R][DW_TAPS], wt[DW_TAPS];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int tap = 0; tap < DW_TAPS; ++tap) xin[r][tap] = *(const float4 *)(din + (u64)(r + tap) * dw.D + 4 * c4);
#pragma unroll
    for (int tap = 0; tap < DW_TAPS; ++tap) wt[tap] = *(const float4 *)(dw.W + (u64)c4 * 4 * DW_TAPS + 4 * tap);
    const float4 gg = ((const float4 *)dw.g)[c4], bb = ((const float4 *)dw.b)[c4];

    __builtin_amdgcn_sched_barrier(0); /* keep the small loads ahead of the weight stream */

    /* 3. weight rows of this wavefront */
    uint4 w[NC][KCH];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const u16 *wr = a.W + (u64)min(j0 + c, a.N - 1) * a.ldw;
#pragma unroll
        for (int q = 0; q < KCH; ++q) w[c][q] = ld_nt16(wr + 8 * (u64)min(lane + 64 * q, nch - 1));
    }

    __builtin_amdgcn_sched_barrier(0);

    /* 4. the C value to accumulate into */
    float *e_dst = a.C + (u64)(u32)e_row * a.ldc + ecol_c;
    const float e_c = a.accumulate ? *e_dst : 0.0f;

    /* 5. conv + LayerNorm + SiLU of every row into LDS */
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    const float *wf = (const float *)wt; /* channel e, tap q: element 9 e + q */
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc[4] = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
        for (int tap = 0; tap < DW_TAPS; ++tap) {
            acc[0] += wf[0 * DW_TAPS + tap] * xin[r][tap].x;
            acc[1] += wf[1 * DW_TAPS + tap] * xin[r][tap].y;
            acc[2] += wf[2 * DW_TAPS + tap] * xin[r][tap].z;
            acc[3] += wf[3 * DW_TAPS + tap] * xin[r][tap].w;
        }
        float4 v[LN_VEC] = { cok ? make_float4(acc[0], acc[1], acc[2], acc[3]) : z, z, z, z };
        const float4 g4[LN_VEC] = { cok ? gg : z, z, z, z }, b4[LN_VEC] = { cok ? bb : z, z, z, z };
        ln_vec(v, g4, b4, D4, dw.D, dw.eps, red);
        if (cok) ys[r][tid] = make_float4(silu_f(v[0].x), silu_f(v[0].y), silu_f(v[0].z), silu_f(v[0].w));
    }
    __syncthreads();

    /* 6. the lane's activation chunks (chunk j = floats 8 j .. 8 j + 7), zero past the row */
    float x[R][KCH][8];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < KCH; ++q) {
            const u32 j = lane + 64 * q;
            const bool ok = j < nch;
            const float4 lo = ys[r][2 * (ok ? j : 0)], hi = ys[r][2 * (ok ? j : 0) + 1];
            x[r][q][0] = ok ? lo.x : 0.f; x[r][q][1] = ok ? lo.y : 0.f;
            x[r][q][2] = ok ? lo.z : 0.f; x[r][q][3] = ok ? lo.w : 0.f;
            x[r][q][4] = ok ? hi.x : 0.f; x[r][q][5] = ok ? hi.y : 0.f;
            x[r][q][6] = ok ? hi.z : 0.f; x[r][q][7] = ok ? hi.w : 0.f;
        }

    /* 7. dot products, reductions, epilogue (no activation) */
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if ((u32)r >= M) break;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            float s = 0.0f;
#pragma unroll
            for (int q = 0; q < KCH; ++q) s = dot8(x[r][q], w[c][q], s);
            s = wsum(s);
            if (lane == (u32)(r * NC + c)) mine = s;
        }
    }
    if (!e_ok) return;
    const float v = (mine + e_ba) * a.alpha;
    *e_dst = a.accumulate ? (e_c + v) : v;
}

#define GEMV_DW(R, NC, KCH)                                                                                  \
    extern "C" __global__ __launch_bounds__(256) void gemv_dw_r##R##_n##NC##_k##KCH(const NkGemvDwArgs p) { \
        gemv_dw_impl<R, NC, KCH>(p);                                                                        \
    }
GEMV_DW(1, 1, 1) GEMV_DW(1, 2, 1) GEMV_DW(1, 4, 1) GEMV_DW(1, 1, 2) GEMV_DW(1, 2, 2) GEMV_DW(1, 4, 2)
GEMV_DW(2, 1, 1) GEMV_DW(2, 2, 1) GEMV_DW(2, 4, 1) GEMV_DW(2, 1, 2) GEMV_DW(2, 2, 2) GEMV_DW(2, 4, 2)
