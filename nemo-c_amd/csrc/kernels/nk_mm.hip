/* Many-row bf16-weight GEMM for gfx950 (M > 16: the batched multi-stream encoder, subsampling
 * 1x1 convs, the position tables): C[crow(m)][n] (= or +=) alpha * act(A W^T + b), act GLU pairs
 * weight rows n and n + N/2.
 *
 * Workgroup tile BM x BN (128 x 128 or 64 x 64), 4 wavefronts in 2 x 2, each wavefront
 * (BM/2) x (BN/2) outputs as 16x16 tiles of v_mfma_f32_16x16x32_bf16.  A is f32 in memory and is
 * split on its way into LDS into bf16 hi + lo (v_cvt_pk_bf16_f32; 16 significant bits), so every
 * K step issues two MFMAs per output tile.  K advances 32 per step through two LDS buffers: while
 * the MFMAs read one, the next tile is converted into the other and the tile after that is
 * already loading into registers.  The per-step barrier waits for LDS traffic only, so the global
 * loads in flight are not drained.  LDS rows are 40 bf16 (80 bytes) apart, which makes the
 * 16-byte fragment reads of 16 consecutive rows conflict-free.
 * GLU: a workgroup's BN weight rows are BN/2 rows of the first half and the matching BN/2 of the
 * second; each wavefront holds both halves of its output columns.
 * Replaces the reference's many-row gemm_mma path (src/kernels.metal:120-208, row blocks on
 * grid.y, src/model.c:86-95). */
#include "nk_common.h"

#define MM_LD 40 /* LDS row stride in bf16 elements */

/* 4 f32 -> hi, lo bf16 quads (8 bytes each) */
__device__ __forceinline__ void split4(floatx4 v, uint2 &hi, uint2 &lo) {
    const floatx2 v0 = { v[0], v[1] }, v1 = { v[2], v[3] };
    const u32 h0 = __builtin_bit_cast(u32, __builtin_convertvector(v0, bf16x2));
    const u32 h1 = __builtin_bit_cast(u32, __builtin_convertvector(v1, bf16x2));
    const floatx2 r0 = v0 - (floatx2){ __uint_as_float(h0 << 16), __uint_as_float(h0 & 0xffff0000u) };
    const floatx2 r1 = v1 - (floatx2){ __uint_as_float(h1 << 16), __uint_as_float(h1 & 0xffff0000u) };
    hi = make_uint2(h0, h1);
    lo = make_uint2(__builtin_bit_cast(u32, __builtin_convertvector(r0, bf16x2)),
                    __builtin_bit_cast(u32, __builtin_convertvector(r1, bf16x2)));
}

template <int BM, int BN, bool GLU>
__device__ __forceinline__ void mm_impl(const NkGemmArgs &a, u16 *smem) {
    constexpr int TI = BM / 32;           /* 16-row tiles per wavefront */
    constexpr int TJ = BN / 32;           /* 16-column tiles per wavefront */
    constexpr int AF = BM / 32;           /* float4 of A per thread per step */
    constexpr int BF = BN / 64;           /* uint4 of W per thread per step */
    constexpr int BUF = (2 * BM + BN) * MM_LD;
    const u32 tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const u32 M = a.M, m0 = blockIdx.y * BM;
    const u32 nout = GLU ? a.N / 2 : a.N;
    const u32 c0 = blockIdx.x * (GLU ? BN / 2 : BN); /* first output column of the workgroup */
    const u32 S = a.K >> 5;
    const u32 s_begin = 0, s_end = S;

    /* global -> register tile loads (rows past M re-read row M-1; their outputs are dropped) */
    const float *arow[AF];
    u32 akq[AF], ar[AF];
#pragma unroll
    for (int j = 0; j < AF; ++j) {
        const u32 f = tid + 256 * j;
        ar[j] = f >> 3;
        akq[j] = (f & 7) * 4;
        arow[j] = a.A + (u64)min(m0 + ar[j], M - 1) * a.lda + akq[j];
    }
    const u16 *wrow[BF];
    u32 br[BF], bkc[BF];
#pragma unroll
    for (int j = 0; j < BF; ++j) {
        const u32 f = tid + 256 * j;
        br[j] = f >> 2;
        bkc[j] = (f & 3) * 8;
        u32 n;
        if (GLU) n = br[j] < BN / 2 ? c0 + br[j] : a.N / 2 + c0 + (br[j] - BN / 2);
        else n = c0 + br[j];
        wrow[j] = a.W + (u64)n * a.ldw + bkc[j];
    }
    floatx4 ra[AF];
    uint4 rb[BF];
    auto load_tile = [&](u32 s) {
#pragma unroll
        for (int j = 0; j < AF; ++j) ra[j] = *(const floatx4 *)(arow[j] + (u64)s * 32);
#pragma unroll
        for (int j = 0; j < BF; ++j) rb[j] = ld_nt16(wrow[j] + (u64)s * 32);
    };
    auto store_tile = [&](u16 *buf) {
        u16 *ah = buf, *al = buf + BM * MM_LD, *bw = buf + 2 * BM * MM_LD;
#pragma unroll
        for (int j = 0; j < AF; ++j) {
            uint2 hi, lo;
            split4(ra[j], hi, lo);
            *(uint2 *)(ah + ar[j] * MM_LD + akq[j]) = hi;
            *(uint2 *)(al + ar[j] * MM_LD + akq[j]) = lo;
        }
#pragma unroll
        for (int j = 0; j < BF; ++j) *(uint4 *)(bw + br[j] * MM_LD + bkc[j]) = rb[j];
    };

    /* fragment addresses within a buffer: A rows wm*BM/2 + 16 i + l%16, B rows of the
     * wavefront's column tiles, k offset 8*(l/16) */
    const u32 fk = 8 * (lane >> 4), fr = lane & 15;
    u32 bcol[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        if (GLU) bcol[j] = j < TJ / 2 ? wn * (BN / 4) + 16 * j : BN / 2 + wn * (BN / 4) + 16 * (j - TJ / 2);
        else bcol[j] = wn * (BN / 2) + 16 * j;
    }

    floatx4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = (floatx4){ 0.f, 0.f, 0.f, 0.f };

    if (s_begin < s_end) {
        load_tile(s_begin);
        store_tile(smem);
        if (s_begin + 1 < s_end) load_tile(s_begin + 1);
        lds_barrier();
    }
    for (u32 s = s_begin; s < s_end; ++s) {
        const u16 *cur = smem + ((s - s_begin) & 1) * BUF;
        const u16 *ah = cur, *al = cur + BM * MM_LD, *bw = cur + 2 * BM * MM_LD;
        uint4 fb[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) fb[j] = *(const uint4 *)(bw + (bcol[j] + fr) * MM_LD + fk);
        uint4 fh[TI], fl[TI];
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const u32 row = wm * (BM / 2) + 16 * i + fr;
            fh[i] = *(const uint4 *)(ah + row * MM_LD + fk);
            fl[i] = *(const uint4 *)(al + row * MM_LD + fk);
        }
        /* all hi products, then all lo products: consecutive MFMAs never share an accumulator */
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[i][j] = mfma_bf16(fh[i], fb[j], acc[i][j]);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[i][j] = mfma_bf16(fl[i], fb[j], acc[i][j]);
        if (s + 1 < s_end) {
            store_tile(smem + ((s - s_begin + 1) & 1) * BUF);
            if (s + 2 < s_end) load_tile(s + 2);
        }
        lds_barrier();
    }

    /* epilogue: lane l holds rows 16 i + 4 (l/16) + e, column 16 j + l%16 of each tile.  Every
     * operand (row map, bias, the C values to accumulate into) is loaded before the first store so
     * the loads overlap instead of alternating with the stores. */
    constexpr int TO = GLU ? TJ / 2 : TJ;
    u32 orow[TI][4];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const u32 r = min(m0 + wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + e, M - 1);
            orow[i][e] = a.crow ? (u32)a.crow[r] : r;
        }
    u32 ocol[TO];
    float ba[TO], bb[TO];
#pragma unroll
    for (int j = 0; j < TO; ++j) {
        ocol[j] = c0 + (GLU ? wn * (BN / 4) : wn * (BN / 2)) + 16 * j + fr;
        const u32 cc = min(ocol[j], nout - 1);
        ba[j] = a.bias ? a.bias[cc] : 0.0f;
        bb[j] = (GLU && a.bias) ? a.bias[cc + a.N / 2] : 0.0f;
    }
    const bool rmw = a.accumulate;
    float cv[TO][TI][4];
#pragma unroll
    for (int j = 0; j < TO; ++j)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                cv[j][i][e] = rmw ? a.C[(u64)orow[i][e] * a.ldc + min(ocol[j], nout - 1)] : 0.0f;
#pragma unroll
    for (int j = 0; j < TO; ++j) {
        if (ocol[j] >= nout) continue;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const u32 r = m0 + wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + e;
                if (r >= M) continue;
                float *dst = a.C + (u64)orow[i][e] * a.ldc + ocol[j];
                float v;
                if constexpr (GLU) {
                    v = (acc[i][j][e] + ba[j]) * sigmoid_f(acc[i][j + TJ / 2][e] + bb[j]) * a.alpha;
                } else {
                    v = acc[i][j][e] + ba[j];
                    if (a.act == NK_ACT_SILU) v = silu_f(v);
                    else if (a.act == NK_ACT_RELU) v = fmaxf(v, 0.0f);
                    v *= a.alpha;
                }
                *dst = rmw ? cv[j][i][e] + v : v;
            }
    }
}

#define GEMM_MM(NAME, BM, BN, GLU)                                                                       \
    extern "C" __global__ __launch_bounds__(256) void NAME(const NkGemmArgs a) {                         \
        __shared__ uint4 smem4[2 * (2 * BM + BN) * MM_LD / 8];                                            \
        mm_impl<BM, BN, GLU>(a, (u16 *)smem4);                                                           \
    }
GEMM_MM(gemm_mm128, 128, 128, false)
GEMM_MM(gemm_mm64, 64, 64, false)
GEMM_MM(gemm_mm128_glu, 128, 128, true)
GEMM_MM(gemm_mm64_glu, 64, 64, true)
