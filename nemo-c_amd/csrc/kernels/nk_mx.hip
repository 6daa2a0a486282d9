/* Many-row bf16-weight GEMM for gfx950, fed by direct global -> LDS loads (M > 16: the batched
 * multi-stream encoder and decoder): C[crow(m)][n] (= or +=) alpha * act(A W^T + b); GLU pairs
 * weight rows n and n + N/2.
 *
 * Workgroup tile BM x BN, 4 wavefronts as WGM (along M) x 4/WGM (along N); each wavefront owns a
 * (BM/WGM) x (BN*WGM/4) block of 16x16 tiles of v_mfma_f32_16x16x32_bf16.
 *
 * Operand staging: a ring of NS LDS stages (NS = 3 or 4 by tile size), each holding one K step of
 * KS = 32 columns of A (f32, BM x 4KS B) and W (bf16, BN x 2KS B).  Stages are filled by
 * global_load_lds_dwordx4 (16 bytes per lane
 * straight into LDS, no registers), issued NS-1 steps ahead of their use, so a wavefront only waits
 * for a stage's loads right before the barrier that publishes it.  A DMA instruction writes 64
 * consecutive 16-byte LDS granules in lane order; the global address each lane reads is chosen so
 * that granule g of row r holds K-granule (g ^ swizzle(r)), which makes the 16-row fragment reads
 * (ds_read_b128) hit distinct banks (swz_a / swz_b below).
 *
 * A enters the MFMAs as bf16 hi = RNE(a) and lo = RNE(a - hi), and every K step issues the hi and
 * the lo product: 16 significant bits of A against exact bf16 weights, f32 accumulation.  The
 * reference's many-row path multiplies f32 A by bf16 W in f32 (src/kernels.metal:120-208,
 * simdgroup_float8x8).  Two A forms:
 *   - f32 rows (AS = false): each fragment (8 consecutive K of one row per lane) is split in
 *     registers (v_cvt_pk_bf16_f32) after its LDS read;
 *   - split rows (AS = true, NkGemmArgs.A2): the producer stored hi and lo (the same values), so
 *     both planes stream into LDS like the weights and the fragments feed the MFMAs directly, with
 *     no VALU work in the K loop.
 * A kernel that produces the next GEMM's A can write split rows itself (OS, NkGemmArgs.C2).
 *
 * Tile order: the grid is 8 x (tiles per XCD); workgroup b runs on XCD b % 8 and takes tile
 * (b % 8) * per + b / 8 of an order that walks groups of group_m row tiles across all column tiles
 * (row tile fastest), so the workgroups of one XCD share weight columns and a few row panels in
 * that XCD's L2.  grid tiles past the end exit at once.
 *
 * Accumulating GEMMs without bias or activation (the residual updates: C += alpha * A W^T) run on
 * the _acc kernels.  They sum K in kblocks equal blocks, each from zero, and add the block sums in
 * block order; with splits = kblocks every workgroup computes one block.  Either way the kernel
 * only writes partial rows (one per split), and the update C + alpha * (((0 + p0) + p1) + ...) is
 * applied by the next kernel that reads C (the batched encoder's LayerNorms) or by resid_fold.
 * Both forms give the same bits, so the host may split K or not by the row count (how many other
 * streams share the step) without changing any row's result, and no result depends on which
 * workgroup finishes first; no workgroup waits for or communicates with another. */
#include "nk_common.h"

/* LDS granule swizzles: granule g of row r lives in slot g ^ swz(r).  A fragment read is one
 * ds_read_b128 per lane over 16 consecutive rows at one K granule (lanes 16 f .. 16 f + 15).  The
 * K-stage-32 forms (A rows of 8 granules, W rows of 4) were chosen by the SQ_LDS_BANK_CONFLICT
 * counter on gfx950 over candidate functions: these two read with zero conflict cycles, where
 * the earlier ((r>>1)&7)^((r&1)<<2) and ((n>>1)&3)^((n>>3)&1) cost 4 extra cycles per read (a
 * 2-way conflict; 1-3% of kernel time) and the plain r % 8 cost a third of the kernel time at
 * 3584 rows. */
__device__ __forceinline__ u32 swz_a(u32 r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ u32 swz_b(u32 n) { return (n >> 1) & 3; }
/* bf16 rows of G granules (4: 32 K, 8: 64 K).  The 8-granule rows have the f32 rows' geometry but
 * another read pattern (lane group f reads granule 4h + f, not 2f and 2f + 1): swz_a costs a 2-way
 * conflict on every read there, (r >> 1) & 7 none (SQ_LDS_BANK_CONFLICT over candidates on gfx950) */
template <int G> __device__ __forceinline__ u32 swz_h(u32 r) { return G == 4 ? swz_b(r) : (r >> 1) & 7; }


/* EPI: 0 bias / activation / GLU / accumulate epilogue; 1 argmax keys; 2 blocked-K residual
 * update into partial rows.  AS: A as split rows; OS: outputs as split rows (EPI 0 without GLU). */
template <int BM, int BN, int WGM, int NS, bool GLU, int EPI = 0, bool AS = false, bool OS = false>
__device__ __forceinline__ void mx_impl(const NkGemmArgs &a, lds_char_t *const (&ring)[NS]) {
    /* K step: 64 for split-row A (128-byte row segments, whole cache lines, per operand row), 32 for
     * f32 A */
    constexpr int KS = AS ? NK_MX_KS_SPLIT : 32, KSUB = KS / 32;
    static_assert(!OS || (EPI == 0 && !GLU), "split outputs from the plain epilogue only");
    constexpr int WGN = 4 / WGM;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TI = WTM / 16, TJ = WTN / 16;
    constexpr int AG = KS / 4, BG = KS / 8; /* 16-byte granules per A row / W row of a stage */
    constexpr int A_BYTES = BM * KS * 4;
    constexpr int AI = BM * AG / 256; /* A granules per thread per stage */
    constexpr int BI = BN * BG / 256; /* W granules per thread per stage */
    static_assert(AI >= 1 && BI >= 1 && TI >= 1 && TJ >= (GLU ? 2 : 1), "tile shape");
    static_assert(EPI != 2 || !GLU, "the residual update has no GLU");
    const u32 tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const u32 wm = wave / WGN, wn = wave % WGN;
    const u32 M = a.mrows ? min(a.M, (u32)max(*a.mrows, 0) * a.mrows_mul) : a.M;
    const u32 nout = GLU ? a.N / 2 : a.N;
    const u32 TMt = (M + BM - 1) / BM, TNt = nout / (GLU ? BN / 2 : BN), KZ = a.splits;

    /* tile of this workgroup */
    const u32 per = gridDim.x / 8;
    const u32 t = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (t >= TMt * TNt * KZ) return;
    const u32 kz = t / (TMt * TNt), tt = t % (TMt * TNt);
    const u32 G = a.group_m, gsz = G * TNt, grp = tt / gsz, first = grp * G;
    const u32 gh = min(TMt - first, G), within = tt % gsz;
    const u32 tm = first + within % gh, tn = within / gh;
    const u32 m0 = tm * BM;
    const u32 c0 = tn * (GLU ? BN / 2 : BN); /* first output column */
    const u32 S = a.K / KS;
    const u32 s_begin = (u32)(((u64)S * kz) / KZ), s_end = (u32)(((u64)S * (kz + 1)) / KZ);
    const u32 nst = s_end - s_begin;
    /* K steps per block of the blocked sum (EPI 2; the whole range otherwise) */
    const u32 spb = EPI == 2 ? S / a.kblocks : nst;

    /* DMA sources: granule p of a stage region is written by lane p % 64 of instruction p / 64
     * (instruction j of wavefront w covers p in [(4j + w) * 64, +64)).  Split A: the stage's A region
     * is the hi plane (BM rows of BG granules, laid out like the weights) then the lo plane. */
    const char *asrc[AI];
#pragma unroll
    for (int j = 0; j < AI; ++j) {
        const u32 p = (4 * j + wave) * 64 + lane;
        if constexpr (AS) {
            const u32 plane = p / (BM * BG), q = p % (BM * BG), r = q / BG, kg = (q % BG) ^ swz_h<BG>(r);
            asrc[j] = (const char *)(a.A2 + (u64)min(m0 + r, M - 1) * a.lda + plane * a.K + 8 * kg + (u64)s_begin * KS);
        } else {
            const u32 r = p / AG, kg = (p % AG) ^ swz_a(r);
            asrc[j] = (const char *)(a.A + (u64)min(m0 + r, M - 1) * a.lda + 4 * kg + (u64)s_begin * KS);
        }
    }
    constexpr u32 A_STEP = AS ? KS * 2 : KS * 4; /* bytes of one K step of one A row (per plane) */
    const u16 *bsrc[BI];
#pragma unroll
    for (int j = 0; j < BI; ++j) {
        const u32 p = (4 * j + wave) * 64 + lane, n = p / BG, kg = (p % BG) ^ swz_h<BG>(n);
        u32 col;
        if (GLU) col = n < BN / 2 ? c0 + n : a.N / 2 + c0 + (n - BN / 2);
        else col = c0 + n;
        bsrc[j] = a.W + (u64)col * a.ldw + 8 * kg + (u64)s_begin * KS;
    }
    auto issue = [&](u32 q, int slot) { /* loads of local step q into ring slot `slot` */
        lds_char_t *st = ring[slot];
#pragma unroll
        for (int j = 0; j < AI; ++j) dma16(asrc[j] + (u64)q * A_STEP, st + (4 * j + wave) * 1024);
#pragma unroll
        for (int j = 0; j < BI; ++j) dma16(bsrc[j] + (u64)q * KS, st + A_BYTES + (4 * j + wave) * 1024);
    };

    /* fragment addresses inside a stage */
    const u32 fr = lane & 15, fg = lane >> 4;
    /* f32 A: the two halves of the 8 K; split A: the hi and the lo fragment of each 32-K substep */
    u32 aoff[TI][KSUB][2];
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const u32 r = wm * WTM + 16 * i + fr;
        if constexpr (AS) {
#pragma unroll
            for (int h = 0; h < KSUB; ++h) {
                aoff[i][h][0] = (r * BG + ((4 * h + fg) ^ swz_h<BG>(r))) * 16;
                aoff[i][h][1] = aoff[i][h][0] + BM * BG * 16;
            }
        } else {
            aoff[i][0][0] = (r * AG + ((2 * fg) ^ swz_a(r))) * 16;
            aoff[i][0][1] = (r * AG + ((2 * fg + 1) ^ swz_a(r))) * 16;
        }
    }
    u32 boff[TJ][KSUB];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        u32 n;
        if (GLU) n = j < TJ / 2 ? wn * (WTN / 2) + 16 * j : BN / 2 + wn * (WTN / 2) + 16 * (j - TJ / 2);
        else n = wn * WTN + 16 * j;
        n += fr;
#pragma unroll
        for (int h = 0; h < KSUB; ++h) boff[j][h] = A_BYTES + (n * BG + ((4 * h + fg) ^ swz_h<BG>(n))) * 16;
    }

    floatx4 acc[TI][TJ];
    /* EPI 2: sum of the finished K blocks, (((0 + b0) + b1) + ...) */
    floatx4 tot[EPI == 2 ? TI : 1][EPI == 2 ? TJ : 1];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = (floatx4){ 0.f, 0.f, 0.f, 0.f };
    if constexpr (EPI == 2)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) tot[i][j] = (floatx4){ 0.f, 0.f, 0.f, 0.f };

    /* Every step issues the loads of the step NS-1 ahead, clamped to the last one (the extra
     * copies land in slots nobody reads), so the loads in flight behind step q are always (NS-2)
     * steps' worth.  The loop is unrolled by NS so every ring slot address is a constant. */
#pragma unroll
    for (int u = 0; u < NS - 1; ++u) issue(min((u32)u, nst - 1), u);
    for (u32 q0 = 0; q0 < nst; q0 += NS) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {
        const u32 q = q0 + u;
        if (q >= nst) break;
        /* this wavefront's loads of step q are done, then the barrier publishes every wavefront's
         * part and retires all reads of the slot the next issue overwrites */
        wait_vm_lgkm<(NS - 2) * (AI + BI)>();
        barrier_mem();
        issue(min(q + NS - 1, nst - 1), (u + NS - 1) % NS);
        const lds_char_t *st = ring[u];
        uint4 fb[KSUB][TJ], fh[KSUB][TI], fl[KSUB][TI];
#pragma unroll
        for (int h = 0; h < KSUB; ++h) {
#pragma unroll
            for (int j = 0; j < TJ; ++j) fb[h][j] = *(const __attribute__((address_space(3))) uint4 *)(st + boff[j][h]);
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                if constexpr (AS) {
                    fh[h][i] = *(const __attribute__((address_space(3))) uint4 *)(st + aoff[i][h][0]);
                    fl[h][i] = *(const __attribute__((address_space(3))) uint4 *)(st + aoff[i][h][1]);
                } else {
                    const floatx4 x0 = *(const __attribute__((address_space(3))) floatx4 *)(st + aoff[i][0][0]);
                    const floatx4 x1 = *(const __attribute__((address_space(3))) floatx4 *)(st + aoff[i][0][1]);
                    const float x[8] = { x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3] };
                    split8(x, fh[h][i], fl[h][i]);
                }
            }
        }
        /* per 32-K substep: every hi product, then every lo product (the same order at every K step
         * size, so every tile and step size gives the same bits) */
#pragma unroll
        for (int h = 0; h < KSUB; ++h) {
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) acc[i][j] = mfma_bf16(fh[h][i], fb[h][j], acc[i][j]);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) acc[i][j] = mfma_bf16(fl[h][i], fb[h][j], acc[i][j]);
        }
        if constexpr (EPI == 2) {
            if ((q + 1) % spb == 0) { /* a K block ends: add its sum, start the next from zero */
#pragma unroll
                for (int i = 0; i < TI; ++i)
#pragma unroll
                    for (int j = 0; j < TJ; ++j) {
                        tot[i][j] += acc[i][j];
                        acc[i][j] = (floatx4){ 0.f, 0.f, 0.f, 0.f };
                    }
            }
        }
    }
    }

    wait_vm_lgkm<0>(); /* no load into LDS may land after the workgroup ends */

    if constexpr (EPI == 2) {
        /* residual update, deferred: block kz's sum (all blocks' ordered sum when K is not split)
         * goes to partials[kz][row][n] (rows of N floats); C is not touched.  The rows are folded
         * into C in block order afterwards, by the LayerNorm that reads them next or by
         * resid_fold: C + alpha * (((0 + p0) + p1) + ...), the unsplit epilogue's bits. */
        float *P = a.ws + (u64)kz * a.M * a.N;
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const u32 r = m0 + wm * WTM + 16 * i + 4 * fg + e;
                    if (r < M) P[(u64)r * a.N + c0 + wn * WTN + 16 * j + fr] = tot[i][j][e];
                }
        return;
    }

    if constexpr (EPI == 1) {
        /* argmax partials: per row, the best (score + bias, lowest column) over this wavefront's
         * columns below keys_n, as one packed key per (row, column tile, wavefront column) */
        unsigned long long best[TI][4];
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) best[i][e] = 0;
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const u32 col = c0 + wn * WTN + 16 * j + fr;
            const bool ok = col < a.keys_n;
            const float bj = a.bias ? a.bias[col] : 0.0f;
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const unsigned long long k = ok ? dec_key(acc[i][j][e] + bj, col) : 0ull;
                    best[i][e] = k > best[i][e] ? k : best[i][e];
                }
        }
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                unsigned long long k = best[i][e];
#pragma unroll
                for (int msk = 1; msk < 16; msk <<= 1) {
                    const unsigned long long o = shfl_xor_u64(k, msk);
                    k = o > k ? o : k;
                }
                const u32 r = m0 + wm * WTM + 16 * i + 4 * fg + e;
                if (fr == 0 && r < M) a.keys[(u64)r * a.keys_ld + tn * WGN + wn] = k;
            }
        return;
    }

    /* epilogue: lane l holds rows 16 i + 4 (l/16) + e, column 16 j + l%16 of each tile; every
     * operand (row map, bias, the C values to accumulate into) is loaded before the first store */
    constexpr int TO = GLU ? TJ / 2 : TJ;
    u32 orow[TI][4];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const u32 r = min(m0 + wm * WTM + 16 * i + 4 * fg + e, M - 1);
            orow[i][e] = a.crow ? (u32)a.crow[r] : r;
        }
    u32 ocol[TO];
    float ba[TO], bb[TO];
#pragma unroll
    for (int j = 0; j < TO; ++j) {
        ocol[j] = c0 + (GLU ? wn * (WTN / 2) : wn * WTN) + 16 * j + fr;
        ba[j] = a.bias ? a.bias[ocol[j]] : 0.0f;
        bb[j] = (GLU && a.bias) ? a.bias[ocol[j] + a.N / 2] : 0.0f;
    }
    if constexpr (OS) {
        /* split rows of nout values: hi at C2[row * ldc + n], lo at + nout */
#pragma unroll
        for (int j = 0; j < TO; ++j)
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    float v[2];
#pragma unroll
                    for (int d = 0; d < 2; ++d) {
                        v[d] = acc[i][j][e + d] + ba[j];
                        if (a.act == NK_ACT_SILU) v[d] = silu_f(v[d]);
                        else if (a.act == NK_ACT_RELU) v[d] = fmaxf(v[d], 0.0f);
                        v[d] *= a.alpha;
                    }
                    u32 hi, lo;
                    split2(v[0], v[1], hi, lo);
#pragma unroll
                    for (int d = 0; d < 2; ++d) {
                        const u32 r = m0 + wm * WTM + 16 * i + 4 * fg + e + d;
                        if (r >= M) continue;
                        u16 *dst = a.C2 + (u64)r * a.ldc + ocol[j];
                        dst[0] = (u16)(hi >> (16 * d));
                        dst[nout] = (u16)(lo >> (16 * d));
                    }
                }
        return;
    }
    const bool rmw = a.accumulate;
    float cv[TO][TI][4];
#pragma unroll
    for (int j = 0; j < TO; ++j)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) cv[j][i][e] = rmw ? a.C[(u64)orow[i][e] * a.ldc + ocol[j]] : 0.0f;
#pragma unroll
    for (int j = 0; j < TO; ++j) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (m0 + wm * WTM + 16 * i + 4 * fg + e >= M) continue;
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

/* Ring depth NS.  Stages are (BM*4 + BN*2)*KS bytes, and the depth is chosen so that two
 * workgroups fit a CU's 160 KB of LDS: the second workgroup's MFMAs run while the first waits at
 * its barrier.  Measured on gfx950 (3584 rows, 128x128: 117 -> 79 us), and again with deeper rings
 * at one workgroup per CU, which were slower at every shape from 448 to 3584 rows.
 *   f32 A, KS 32:        3 x 24 KB for 128x128, 4 x 16 KB for 64x128, 4 x 12 KB for 64x64;
 *   split-row A, KS 64:  2 x 32 KB for 64x128, 3 x 24 KB for 64x64 (2 x 48 KB for 128x128, one
 *                        workgroup per CU, which the host does not pick for split rows).
 * The 64-wide K step reads whole 128-byte row segments and halves the barriers: 10-15% faster
 * than 32 at 448 and 1792 rows. */
#ifndef MX_NS_L
#define MX_NS_L 3
#endif
#ifndef MX_NS_M
#define MX_NS_M 4
#endif
#ifndef MX_NS_S
#define MX_NS_S 4
#endif
#ifndef MX_NS_LS
#define MX_NS_LS 2
#endif
#ifndef MX_NS_MS
#define MX_NS_MS 2
#endif
#ifndef MX_NS_SS
#define MX_NS_SS 3
#endif
#define GEMM_MX_T(NAME, BM, BN, WGM, NS, GLU, EPI, AS, OS)                                              \
    extern "C" __global__ __launch_bounds__(256) void NAME(const NkGemmArgs a) {                          \
        __shared__ uint4 ring_mem[NS][(BM * 4 + BN * 2) * (AS ? NK_MX_KS_SPLIT : 32) / 16];                    \
        lds_char_t *ring[NS];                                                                             \
        _Pragma("unroll") for (int i = 0; i < NS; ++i) ring[i] = (lds_char_t *)ring_mem[i];               \
        mx_impl<BM, BN, WGM, NS, GLU, EPI, AS, OS>(a, ring);                                              \
    }
#define GEMM_MX(NAME, BM, BN, WGM, NS, GLU, EPI) GEMM_MX_T(NAME, BM, BN, WGM, NS, GLU, EPI, false, false)
GEMM_MX(gemm_mx128x128, 128, 128, 2, MX_NS_L, false, 0)
GEMM_MX(gemm_mx64x128, 64, 128, 2, MX_NS_M, false, 0)
GEMM_MX(gemm_mx64x64, 64, 64, 2, MX_NS_S, false, 0)
GEMM_MX(gemm_mx128x128_glu, 128, 128, 2, MX_NS_L, true, 0)
GEMM_MX(gemm_mx64x128_glu, 64, 128, 2, MX_NS_M, true, 0)
GEMM_MX(gemm_mx64x64_glu, 64, 64, 2, MX_NS_S, true, 0)
/* residual updates: blocked K, optional ordered split */
GEMM_MX(gemm_mx128x128_acc, 128, 128, 2, MX_NS_L, false, 2)
GEMM_MX(gemm_mx64x128_acc, 64, 128, 2, MX_NS_M, false, 2)
GEMM_MX(gemm_mx64x64_acc, 64, 64, 2, MX_NS_S, false, 2)
/* joint scores -> argmax partials (keys), 64x64 tiles: two keys per row per column tile */
GEMM_MX(gemm_mx64x64_argmax, 64, 64, 2, MX_NS_S, false, 1)
/* split-row A (suffix _s), split-row outputs (suffix _so) */
GEMM_MX_T(gemm_mx128x128_s, 128, 128, 2, MX_NS_LS, false, 0, true, false)
GEMM_MX_T(gemm_mx64x128_s, 64, 128, 2, MX_NS_MS, false, 0, true, false)
GEMM_MX_T(gemm_mx64x64_s, 64, 64, 2, MX_NS_SS, false, 0, true, false)
GEMM_MX_T(gemm_mx128x128_glu_s, 128, 128, 2, MX_NS_LS, true, 0, true, false)
GEMM_MX_T(gemm_mx64x128_glu_s, 64, 128, 2, MX_NS_MS, true, 0, true, false)
GEMM_MX_T(gemm_mx64x64_glu_s, 64, 64, 2, MX_NS_SS, true, 0, true, false)
GEMM_MX_T(gemm_mx128x128_acc_s, 128, 128, 2, MX_NS_LS, false, 2, true, false)
GEMM_MX_T(gemm_mx64x128_acc_s, 64, 128, 2, MX_NS_MS, false, 2, true, false)
GEMM_MX_T(gemm_mx64x64_acc_s, 64, 64, 2, MX_NS_SS, false, 2, true, false)
GEMM_MX_T(gemm_mx128x128_so, 128, 128, 2, MX_NS_L, false, 0, false, true)
GEMM_MX_T(gemm_mx64x128_so, 64, 128, 2, MX_NS_M, false, 0, false, true)
GEMM_MX_T(gemm_mx64x64_so, 64, 64, 2, MX_NS_S, false, 0, false, true)
GEMM_MX_T(gemm_mx128x128_s_so, 128, 128, 2, MX_NS_LS, false, 0, true, true)
GEMM_MX_T(gemm_mx64x128_s_so, 64, 128, 2, MX_NS_MS, false, 0, true, true)
GEMM_MX_T(gemm_mx64x64_s_so, 64, 64, 2, MX_NS_SS, false, 0, true, true)
