/* Persistent encoder chain for one-row chunks (the 80 ms single-stream path): the 24 conformer
 * blocks of reference src/encoder.c:152-188 in one launch, in place of the ~190 kernels of the
 * per-kernel graph whose every boundary costs ~1.8 us.
 *
 * NK_CHAIN_G = 256 workgroups, one per CU (the LDS footprint admits one), all resident.  Every
 * workgroup owns a slice of every weight matrix (16 rows of the 4096-row matrices, 4 rows of the
 * 1024-row ones, 12 of q|k|v, 4 GLU channel pairs of pw1), so each streams 1/256 of a block's
 * weights.  A block is nine phases; each phase turns the whole row produced by the previous one
 * into this workgroup's slice of the next row, and the slices are handed to every workgroup
 * through a hand-off slot:
 *   A  LN_out(prev) -> LN_ff1 -> ff1_w1, SiLU          (4096)   src/encoder.c:155-157
 *   B  x + 0.5 * ff1_w2 h                              (1024)
 *   C  LN_att -> q|k|v (also written to the K/V cache)  (3072)   src/encoder.c:159-162
 *   D  relative-position attention, one workgroup per head (1024)  src/encoder.c:163-165
 *   E  x + wo att                                      (1024)
 *   F  LN_conv -> pw1, GLU (written to the conv history) -> causal depthwise conv  (1024)
 *   G  LN_bn -> SiLU -> x + pw2 y                       (1024)   src/encoder.c:169-175
 *   H  LN_ff2 -> ff2_w1, SiLU                           (4096)   src/encoder.c:177-179
 *   I  x + 0.5 * ff2_w2 h                              (1024)   (LN_out in the next block's A)
 * The math of each operation is that of the per-kernel path (reference src/kernels.metal: GEMMs
 * with bf16 weights and f32 activations :51-118, LayerNorm :211-255, attention :290-348, conv
 * :359-409); only the summation orders differ.
 *
 * Hand-off.  An entry is 8 bytes {f32 value, u32 tag}, stored with one agent-coherent (sc1)
 * 8-byte store, so value and tag arrive together: no flag, no fence, no counter.  The reader
 * loads 16 bytes (two entries) per lane with sc1 loads and retries until every entry it needs
 * carries the tag of this hand-off.  Tag = epoch * 1024 + hand-off index; the epoch comes from
 * the chunk descriptor and differs on consecutive chunks, so entries of the previous chunk never
 * match.  Hand-off i uses slot i mod 3: a slot is rewritten three hand-offs later, and by then
 * every reader of its previous contents has finished (a writer of hand-off i + 3 has seen all of
 * hand-off i + 2, whose writers had all seen i + 1, whose writers are, directly or through the
 * attention heads, every workgroup that waits for i).  Two slots would not do: hand-off D -> E
 * is written by the 8 attention workgroups alone, which do not wait for all of C -> D.
 * Every wait is bounded (spin_max polls, and the epoch written to abort_word by any workgroup
 * that gave up ends the others' waits), and a time-out is reported in the host-visible err_word.
 *
 * Roles within a workgroup (6 wavefronts, one LDS barrier per phase):
 *   - wavefronts 0-3 compute: after the barrier of phase p they issue the weight loads of phase
 *     p + 2 into registers, read the phase's input row from LDS, form their dot products (lane l
 *     holds 16-byte chunks l, l + 64, ... of a weight row, 1 KB per load instruction), reduce
 *     them across the wavefront and store the outputs as hand-off entries;
 *   - wavefront 4 waits for the next phase's input while they compute, applies that phase's
 *     LayerNorm (the whole row: every workgroup normalises it itself), keeps the residual row
 *     and writes the input row to LDS for the next barrier; its LayerNorm parameters are loaded
 *     one LayerNorm ahead;
 *   - wavefront 5 shares the waits of the 4096-wide rows and, in the attention workgroups, moves
 *     the head's cached K and V rows and its position rows into LDS by direct-to-LDS loads two
 *     phases before the attention. */
#include "nk_common.h"

namespace chain {

constexpr u32 G = NK_CHAIN_G, D = NK_CHAIN_D, FF = NK_CHAIN_FF, QKV = 3 * NK_CHAIN_D, H = NK_CHAIN_HEADS, DH = 128;
constexpr u32 SLOT = NK_CHAIN_SLOT, MAXL = NK_CHAIN_MAX_L;
static_assert(H * DH == D && G * 4 == D && G * 16 == FF && G * 12 == QKV, "slices assume these shapes");

struct Shared {
    float ib[2][FF];                            /* phase input rows, by phase parity */
    float xr[2][D];                             /* residual rows (alternating) */
    float ks[MAXL][DH], vs[MAXL][DH], ps[MAXL][DH]; /* attention: the head's cached K, V rows and position rows */
    float knew[DH], vnew[DH];                   /* attention: the chunk's own K and V of the head */
    float lnp[4][D];                            /* LayerNorm parameters of the next LayerNorm(s) */
    floatx4 qu4[32], qv4[32];
    float s[MAXL];
    floatx4 part[8][32];
    int bad;
};

/* 16 bytes = entries e, e + 1 (e even) of a slot, loaded agent-coherent (sc1) */
__device__ __forceinline__ u32x4 ll_load(const u64 *slot, u32 e) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)slot, 0, 0x7fffffff, 0x00020000);
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, 8 * e, 0, 16));
}

/* one entry, value and tag in one agent-coherent 8-byte store */
__device__ __forceinline__ void ll_put(u64 *slot, u32 e, float v, u32 tag) {
    __hip_atomic_store(slot + e, ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Ctl {
    u64 *ll;
    const u32 *abort_word;
    u32 epoch, base, spin_max;
    __device__ u64 *slot(u32 hand) const { return ll + (u64)(hand % NK_CHAIN_SLOTS) * SLOT; }
    __device__ u32 tag(u32 hand) const { return base + hand; }
};

/* Wavefront-wide wait: load i of this lane covers entries ent[i], ent[i] + 1 of the slot of
 * hand-off `hand`; returns once every entry of the wavefront carries its tag, with the values in
 * v (false after spin_max rounds, or once another workgroup has given up on this epoch). */
template <int NL>
__device__ __forceinline__ bool ll_wait(const Ctl &c, u32 hand, const u32 (&ent)[NL], float2 (&v)[NL]) {
    const u64 *slot = c.slot(hand);
    const u32 tag = c.tag(hand);
    u32 spins = 0;
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const u32x4 r = ll_load(slot, ent[i]);
            v[i] = make_float2(__uint_as_float(r.x), __uint_as_float(r.z));
            ok = ok & (r.y == tag) & (r.w == tag);
        }
        if (__all(ok)) return true;
        if (++spins > c.spin_max) return false;
        if ((spins & 255) == 0 && __hip_atomic_load(c.abort_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == c.epoch)
            return false;
    }
}

/* a wait that gave up: the workgroup leaves at the next barrier, the others at their next wait */
__device__ __forceinline__ void give_up(const NkChainArgs &a, const Ctl &c, Shared &sh, u32 hand) {
    if ((threadIdx.x & 63) == 0) {
        sh.bad = 1;
        __hip_atomic_store(a.abort_word, c.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.err_word, (int)hand + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

/* LayerNorm of a 1024-row held as float2 pairs by one wavefront (lane l: elements 2(l + 64i),
 * +1): mean, then the centred variance, y = (x - mean) * (1 / sqrt(var + eps)) * g + b. */
__device__ __forceinline__ void ln_pairs(float2 (&v)[8], const float2 (&g)[8], const float2 (&b)[8], float eps) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) { s += v[i].x; s += v[i].y; }
    const float mean = wsum(s) / (float)D;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float d0 = v[i].x - mean, d1 = v[i].y - mean;
        ss += d0 * d0;
        ss += d1 * d1;
    }
    const float inv = 1.0f / sqrtf(wsum(ss) / (float)D + eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i].x = (v[i].x - mean) * inv * g[i].x + b[i].x;
        v[i].y = (v[i].y - mean) * inv * g[i].y + b[i].y;
    }
}

__device__ __forceinline__ void ld_pairs(float2 (&p)[8], const float *src, u32 lane) {
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = *(const float2 *)(src + 2 * (lane + 64 * i));
}

/* LayerNorm parameter vectors (D floats each) into lnp[k], lnp[k + 1] by direct-to-LDS loads of
 * the hand-off wavefront.  They are issued after the LayerNorm that last read those rows (the
 * lgkmcnt wait makes sure its LDS reads are done) and before the next hand-off wait, whose own
 * loads complete after them: the vmcnt(0) that follows that wait covers them. */
__device__ __forceinline__ void ln_params_to_lds(Shared &sh, u32 k, const float *gam, const float *bet, u32 lane) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < (int)D / 256; ++i) {
        dma16(gam + 256 * i + 4 * lane, (lds_char_t *)&sh.lnp[k][256 * i]);
        dma16(bet + 256 * i + 4 * lane, (lds_char_t *)&sh.lnp[k + 1][256 * i]);
    }
}

/* LayerNorm with the parameters in lnp[k], lnp[k + 1] (after the wait that covers their loads) */
__device__ __forceinline__ void ln_lds(float2 (&v)[8], const Shared &sh, u32 k, float eps, u32 lane) {
    float2 g[8], b[8];
    ld_pairs(g, sh.lnp[k], lane);
    ld_pairs(b, sh.lnp[k + 1], lane);
    ln_pairs(v, g, b, eps);
}
__device__ __forceinline__ void st_pairs(float *dst, const float2 (&v)[8], u32 lane) {
#pragma unroll
    for (int i = 0; i < 8; ++i) *(float2 *)(dst + 2 * (lane + 64 * i)) = v[i];
}

/* Global-memory accesses through pointers read from the layer table.  The compiler cannot tell
 * that such a pointer is global and would emit flat instructions, which also count in lgkmcnt:
 * then every LDS wait (each barrier) would wait for the weight loads in flight as well. */
typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
typedef __attribute__((address_space(1))) const float g_float;
typedef __attribute__((address_space(1))) const floatx4 g_floatx4;
typedef __attribute__((address_space(1))) float g_float_w;
__device__ __forceinline__ uint4 ldg_nt16(const u16 *p) {
    const u32x4 v = __builtin_nontemporal_load((g_u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float ldg(const float *p) { return *(g_float *)p; }
__device__ __forceinline__ floatx4 ldg4(const float *p) { return *(g_floatx4 *)p; }
__device__ __forceinline__ void stg(float *p, float v) { *(g_float_w *)p = v; }

/* weight rows row0 .. row0 + NC - 1 of a [.][K] bf16 matrix, chunks lane + 64 q */
template <int NC, int KCH>
__device__ __forceinline__ void ld_rows(uint4 (&w)[NC][KCH], const u16 *W, u32 row0, u32 K, u32 lane) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < KCH; ++q) w[c][q] = ldg_nt16(W + (u64)(row0 + c) * K + 8 * (lane + 64 * q));
}

/* the lane's chunks lane + 64 q of an input row in LDS */
template <int KCH>
__device__ __forceinline__ void ld_x(float (&x)[KCH][8], const float *row, u32 lane) {
#pragma unroll
    for (int q = 0; q < KCH; ++q) {
        const floatx4 a = *(const floatx4 *)(row + 8 * (lane + 64 * q));
        const floatx4 b = *(const floatx4 *)(row + 8 * (lane + 64 * q) + 4);
        x[q][0] = a[0]; x[q][1] = a[1]; x[q][2] = a[2]; x[q][3] = a[3];
        x[q][4] = b[0]; x[q][5] = b[1]; x[q][6] = b[2]; x[q][7] = b[3];
    }
}

/* dot product of one weight row with the row held in x, summed over the wavefront (uniform) */
template <int KCH>
__device__ __forceinline__ float dot_row(const float (&x)[KCH][8], const uint4 (&w)[KCH]) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < KCH; ++q) s = dot8(x[q], w[q], s);
    return wsum(s);
}

/* the head's cached K and V rows (window rows 0 .. cl-1) and its position rows (0 .. L-1) into
 * LDS: each direct load moves two 512-byte row segments (lanes 0-31, 32-63) */
__device__ __forceinline__ void kpv_to_lds(const NkChainArgs &a, Shared &sh, u32 l, u32 h, u32 pos, u32 cl, u32 lane) {
    const float *kvl = a.kv + (u64)l * a.kv_stride;
    const float *pt = a.L[l].ptab;
    const u32 L = cl + 1, half = lane >> 5, c4 = lane & 31;
    for (u32 r = 0; r < cl; r += 2) {
        const u32 row = r + half;
        if (row < cl) {
            const float *src = kvl + (u64)(pos - cl + row) * QKV + h * DH + 4 * c4;
            dma16(src + D, (lds_char_t *)&sh.ks[r][0]);
            dma16(src + 2 * D, (lds_char_t *)&sh.vs[r][0]);
        }
    }
    for (u32 r = 0; r < L; r += 2) {
        const u32 row = r + half;
        if (row < L) dma16(pt + (u64)(a.Lmax - L + row) * D + h * DH + 4 * c4, (lds_char_t *)&sh.ps[r][0]);
    }
}

/* Relative-position attention of head h for the chunk's one row (c = 1, i = 0), the math of
 * attention_rel: score_j = ((q + u) . K_j + (q + v) . P[Lmax - L + j]) * scale over the L window
 * rows (cached rows, then the row itself), softmax, O = sum_j p_j V_j.  256 threads: scores by
 * thread quads (key tid / 4, head dims 4 (tid % 4 + 4 t)), softmax on wavefront 0, the output by
 * 8 key groups of 32 threads summed in order.  Four LDS barriers, matched by the hand-off
 * wavefronts.  Returns dims 4 tid .. 4 tid + 3 on threads tid < 32. */
__device__ __forceinline__ floatx4 attend(Shared &sh, const float *q, floatx4 bu, floatx4 bv, u32 cl, float scale) {
    const u32 tid = threadIdx.x, L = cl + 1;
    if (tid < 32) {
        const floatx4 qx = *(const floatx4 *)(q + 4 * tid);
        sh.qu4[tid] = qx + bu;
        sh.qv4[tid] = qx + bv;
    }
    lds_barrier();
    const u32 ks = tid >> 2, part4 = tid & 3;
    float acc = 0.0f;
    if (ks < L) {
        const floatx4 *kr = (const floatx4 *)(ks < cl ? &sh.ks[ks][0] : sh.knew);
        const floatx4 *pr = (const floatx4 *)&sh.ps[ks][0];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const u32 cq = part4 + 4 * t;
            const floatx4 u = sh.qu4[cq], w = sh.qv4[cq], k = kr[cq], p = pr[cq];
            acc += u[0] * k[0] + u[1] * k[1] + u[2] * k[2] + u[3] * k[3];
            acc += w[0] * p[0] + w[1] * p[1] + w[2] * p[2] + w[3] * p[3];
        }
    }
    acc += dpp_f<DPP_QUAD_1032>(acc);
    acc += dpp_f<DPP_QUAD_2301>(acc);
    if (part4 == 0 && ks < L) sh.s[ks] = acc * scale;
    lds_barrier();
    if (tid < 64) {
        const float sv = tid < L ? sh.s[tid] : -INFINITY;
        const float mx = wmax(sv);
        const float ev = tid < L ? expf(sv - mx) : 0.0f;
        const float sum = wsum(ev);
        if (tid < L) sh.s[tid] = ev / sum;
    }
    lds_barrier();
    const u32 vg = tid >> 5, d4 = tid & 31;
    floatx4 o = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
    for (int t = 0; t < MAXL / 8; ++t) {
        const u32 j = vg + 8 * t;
        if (j < L) {
            const floatx4 *vr = (const floatx4 *)(j < cl ? &sh.vs[j][0] : sh.vnew);
            o += sh.s[j] * vr[d4];
        }
    }
    sh.part[vg][d4] = o;
    lds_barrier();
    floatx4 r = { 0.f, 0.f, 0.f, 0.f };
    if (tid < 32) {
        r = sh.part[0][tid];
#pragma unroll
        for (int gq = 1; gq < 8; ++gq) r += sh.part[gq][tid];
    }
    return r;
}

/* wavefronts 0-3 */
__device__ __forceinline__ void compute_loop(const NkChainArgs &a, Shared &sh, const Ctl &c, u32 g, u32 w, u32 lane) {
    const u32 nl = a.n_layers, tid = threadIdx.x;
    const u32 pos = (u32)a.desc[NK_DESC_POS], cl = (u32)a.desc[NK_DESC_CACHE];
    const bool attn = g < H;
    const u32 col1 = 4 * g + w;      /* this wavefront's column of the 1024-wide outputs */
    const u32 colA = 16 * g + 4 * w; /* first of its 4 columns of the 4096-wide outputs */
    const u32 colC = 12 * g + 3 * w; /* first of its 3 columns of q|k|v */
    uint4 wA[4][2], wB[1][8];
    ld_rows<4, 2>(wA, a.L[0].ff1_w1, colA, D, lane);
    ld_rows<1, 8>(wB, a.L[0].ff1_w2, col1, FF, lane);
    for (u32 l = 0; l < nl; ++l) {
        const NkChainLayer &W = a.L[l];
        const u32 h0 = 9 * l; /* hand-off index of this block's first input */
        float *kvl = a.kv + (u64)l * a.kv_stride;
        float *dinl = a.din + (u64)l * a.din_stride;

        /* A: ff1_w1 (LayerNorms applied by the hand-off wavefront), SiLU */
        lds_barrier();
        if (sh.bad) return;
        uint4 wC[3][2];
        ld_rows<3, 2>(wC, W.wqkv, colC, D, lane);
        {
            float x[2][8];
            ld_x<2>(x, sh.ib[h0 & 1], lane);
            float mine = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float s = silu_f(dot_row<2>(x, wA[j]));
                if (lane == (u32)j) mine = s;
            }
            if (lane < 4) ll_put(c.slot(h0 + 1), colA + lane, mine, c.tag(h0 + 1));
        }

        /* B: x + 0.5 * ff1_w2 h */
        lds_barrier();
        if (sh.bad) return;
        {
            float x[8][8];
            ld_x<8>(x, sh.ib[(h0 + 1) & 1], lane);
            const float s = dot_row<8>(x, wB[0]);
            const float v = sh.xr[0][col1] + s * 0.5f;
            if (lane == 0) ll_put(c.slot(h0 + 2), col1, v, c.tag(h0 + 2));
        }

        /* C: q|k|v of the normalised row, also written to the cache row */
        lds_barrier();
        if (sh.bad) return;
        uint4 wE[1][2];
        ld_rows<1, 2>(wE, W.wo, col1, D, lane);
        floatx4 bu = { 0.f, 0.f, 0.f, 0.f }, bv = bu;
        if (attn && tid < 32) {
            bu = ldg4(W.bias_u + g * DH + 4 * tid);
            bv = ldg4(W.bias_v + g * DH + 4 * tid);
        }
        {
            float x[2][8];
            ld_x<2>(x, sh.ib[(h0 + 2) & 1], lane);
            float mine = 0.0f;
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const float s = dot_row<2>(x, wC[j]);
                if (lane == (u32)j) mine = s;
            }
            if (lane < 3) {
                ll_put(c.slot(h0 + 3), colC + lane, mine, c.tag(h0 + 3));
                stg(kvl + (u64)pos * QKV + colC + lane, mine);
            }
        }

        /* D: attention of head g (workgroups 0 .. H-1) */
        lds_barrier();
        if (sh.bad) return;
        uint4 wF[2][2];
        {
            uint4 t0[1][2], t1[1][2];
            ld_rows<1, 2>(t0, W.pw1, col1, D, lane);
            ld_rows<1, 2>(t1, W.pw1, col1 + D, D, lane);
            wF[0][0] = t0[0][0]; wF[0][1] = t0[0][1];
            wF[1][0] = t1[0][0]; wF[1][1] = t1[0][1];
        }
        float taps[NK_CONV_TAPS], hist[NK_CONV_TAPS - 1];
#pragma unroll
        for (int t = 0; t < NK_CONV_TAPS; ++t) taps[t] = ldg(W.dw_w + col1 * NK_CONV_TAPS + t);
#pragma unroll
        for (int t = 0; t < NK_CONV_TAPS - 1; ++t) hist[t] = ldg(dinl + (u64)(pos - (NK_CONV_TAPS - 1) + t) * D + col1);
        if (attn) {
            const floatx4 r = attend(sh, sh.ib[(h0 + 3) & 1], bu, bv, cl, a.scale);
            if (tid < 32) {
                u64 *sl = c.slot(h0 + 4);
                const u32 tg = c.tag(h0 + 4), e0 = g * DH + 4 * tid;
                ll_put(sl, e0, r[0], tg);
                ll_put(sl, e0 + 1, r[1], tg);
                ll_put(sl, e0 + 2, r[2], tg);
                ll_put(sl, e0 + 3, r[3], tg);
            }
        }

        /* E: x + wo att */
        lds_barrier();
        if (sh.bad) return;
        uint4 wG[1][2];
        ld_rows<1, 2>(wG, W.pw2, col1, D, lane);
        {
            float x[2][8];
            ld_x<2>(x, sh.ib[(h0 + 4) & 1], lane);
            const float s = dot_row<2>(x, wE[0]);
            const float v = sh.xr[1][col1] + s;
            if (lane == 0) ll_put(c.slot(h0 + 5), col1, v, c.tag(h0 + 5));
        }

        /* F: pw1 GLU channel col1 (into the conv history), then its causal depthwise conv */
        lds_barrier();
        if (sh.bad) return;
        uint4 wH[4][2];
        ld_rows<4, 2>(wH, W.ff2_w1, colA, D, lane);
        {
            float x[2][8];
            ld_x<2>(x, sh.ib[(h0 + 5) & 1], lane);
            const float sa = dot_row<2>(x, wF[0]);
            const float sb = dot_row<2>(x, wF[1]);
            const float gl = sa * sigmoid_f(sb);
            float d = 0.0f;
#pragma unroll
            for (int t = 0; t < NK_CONV_TAPS - 1; ++t) d += taps[t] * hist[t];
            d += taps[NK_CONV_TAPS - 1] * gl;
            if (lane == 0) {
                stg(dinl + (u64)pos * D + col1, gl);
                ll_put(c.slot(h0 + 6), col1, d, c.tag(h0 + 6));
            }
        }

        /* G: x + pw2 SiLU(LN_bn(conv)) (normalised and activated by the hand-off wavefront) */
        lds_barrier();
        if (sh.bad) return;
        uint4 wI[1][8];
        ld_rows<1, 8>(wI, W.ff2_w2, col1, FF, lane);
        {
            float x[2][8];
            ld_x<2>(x, sh.ib[(h0 + 6) & 1], lane);
            const float s = dot_row<2>(x, wG[0]);
            const float v = sh.xr[0][col1] + s;
            if (lane == 0) ll_put(c.slot(h0 + 7), col1, v, c.tag(h0 + 7));
        }

        /* H: ff2_w1, SiLU */
        lds_barrier();
        if (sh.bad) return;
        /* the next block's first weights (the last block reloads its own: unconditional loads
         * keep the registers of the previous ones from staying live through the loop) */
        const NkChainLayer &Wn = a.L[l + 1 < nl ? l + 1 : l];
        ld_rows<4, 2>(wA, Wn.ff1_w1, colA, D, lane);
        {
            float x[2][8];
            ld_x<2>(x, sh.ib[(h0 + 7) & 1], lane);
            float mine = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float s = silu_f(dot_row<2>(x, wH[j]));
                if (lane == (u32)j) mine = s;
            }
            if (lane < 4) ll_put(c.slot(h0 + 8), colA + lane, mine, c.tag(h0 + 8));
        }

        /* I: x + 0.5 * ff2_w2 h: the next block's input, or the chain's output */
        lds_barrier();
        if (sh.bad) return;
        ld_rows<1, 8>(wB, Wn.ff1_w2, col1, FF, lane);
        {
            float x[8][8];
            ld_x<8>(x, sh.ib[(h0 + 8) & 1], lane);
            const float s = dot_row<8>(x, wI[0]);
            const float v = sh.xr[1][col1] + s * 0.5f;
            if (lane == 0) {
                if (l + 1 < nl) ll_put(c.slot(h0 + 9), col1, v, c.tag(h0 + 9));
                else stg(a.x_out + col1, v);
            }
        }
    }
}

/* wavefronts 4 and 5 */
__device__ __forceinline__ void handoff_loop(const NkChainArgs &a, Shared &sh, const Ctl &c, u32 g, u32 wave, u32 lane) {
    const u32 nl = a.n_layers;
    const u32 pos = (u32)a.desc[NK_DESC_POS], cl = (u32)a.desc[NK_DESC_CACHE];
    const bool attn = g < H, w4 = wave == 4;
    const float eps = a.eps;
    const u32 pl = threadIdx.x - 4 * 64; /* 0 .. 127 over both wavefronts */
    u32 e8[8], e16[16], eq[3];
#pragma unroll
    for (int i = 0; i < 8; ++i) e8[i] = 2 * (lane + 64 * i);
#pragma unroll
    for (int i = 0; i < 16; ++i) e16[i] = 2 * (pl + 128 * i);
#pragma unroll
    for (int i = 0; i < 3; ++i) eq[i] = i * D + g * DH + 2 * lane;
    if (w4) ln_params_to_lds(sh, 2, a.L[0].ln_ff1_g, a.L[0].ln_ff1_b, lane);
    else if (attn) kpv_to_lds(a, sh, 0, g, pos, cl, lane);
    for (u32 l = 0; l < nl; ++l) {
        const NkChainLayer &W = a.L[l];
        const u32 h0 = 9 * l;

        /* A: LN_out of the previous block (lnp[0..1]) gives the residual row, LN_ff1 (lnp[2..3])
         * the input of ff1_w1 */
        if (w4) {
            float2 v[8];
            bool ok = true;
            if (l == 0) {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = *(const float2 *)(a.x_in + e8[i]);
            } else {
                ok = ll_wait<8>(c, h0, e8, v);
            }
            if (!ok) {
                give_up(a, c, sh, h0);
            } else {
                wait_vm_lgkm<0>();
                if (l > 0) ln_lds(v, sh, 0, eps, lane);
                st_pairs(sh.xr[0], v, lane);
                if (l > 0 && a.dump && g == 0) st_pairs(a.dump + (u64)(l - 1) * D, v, lane);
                ln_lds(v, sh, 2, eps, lane);
                st_pairs(sh.ib[h0 & 1], v, lane);
            }
            ln_params_to_lds(sh, 0, W.ln_att_g, W.ln_att_b, lane);
        }
        lds_barrier();
        if (sh.bad) return;

        /* B: the 4096-wide row, both wavefronts */
        {
            float2 v[16];
            if (!ll_wait<16>(c, h0 + 1, e16, v)) give_up(a, c, sh, h0 + 1);
            else {
#pragma unroll
                for (int i = 0; i < 16; ++i) *(float2 *)(sh.ib[(h0 + 1) & 1] + e16[i]) = v[i];
            }
        }
        lds_barrier();
        if (sh.bad) return;

        /* C: LN_att */
        if (w4) {
            float2 v[8];
            if (!ll_wait<8>(c, h0 + 2, e8, v)) give_up(a, c, sh, h0 + 2);
            else {
                wait_vm_lgkm<0>();
                st_pairs(sh.xr[1], v, lane);
                ln_lds(v, sh, 0, eps, lane);
                st_pairs(sh.ib[(h0 + 2) & 1], v, lane);
            }
            ln_params_to_lds(sh, 0, W.ln_conv_g, W.ln_conv_b, lane);
        }
        lds_barrier();
        if (sh.bad) return;

        /* D: the head's q, k, v (attention workgroups) */
        if (attn) {
            if (w4) {
                float2 v[3];
                if (!ll_wait<3>(c, h0 + 3, eq, v)) give_up(a, c, sh, h0 + 3);
                else {
                    *(float2 *)(sh.ib[(h0 + 3) & 1] + 2 * lane) = v[0];
                    *(float2 *)(sh.knew + 2 * lane) = v[1];
                    *(float2 *)(sh.vnew + 2 * lane) = v[2];
                }
            } else {
                wait_vm_lgkm<0>(); /* the K, V and position rows have landed */
            }
        }
        lds_barrier();
        if (sh.bad) return;
        if (attn) {
            lds_barrier();
            lds_barrier();
            lds_barrier();
            lds_barrier();
        }

        /* E */
        if (w4) {
            float2 v[8];
            if (!ll_wait<8>(c, h0 + 4, e8, v)) give_up(a, c, sh, h0 + 4);
            else st_pairs(sh.ib[(h0 + 4) & 1], v, lane);
        }
        lds_barrier();
        if (sh.bad) return;

        /* F: LN_conv */
        if (w4) {
            float2 v[8];
            if (!ll_wait<8>(c, h0 + 5, e8, v)) give_up(a, c, sh, h0 + 5);
            else {
                wait_vm_lgkm<0>();
                st_pairs(sh.xr[0], v, lane);
                ln_lds(v, sh, 0, eps, lane);
                st_pairs(sh.ib[(h0 + 5) & 1], v, lane);
            }
            ln_params_to_lds(sh, 0, W.bn_g, W.bn_b, lane);
        } else if (attn && l + 1 < nl) {
            kpv_to_lds(a, sh, l + 1, g, pos, cl, lane); /* this block's attention has read them */
        }
        lds_barrier();
        if (sh.bad) return;

        /* G: SiLU(LN_bn(conv)) */
        if (w4) {
            float2 v[8];
            if (!ll_wait<8>(c, h0 + 6, e8, v)) give_up(a, c, sh, h0 + 6);
            else {
                wait_vm_lgkm<0>();
                ln_lds(v, sh, 0, eps, lane);
#pragma unroll
                for (int i = 0; i < 8; ++i) { v[i].x = silu_f(v[i].x); v[i].y = silu_f(v[i].y); }
                st_pairs(sh.ib[(h0 + 6) & 1], v, lane);
            }
            ln_params_to_lds(sh, 0, W.ln_ff2_g, W.ln_ff2_b, lane);
        }
        lds_barrier();
        if (sh.bad) return;

        /* H: LN_ff2; then the next block's LN_out (this block's) and LN_ff1 */
        if (w4) {
            float2 v[8];
            if (!ll_wait<8>(c, h0 + 7, e8, v)) give_up(a, c, sh, h0 + 7);
            else {
                wait_vm_lgkm<0>();
                st_pairs(sh.xr[1], v, lane);
                ln_lds(v, sh, 0, eps, lane);
                st_pairs(sh.ib[(h0 + 7) & 1], v, lane);
            }
            if (l + 1 < nl) {
                ln_params_to_lds(sh, 0, W.ln_out_g, W.ln_out_b, lane);
                ln_params_to_lds(sh, 2, a.L[l + 1].ln_ff1_g, a.L[l + 1].ln_ff1_b, lane);
            }
        }
        lds_barrier();
        if (sh.bad) return;

        /* I: the 4096-wide row, both wavefronts */
        {
            float2 v[16];
            if (!ll_wait<16>(c, h0 + 8, e16, v)) give_up(a, c, sh, h0 + 8);
            else {
#pragma unroll
                for (int i = 0; i < 16; ++i) *(float2 *)(sh.ib[(h0 + 8) & 1] + e16[i]) = v[i];
            }
        }
        lds_barrier();
        if (sh.bad) return;
    }
}

} // namespace chain

extern "C" __global__ __launch_bounds__(NK_CHAIN_THREADS) void enc_chain(const NkChainArgs a) {
    __shared__ chain::Shared sh;
    const u32 tid = threadIdx.x, lane = tid & 63, g = blockIdx.x;
    const u32 wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    chain::Ctl c;
    c.ll = a.ll;
    c.abort_word = a.abort_word;
    c.epoch = (u32)a.desc[NK_DESC_EPOCH];
    c.base = c.epoch << 10;
    c.spin_max = a.spin_max;
    if (tid == 0) sh.bad = 0;
    __syncthreads();
    if (wave < 4) chain::compute_loop(a, sh, c, g, wave, lane);
    else chain::handoff_loop(a, sh, c, g, wave, lane);
    wait_vm_lgkm<0>(); /* no direct-to-LDS load outlives the workgroup */
}
