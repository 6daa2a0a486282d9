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
 *   D  relative-position attention: 4 workgroups per head, each over a quarter of the window,
 *      hand over their unnormalised outputs with their softmax max and sum  (8 x 4 x 130)
 *   E  merge of the quarters, x + wo att               (1024)   src/encoder.c:163-165
 *   F  LN_conv -> pw1, GLU (written to the conv history) -> causal depthwise conv  (1024)
 *   G  LN_bn -> SiLU -> x + pw2 y                       (1024)   src/encoder.c:169-175
 *   H  LN_ff2 -> ff2_w1, SiLU                           (4096)   src/encoder.c:177-179
 *   I  x + 0.5 * ff2_w2 h                              (1024)   (LN_out in the next block's A)
 * The math of each operation is that of the per-kernel path (reference src/kernels.metal: GEMMs
 * with bf16 weights and f32 activations :51-118, LayerNorm :211-255, attention :290-348, conv
 * :359-409); only the summation orders differ (the attention's softmax is summed per quarter and
 * the quarters combined with their max: the same value up to rounding).
 *
 * Hand-off.  An entry is 8 bytes {f32 value, u32 tag}, stored with one agent-coherent (sc1)
 * 8-byte store, so value and tag arrive together: no flag, no fence, no counter.  The reader
 * loads 16 bytes (two entries) per lane with sc1 loads and retries until every entry it needs
 * carries the tag of this hand-off.  Tag = epoch * 1024 + hand-off index; the epoch comes from
 * the chunk descriptor and differs on consecutive chunks, so entries of the previous chunk never
 * match.  Hand-off i uses slot i mod 3: a slot is rewritten three hand-offs later, and by then
 * every reader of its previous contents has finished (a writer of hand-off i + 3 has seen all of
 * hand-off i + 2, whose writers had all seen i + 1, whose writers are, directly or through the
 * attention workgroups, every workgroup that waits for i).  Two slots would not do: hand-off
 * D -> E is written by the attention workgroups alone, which do not wait for all of C -> D.
 * Every wait is bounded (spin_max polls, and the epoch written to abort_word by any workgroup
 * that gave up ends the others' waits), and a time-out is reported in the host-visible err_word.
 *
 * Weight stream.  A CU keeps only so many lines in flight, so a wavefront that issues a burst of
 * loads stalls until they drain; issued by the wavefronts that compute, the weight loads would
 * put that stall on every phase's critical path.  Instead one wavefront per workgroup streams the
 * workgroup's whole sequence of weight slices (with the LayerNorm parameters, the conv taps and
 * history and, in the attention workgroups, the head's K, V and position rows) into a 120 KB LDS
 * area by direct-to-LDS loads, two phases ahead: after the barrier of phase p it issues the
 * segment of phase p + 2, then waits for the segment of phase p + 1 before the next barrier.
 * Each kind of phase has a segment of fixed size (SEG_*) at a fixed place in the area (AT_*),
 * chosen so that any three consecutive segments are disjoint: every LDS address of a weight block
 * is a constant of the code that reads it.
 *
 * Roles within a workgroup (7 wavefronts, one LDS barrier per phase):
 *   - wavefronts 0-3 compute: read the phase's input row and their weight rows from LDS (lane l
 *     holds 16-byte chunks l, l + 64, ... of a weight row), reduce the dot products across the
 *     wavefront and store the outputs as hand-off entries;
 *   - wavefront 4 waits for the next phase's input while they compute, applies that phase's
 *     LayerNorm (the whole row: every workgroup normalises it itself) with parameters from the
 *     weight area, keeps the residual row and writes the input row to LDS for the next barrier;
 *   - wavefront 5 shares the waits of the 4096-wide rows;
 *   - wavefront 6 streams the weights. */
#include "nk_common.h"

namespace chain {

constexpr u32 G = NK_CHAIN_G, D = NK_CHAIN_D, FF = NK_CHAIN_FF, QKV = 3 * NK_CHAIN_D, H = NK_CHAIN_HEADS, DH = 128;
constexpr u32 NP = NK_CHAIN_PARTS, NATT = H * NP, SLOT = NK_CHAIN_SLOT, MAXL = NK_CHAIN_MAX_L;
constexpr u32 ML = H * NP * DH; /* E-input entry of the attention quarters' (max, sum) pairs */
constexpr u32 RING = 120;       /* KB */
/* Direct-to-LDS loads the streaming wavefront keeps in flight.  The CU's vector memory queue is
 * shared by all its wavefronts: a deeper stream would hold the hand-off stores and waits of the
 * other wavefronts behind it. */
constexpr int STREAM_INFLIGHT = 16;
/* segment of each kind of phase: its size and its first block in the area (KB blocks) */
constexpr u32 SEG_A = 32, SEG_B = 40, SEG_C = 24, SEG_D = 25, SEG_E = 16, SEG_F = 25, SEG_G = 16, SEG_H = 32, SEG_I = 48;
constexpr u32 AT_A = 88, AT_B = 48, AT_C = 0, AT_D = 88, AT_E = 25, AT_F = 0, AT_G = 80, AT_H = 48, AT_I = 0;
constexpr u32 SEG_N[9] = { SEG_A, SEG_B, SEG_C, SEG_D, SEG_E, SEG_F, SEG_G, SEG_H, SEG_I };
constexpr u32 SEG_AT[9] = { AT_A, AT_B, AT_C, AT_D, AT_E, AT_F, AT_G, AT_H, AT_I };
constexpr bool seg_apart(u32 j, u32 k) { return SEG_AT[j] + SEG_N[j] <= SEG_AT[k] || SEG_AT[k] + SEG_N[k] <= SEG_AT[j]; }
constexpr bool segs_placed() {
    for (u32 j = 0; j < 9; ++j)
        if (SEG_AT[j] + SEG_N[j] > RING || !seg_apart(j, (j + 1) % 9) || !seg_apart(j, (j + 2) % 9)) return false;
    return true;
}
static_assert(H * DH == D && G * 4 == D && G * 16 == FF && G * 12 == QKV, "slices assume these shapes");
static_assert(ML + 2 * NATT <= SLOT && NATT <= G && MAXL % NP == 0 && MAXL / NP <= 16, "attention split");
static_assert(segs_placed(), "every segment lies in the area and apart from the next two (the phase in flight and the one "
                             "computing)");
static_assert(SEG_A >= STREAM_INFLIGHT && SEG_B >= STREAM_INFLIGHT && SEG_C >= STREAM_INFLIGHT &&
                  SEG_D >= STREAM_INFLIGHT && SEG_E >= STREAM_INFLIGHT && SEG_F >= STREAM_INFLIGHT &&
                  SEG_G >= STREAM_INFLIGHT && SEG_H >= STREAM_INFLIGHT && SEG_I >= STREAM_INFLIGHT,
              "a nonempty segment holds more loads than are in flight");

struct Shared {
    char ring[RING * 1024]; /* the weight area: each kind of phase's segment at its fixed place */
    float big[FF + 2 * NATT]; /* inputs of B, E (with the heads' merge weights), I */
    float sm[2][D];           /* inputs of A, C, F, H (sm[0]) and D, G (sm[1]) */
    float xr[2][D];           /* residual rows (alternating) */
    float knew[DH], vnew[DH]; /* attention: the chunk's own K and V of the head */
    floatx4 qu4[32], qv4[32];
    float s[MAXL];
    floatx4 part[8][32];
    float outv[16], aux[4];   /* the compute wavefronts' outputs of a phase, stored by the last one */
    float att_out[DH];        /* the attention quarter's output, stored by wavefront 0 */
    u32 done;                 /* compute wavefronts finished, counted across phases */
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

/* Wavefront-wide wait: load i of this lane covers entries e0 + i * es, +1 of the slot of hand-off
 * `hand`; returns once every entry of the wavefront carries its tag, with the values in v (false
 * after spin_max rounds, or once another workgroup has given up on this epoch).  Every workgroup
 * waits at once, so the wait keeps its memory traffic small: after a full pass that finds entries
 * missing it re-reads only the first incomplete group (one 16-byte load per lane) until that group
 * is complete, then makes the next full pass. */
template <int NL>
__device__ __forceinline__ bool ll_wait(const Ctl &c, u32 hand, u32 e0, u32 es, float2 (&v)[NL]) {
    const u64 *slot = c.slot(hand);
    const u32 tag = c.tag(hand);
    u32 spins = 0;
    for (;;) {
        /* the complete pass is the one on the hand-off's critical path: one test per lane for all
         * its groups (a vector OR of the tag differences), the first incomplete group only
         * sought after a failed pass */
        u32x4 r[NL];
        u32 miss = 0;
#pragma unroll
        for (int i = 0; i < NL; ++i) r[i] = ll_load(slot, e0 + i * es);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            v[i] = make_float2(__uint_as_float(r[i].x), __uint_as_float(r[i].z));
            miss |= (r[i].y ^ tag) | (r[i].w ^ tag);
        }
        if (__all(miss == 0)) return true;
        u32 first_bad = NL - 1;
#pragma unroll
        for (int i = NL - 2; i >= 0; --i)
            if (!__all((r[i].y == tag) & (r[i].w == tag))) first_bad = i;
        const u32 eb = e0 + first_bad * es;
        for (;;) {
            if (++spins > c.spin_max) return false;
            if ((spins & 255) == 0 && __hip_atomic_load(c.abort_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == c.epoch)
                return false;
            const u32x4 u = ll_load(slot, eb);
            if (__all((u.y == tag) & (u.w == tag))) break;
        }
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

/* block kb of the weight area */
__device__ __forceinline__ const char *rblk(const Shared &sh, u32 kb) { return sh.ring + kb * 1024; }
__device__ __forceinline__ uint4 rw16(const Shared &sh, u32 kb, u32 lane) { return *(const uint4 *)(rblk(sh, kb) + 16 * lane); }

/* x * sigmoid(x) with the hardware exp2 and reciprocal (about 1 ulp each): one wavefront
 * evaluates it on a whole 1024-row between a hand-off and the next GEMV */
__device__ __forceinline__ float silu_fast(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

/* LayerNorm of a 1024-row held as float2 pairs by one wavefront (lane l: elements 2(l + 64i),
 * +1): mean, then the centred variance (the reference's two passes, summed in another order),
 * y = (x - mean) * rsqrt(var + eps) * g + b (hardware reciprocal square root, about 1 ulp). */
__device__ __forceinline__ void ln_pairs(float2 (&v)[8], const float2 (&g)[8], const float2 (&b)[8], float eps) {
    /* the lane's 16 terms summed as a tree (a short dependent chain), then across the wavefront */
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = v[i].x + v[i].y;
    const float mean = wsum(((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]))) / (float)D;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float d0 = v[i].x - mean, d1 = v[i].y - mean;
        t[i] = d0 * d0 + d1 * d1;
    }
    const float inv = __builtin_amdgcn_rsqf(wsum(((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]))) / (float)D + eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i].x = (v[i].x - mean) * inv * g[i].x + b[i].x;
        v[i].y = (v[i].y - mean) * inv * g[i].y + b[i].y;
    }
}

/* LayerNorm with its parameters in the weight area: gamma in the 4 blocks from kg, beta from kb */
__device__ __forceinline__ void ln_ring(float2 (&v)[8], const Shared &sh, u32 kg, u32 kb, float eps, u32 lane) {
    float2 g[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        g[i] = *(const float2 *)(rblk(sh, kg + (i >> 1)) + 8 * lane + 512 * (i & 1));
        b[i] = *(const float2 *)(rblk(sh, kb + (i >> 1)) + 8 * lane + 512 * (i & 1));
    }
    ln_pairs(v, g, b, eps);
}

__device__ __forceinline__ void st_pairs(float *dst, const float2 (&v)[8], u32 lane) {
#pragma unroll
    for (int i = 0; i < 8; ++i) *(float2 *)(dst + 2 * (lane + 64 * i)) = v[i];
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

/* dot product of the weight row in blocks kb .. kb + KCH - 1 with the row held in x, summed
 * over the wavefront (uniform) */
template <int KCH>
__device__ __forceinline__ float dot_ring(const float (&x)[KCH][8], const Shared &sh, u32 kb, u32 lane) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < KCH; ++q) s = dot8(x[q], rw16(sh, kb + q, lane), s);
    return wsum(s);
}

/* dot products of NR weight rows of K = 1024 (blocks kb[k], kb[k] + 1) with the row in x,
 * each summed over the wavefront (uniform): every LDS read first, then the sums side by side */
template <int NR>
__device__ __forceinline__ void dots_ring(float (&sums)[NR], const float (&x)[2][8], const Shared &sh, const u32 (&kb)[NR], u32 lane) {
    uint4 wv[NR][2];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
        wv[k][0] = rw16(sh, kb[k], lane);
        wv[k][1] = rw16(sh, kb[k] + 1, lane);
    }
    float acc[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) acc[k] = dot8(x[1], wv[k][1], dot8(x[0], wv[k][0], 0.0f));
#pragma unroll
    for (int k = 0; k < NR; ++k) sums[k] = wsum(acc[k]);
}

/* The attention quarter of this workgroup: head h's window rows j0 .. j0 + nk - 1 (cached rows,
 * then the row itself) with the math of attention_rel: score_j = ((q + u) . K_j + (q + v) .
 * P[Lmax - L + j]) * scale, m = max score, p_j = exp(score_j - m), l = sum p_j, o = sum p_j V_j
 * (unnormalised; the E phase combines the quarters).  256 threads: scores by thread quads (key
 * tid / 4, head dims 4 (tid % 4 + 4 t)), the exponentials on wavefront 0, the output by 8 key
 * groups of 32 threads summed in order.  K, V and P rows are in the segment at block kd (K rows
 * 2 per block from kd, V from kd + 8, P from kd + 16, then u | v in kd + 24).  Four LDS barriers,
 * matched by the other wavefronts.  Returns o[4 tid .. 4 tid + 3] on threads tid < 32. */
__device__ __forceinline__ floatx4 attend_part(Shared &sh, u32 kd, const float *q, u32 cl, u32 j0, u32 nk, float scale,
                                               float &m_out, float &l_out) {
    const u32 tid = threadIdx.x;
    const float *uv = (const float *)rblk(sh, kd + 24);
    if (tid < 32) {
        const floatx4 qx = *(const floatx4 *)(q + 4 * tid);
        sh.qu4[tid] = qx + *(const floatx4 *)(uv + 4 * tid);
        sh.qv4[tid] = qx + *(const floatx4 *)(uv + DH + 4 * tid);
    }
    lds_barrier();
    const u32 ks = tid >> 2, part4 = tid & 3;
    float acc = 0.0f;
    if (ks < nk) {
        const floatx4 *kr = (const floatx4 *)(j0 + ks < cl ? rblk(sh, kd + (ks >> 1)) + 512 * (ks & 1) : (const char *)sh.knew);
        const floatx4 *pr = (const floatx4 *)(rblk(sh, kd + 16 + (ks >> 1)) + 512 * (ks & 1));
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
    if (part4 == 0 && ks < nk) sh.s[ks] = acc * scale;
    lds_barrier();
    if (tid < 64) {
        const float sv = tid < nk ? sh.s[tid] : -INFINITY;
        const float mx = wmax(sv);
        const float ev = tid < nk ? expf(sv - mx) : 0.0f;
        const float sum = wsum(ev);
        if (tid < nk) sh.s[tid] = ev;
        if (tid == 0) {
            sh.s[MAXL - 2] = mx;
            sh.s[MAXL - 1] = sum;
        }
    }
    lds_barrier();
    const u32 vg = tid >> 5, d4 = tid & 31;
    floatx4 o = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const u32 jj = vg + 8 * t;
        if (jj < nk) {
            const floatx4 *vr = (const floatx4 *)(j0 + jj < cl ? rblk(sh, kd + 8 + (jj >> 1)) + 512 * (jj & 1)
                                                                : (const char *)sh.vnew);
            o += sh.s[jj] * vr[d4];
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
    m_out = sh.s[MAXL - 2];
    l_out = sh.s[MAXL - 1];
    return r;
}

/* The lane's chunks (as ld_x<2>) of the attention output: each head's quarters combined,
 * att = sum_k w_k o_k in quarter order, with the merge weights w_k = exp(m_k - max m) /
 * sum_k' exp(m_k' - max m) l_k' that the hand-off wavefront left after the quarters' outputs. */
__device__ __forceinline__ void ld_att(float (&x)[2][8], const Shared &sh, u32 lane) {
    static_assert(NP == 4, "one floatx4 of merge weights per head");
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const u32 hh = (lane >> 4) + 4 * q, d0 = 8 * (lane & 15);
        const floatx4 w = *(const floatx4 *)(sh.big + ML + NP * hh);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float o = 0.0f;
#pragma unroll
            for (int k = 0; k < (int)NP; ++k) o += w[k] * sh.big[(hh * NP + k) * DH + d0 + i];
            x[q][i] = o;
        }
    }
}

/* the window quarter of attention workgroup part k: rows j0 .. j0 + nk - 1 of the L rows */
struct Quarter {
    u32 j0, nk;
};
__device__ __forceinline__ Quarter quarter(u32 L, u32 k) {
    const u32 S = (L + NP - 1) / NP, j0 = k * S;
    return { j0, L > j0 ? min(S, L - j0) : 0u };
}

/* Phase j = p % 9 of block l = p / 9 reads hand-off p (its input) and writes hand-off p + 1.  The
 * three loops below run every phase through one copy of their code (the whole kernel must stay
 * resident in the instruction cache, which the CU pair shares: unrolled per phase, the code of the
 * seven wavefronts missed it at every phase). */
constexpr u32 PH_A = 0, PH_B = 1, PH_C = 2, PH_D = 3, PH_E = 4, PH_F = 5, PH_G = 6, PH_H = 7, PH_I = 8;

/* wavefronts 0-3 */
__device__ __forceinline__ void compute_loop(const NkChainArgs &a, Shared &sh, const Ctl &c, u32 g, u32 w, u32 lane) {
    const u32 nl = a.n_layers, tid = threadIdx.x, P = NK_CHAIN_PH * nl;
    const u32 pos = (u32)a.desc[NK_DESC_POS], cl = (u32)a.desc[NK_DESC_CACHE], L = cl + 1;
    const bool attn = g < NATT;
    const Quarter qt = quarter(L, g % NP);
    const u32 col1 = 4 * g + w; /* this wavefront's column of the 1024-wide outputs */
#pragma nounroll
    for (u32 p = 0; p < P; ++p) {
        const u32 l = p / NK_CHAIN_PH, j = p % NK_CHAIN_PH;
        u64 *out = c.slot(p + 1);
        const u32 tag = c.tag(p + 1);
        lds_barrier();
        if (sh.bad) return;
        if (j == PH_D) {
            /* attention quarter (workgroups 0 .. NATT-1): its unnormalised output and (max, sum),
             * stored by wavefront 0 as two 512-byte runs of entries and one pair */
            if (attn) {
                float m, lsum;
                const floatx4 r = attend_part(sh, AT_D, sh.sm[1], cl, qt.j0, qt.nk, a.scale, m, lsum);
                if (tid < 32) *(floatx4 *)&sh.att_out[4 * tid] = r;
                if (w == 0) {
                    ll_put(out, g * DH + lane, sh.att_out[lane], tag);
                    ll_put(out, g * DH + 64 + lane, sh.att_out[64 + lane], tag);
                    if (lane < 2) ll_put(out, ML + 2 * g + lane, lane ? lsum : m, tag);
                }
            }
            continue;
        }
        /* Each wavefront leaves its outputs in LDS; the last of the four to finish stores the
         * workgroup's entries with one instruction (entries of one 32-byte run written by four
         * wavefronts separately reach the other workgroups measurably later). */
        u32 n_out, e_out; /* entries of the workgroup and the first of them */
        if (j == PH_B || j == PH_I) {
            /* x + 0.5 * ff_w2 h: one row of K = 4096 per wavefront */
            float x[8][8];
            ld_x<8>(x, sh.big, lane);
            const float s = dot_ring<8>(x, sh, (j == PH_B ? AT_B : AT_I) + 8 * w, lane);
            if (lane == 0) sh.outv[w] = sh.xr[j == PH_B ? 0 : 1][col1] + s * 0.5f;
            n_out = 4;
            e_out = 4 * g;
        } else {
            /* K = 1024: A, H (4 rows, SiLU), C (3 rows of q|k|v), E (wo on the merged attention),
             * F (the GLU pair, then the causal depthwise conv), G (pw2) */
            float x[2][8];
            if (j == PH_E) ld_att(x, sh, lane);
            else ld_x<2>(x, sh.sm[j == PH_G ? 1 : 0], lane);
            if (j == PH_A || j == PH_H) {
                const u32 kb = (j == PH_A ? AT_A : AT_H) + 8 * w; /* rows 4w .. 4w+3 */
                const u32 kbs[4] = { kb, kb + 2, kb + 4, kb + 6 };
                float sums[4];
                dots_ring<4>(sums, x, sh, kbs, lane);
                const float mine = lane == 0 ? sums[0] : lane == 1 ? sums[1] : lane == 2 ? sums[2] : sums[3];
                if (lane < 4) sh.outv[4 * w + lane] = silu_f(mine);
                n_out = 16;
                e_out = 16 * g;
            } else if (j == PH_C) {
                const u32 kb = AT_C + 6 * w; /* rows 3w .. 3w+2 */
                const u32 kbs[3] = { kb, kb + 2, kb + 4 };
                float sums[3];
                dots_ring<3>(sums, x, sh, kbs, lane);
                if (lane < 3) sh.outv[3 * w + lane] = lane == 0 ? sums[0] : lane == 1 ? sums[1] : sums[2];
                n_out = 12;
                e_out = 12 * g;
            } else if (j == PH_F) {
                const u32 kbs[2] = { AT_F + 2 * w, AT_F + 2 * (4 + w) }; /* GLU rows w, 4 + w */
                float sums[2];
                dots_ring<2>(sums, x, sh, kbs, lane);
                const float gl = sums[0] * sigmoid_f(sums[1]);
                const float *th = (const float *)rblk(sh, AT_F + 16); /* taps [4][9], then history [8][4] */
                float d = 0.0f;
#pragma unroll
                for (int t = 0; t < NK_CONV_TAPS - 1; ++t) d += th[w * NK_CONV_TAPS + t] * th[4 * NK_CONV_TAPS + 4 * t + w];
                d += th[w * NK_CONV_TAPS + NK_CONV_TAPS - 1] * gl;
                if (lane == 0) {
                    sh.aux[w] = gl;
                    sh.outv[w] = d;
                }
                n_out = 4;
                e_out = 4 * g;
            } else {
                const u32 kbs[1] = { (j == PH_E ? AT_E : AT_G) + 2 * w };
                float sums[1];
                dots_ring<1>(sums, x, sh, kbs, lane);
                if (lane == 0) sh.outv[w] = sh.xr[j == PH_E ? 1 : 0][col1] + sums[0];
                n_out = 4;
                e_out = 4 * g;
            }
        }
        u32 before = 0;
        if (lane == 0) before = atomicAdd(&sh.done, 1u);
        if ((__builtin_amdgcn_readfirstlane(before) & 3) == 3) {
            /* the last wavefront: the others' LDS writes precede their count */
            if (lane < n_out) {
                const float v = sh.outv[lane];
                if (p + 1 < P) ll_put(out, e_out + lane, v, tag);
                else a.x_out[e_out + lane] = v;
                if (j == PH_C) a.kv[(u64)l * a.kv_stride + (u64)pos * QKV + e_out + lane] = v;
                if (j == PH_F) a.din[(u64)l * a.din_stride + (u64)pos * D + e_out + lane] = sh.aux[lane];
            }
        }
    }
}

/* wavefronts 4 and 5: the input of phase p + 1 while phase p computes */
__device__ __forceinline__ void handoff_loop(const NkChainArgs &a, Shared &sh, const Ctl &c, u32 g, u32 wave, u32 lane) {
    const u32 nl = a.n_layers, P = NK_CHAIN_PH * nl;
    const u32 cl = (u32)a.desc[NK_DESC_CACHE], L = cl + 1;
    const bool attn = g < NATT, w4 = wave == 4;
    const u32 head = g / NP;
    const Quarter qt = quarter(L, g % NP);
    const bool has_new = qt.j0 + qt.nk == L && qt.nk > 0; /* this quarter holds the chunk's own row */
    const float eps = a.eps;
    const u32 pl = threadIdx.x - 4 * 64; /* 0 .. 127 over both wavefronts */
    float2 f_g[8], f_b[8];               /* block 0's LN_ff1 (later blocks take it from the weight area) */
    if (w4) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            f_g[i] = *(const float2 *)(a.L[0].ln_ff1_g + 2 * (lane + 64 * i));
            f_b[i] = *(const float2 *)(a.L[0].ln_ff1_b + 2 * (lane + 64 * i));
        }
    }
#pragma nounroll
    for (u32 p = 0; p < P; ++p) {
        const u32 l = p / NK_CHAIN_PH, j = p % NK_CHAIN_PH;
        bool ok = true;
        if (j == PH_B || j == PH_E || j == PH_I) {
            /* the 4096-wide row, both wavefronts (E: the attention quarters' outputs, then their
             * (max, sum) pairs) */
            float2 v[16];
            ok = ll_wait<16>(c, p, 2 * pl, 256, v);
            if (ok) {
#pragma unroll
                for (int i = 0; i < 16; ++i) *(float2 *)(sh.big + 2 * (pl + 128 * i)) = v[i];
                if (j == PH_E && w4) {
                    /* lane g (and g + 32): quarter g's (max, sum); its weight in the merge of its
                     * head (quarters 4h .. 4h + 3 in lanes 4h .. 4h + 3), in ld_att's order:
                     * w = exp(m - max m) / ((e0 l0 + e1 l1) + e2 l2) + e3 l3 */
                    float2 u[1];
                    ok = ll_wait<1>(c, p, ML + 2 * (lane & 31), 0, u);
                    if (ok) {
                        const float m = u[0].x;
                        const float mx = fmaxf(fmaxf(fmaxf(fmaxf(-INFINITY, dpp_f<DPP_QUAD_0000>(m)), dpp_f<DPP_QUAD_1111>(m)),
                                                     dpp_f<DPP_QUAD_2222>(m)),
                                               dpp_f<DPP_QUAD_3333>(m));
                        const float e = expf(m - mx), el = e * u[0].y;
                        const float lsum = ((dpp_f<DPP_QUAD_0000>(el) + dpp_f<DPP_QUAD_1111>(el)) + dpp_f<DPP_QUAD_2222>(el)) +
                                           dpp_f<DPP_QUAD_3333>(el);
                        if (lane < 32) sh.big[ML + lane] = e * (1.0f / lsum);
                    }
                }
            }
        } else if (j == PH_D) {
            /* the head's q (and k, v in the quarter that holds the chunk's row) */
            if (attn && w4) {
                float2 v[3];
                ok = ll_wait<3>(c, p, head * DH + 2 * lane, has_new ? D : 0, v);
                if (ok) {
                    *(float2 *)(sh.sm[1] + 2 * lane) = v[0];
                    if (has_new) {
                        *(float2 *)(sh.knew + 2 * lane) = v[1];
                        *(float2 *)(sh.vnew + 2 * lane) = v[2];
                    }
                }
            }
        } else if (w4) {
            /* a 1024-wide row: A (LN_out of the previous block gives the residual row, LN_ff1 the
             * GEMV input, both from the previous block's I segment; block 0 reads its input row
             * and keeps LN_ff1 in registers), C (LN_att, B segment), F (LN_conv, E segment),
             * G (LN_bn then SiLU, F segment), H (LN_ff2, G segment); C, F, H keep the row itself
             * as the residual */
            float2 v[8];
            if (p == 0) {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = *(const float2 *)(a.x_in + 2 * (lane + 64 * i));
            } else {
                ok = ll_wait<8>(c, p, 2 * lane, 128, v);
            }
            if (ok) {
                if (j == PH_A) {
                    if (l > 0) ln_ring(v, sh, AT_I + 32, AT_I + 36, eps, lane);
                    st_pairs(sh.xr[0], v, lane);
                    if (l > 0 && a.dump && g == 0) st_pairs(a.dump + (u64)(l - 1) * D, v, lane);
                    if (l > 0) ln_ring(v, sh, AT_I + 40, AT_I + 44, eps, lane);
                    else ln_pairs(v, f_g, f_b, eps);
                } else {
                    if (j != PH_G) st_pairs(sh.xr[j == PH_F ? 0 : 1], v, lane);
                    const u32 kg = j == PH_C ? AT_B + 32 : j == PH_F ? AT_E + 8 : j == PH_G ? AT_F + 17 : AT_G + 8;
                    ln_ring(v, sh, kg, kg + 4, eps, lane);
                    if (j == PH_G) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            v[i].x = silu_fast(v[i].x);
                            v[i].y = silu_fast(v[i].y);
                        }
                    }
                }
                st_pairs(sh.sm[j == PH_G ? 1 : 0], v, lane);
            }
        }
        if (!ok) give_up(a, c, sh, p);
        lds_barrier();
        if (sh.bad) return;
        if (j == PH_D && attn) { /* the attention's four barriers */
            lds_barrier();
            lds_barrier();
            lds_barrier();
            lds_barrier();
        }
    }
}

typedef __attribute__((address_space(4))) const NkChainLayer const_layer_t;

/* Segment p of the stream (block p / 9, phase j = p % 9) into the weight area: its KB blocks go
 * to blocks AT_j + i, one direct-to-LDS load of 16 bytes per lane each; the count of loads per
 * segment is fixed (SEG_j; none for D outside the attention workgroups). */
struct Stream {
    const_layer_t *Lt; /* constant address space: the pointers are read with scalar loads, which
                        * do not count in vmcnt (a vector load would need a vmcnt(0) wait, i.e. for
                        * every segment in flight) */
    const float *kv, *din;
    u64 kv_stride, din_stride;
    lds_char_t *ring; /* the LDS ring as an LDS address (a generic pointer here miscompiles) */
    u32 g, lane, pos, cl, L, head, Lmax, nl;
    Quarter qt;
    bool attn;
    __device__ void put(u32 kb, const void *src) const {
        wait_vm_lgkm<STREAM_INFLIGHT - 1>();
        dma16(src, ring + kb * 1024);
    }
    /* n rows of nb blocks from src, rows row_bytes apart: block q of row r is bytes
     * [1024 q, 1024 q + 1024) of that row (16 bytes per lane) */
    __device__ void blocks(u32 kb, const void *src, u64 row_bytes, u32 n, u32 nb) const {
        const char *s = (const char *)src + 16 * lane;
#pragma nounroll
        for (u32 r = 0; r < n; ++r)
#pragma nounroll
            for (u32 q = 0; q < nb; ++q) put(kb + r * nb + q, s + r * row_bytes + 1024 * q);
    }
    /* rows r0 .. r0 + n - 1 of a [.][K] bf16 matrix; a D-float vector */
    __device__ void rows(u32 kb, const u16 *W, u32 r0, u32 n, u32 K) const { blocks(kb, W + (u64)r0 * K, 2ull * K, n, K / 512); }
    __device__ void vec(u32 kb, const float *p) const { blocks(kb, p, 0, 1, D / 256); }
    __device__ void seg(u32 p) const {
        const u32 l = p / NK_CHAIN_PH, j = p % NK_CHAIN_PH;
        const_layer_t &W = Lt[l];
        if (j == PH_A) {
            rows(AT_A, W.ff1_w1, 16 * g, 16, D);
        } else if (j == PH_B) {
            rows(AT_B, W.ff1_w2, 4 * g, 4, FF);
            vec(AT_B + 32, W.ln_att_g);
            vec(AT_B + 36, W.ln_att_b);
        } else if (j == PH_C) {
            rows(AT_C, W.wqkv, 12 * g, 12, D);
        } else if (j == PH_D) {
            if (attn) {
                /* K, V rows of the quarter's cached window rows, P rows of all its rows (two rows
                 * of 128 floats per block; rows past the quarter repeat a valid row) */
                const float *kvl = kv + (u64)l * kv_stride;
                const u32 half = lane >> 5, c4 = 4 * (lane & 31);
#pragma nounroll
                for (u32 b = 0; b < 8; ++b) {
                    const u32 jr = qt.j0 + 2 * b + half;
                    const u32 kvrow = cl > 0 ? pos - cl + min(jr, cl - 1) : pos;
                    const float *src = kvl + (u64)kvrow * QKV + head * DH + c4;
                    put(AT_D + b, src + D);
                    put(AT_D + 8 + b, src + 2 * D);
                    put(AT_D + 16 + b, W.ptab + (u64)(Lmax - L + min(jr, L - 1)) * D + head * DH + c4);
                }
                /* u for lanes 0-31, v for 32-63, as an offset from u: a per-lane choice of which
                 * table entry to read would make the read a vector load (and a vmcnt(0) wait) */
                const u64 bu = (u64)W.bias_u, dv = (u64)W.bias_v - bu;
                put(AT_D + 24, (const float *)(bu + (half ? dv : 0)) + head * DH + c4);
            }
        } else if (j == PH_E) {
            rows(AT_E, W.wo, 4 * g, 4, D);
            vec(AT_E + 8, W.ln_conv_g);
            vec(AT_E + 12, W.ln_conv_b);
        } else if (j == PH_F) {
            rows(AT_F, W.pw1, 4 * g, 4, D);
            rows(AT_F + 8, W.pw1, D + 4 * g, 4, D);
            /* lanes 0-8: the 36 taps of channels 4g .. 4g+3; lanes 9-16: their 8 history rows */
            const float *dinl = din + (u64)l * din_stride;
            const u32 t = lane - 9;
            const float *src = lane < 9    ? W.dw_w + 4 * g * NK_CONV_TAPS + 4 * lane
                               : lane < 17 ? dinl + (u64)(pos - (NK_CONV_TAPS - 1) + t) * D + 4 * g
                                           : W.dw_w + 4 * g * NK_CONV_TAPS;
            put(AT_F + 16, src);
            vec(AT_F + 17, W.bn_g);
            vec(AT_F + 21, W.bn_b);
        } else if (j == PH_G) {
            rows(AT_G, W.pw2, 4 * g, 4, D);
            vec(AT_G + 8, W.ln_ff2_g);
            vec(AT_G + 12, W.ln_ff2_b);
        } else if (j == PH_H) {
            rows(AT_H, W.ff2_w1, 16 * g, 16, D);
        } else {
            rows(AT_I, W.ff2_w2, 4 * g, 4, FF);
            vec(AT_I + 32, W.ln_out_g);
            vec(AT_I + 36, W.ln_out_b);
            const_layer_t &Wn = Lt[l + 1 < nl ? l + 1 : l];
            vec(AT_I + 40, Wn.ln_ff1_g);
            vec(AT_I + 44, Wn.ln_ff1_b);
        }
    }
};

/* wavefront 6: segment p + 2 after the barrier of phase p, then a wait for segment p + 1 before
 * the barrier of phase p + 1.  The loads complete in order and at most STREAM_INFLIGHT are in
 * flight, all of them (when it is not empty) from segment p + 2, which holds more than that. */
__device__ __forceinline__ void stream_loop(const NkChainArgs &a, Shared &sh, u32 g, u32 lane) {
    const u32 nl = a.n_layers, P = NK_CHAIN_PH * nl;
    Stream st;
    st.Lt = (const_layer_t *)a.L;
    st.kv = a.kv;
    st.din = a.din;
    st.kv_stride = a.kv_stride;
    st.din_stride = a.din_stride;
    st.Lmax = a.Lmax;
    st.nl = nl;
    st.ring = (lds_char_t *)sh.ring;
    st.g = g;
    st.lane = lane;
    st.pos = (u32)a.desc[NK_DESC_POS];
    st.cl = (u32)a.desc[NK_DESC_CACHE];
    st.L = st.cl + 1;
    st.attn = g < NATT;
    st.head = g / NP;
    st.qt = quarter(st.L, g % NP);
    st.seg(0);
    st.seg(1);
    wait_vm_lgkm<STREAM_INFLIGHT>();
#pragma nounroll
    for (u32 p = 0; p < P; ++p) {
        lds_barrier();
        if (sh.bad) return;
        if (p % NK_CHAIN_PH == PH_D && st.attn) {
            lds_barrier();
            lds_barrier();
            lds_barrier();
            lds_barrier();
        }
        const u32 q = p + 2;
        if (q < P) st.seg(q);
        if (q < P && (q % NK_CHAIN_PH != PH_D || st.attn)) wait_vm_lgkm<STREAM_INFLIGHT>();
        else wait_vm_lgkm<0>();
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
    if (tid == 0) {
        sh.bad = 0;
        sh.done = 0;
    }
    __syncthreads();
    if (wave < 4) chain::compute_loop(a, sh, c, g, wave, lane);
    else if (wave < 6) chain::handoff_loop(a, sh, c, g, wave, lane);
    else chain::stream_loop(a, sh, g, lane);
    wait_vm_lgkm<0>(); /* no direct-to-LDS load outlives the workgroup */
}
