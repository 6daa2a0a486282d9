/* Device helpers shared by the gfx950 kernels. */
#ifndef NK_COMMON_H
#define NK_COMMON_H
#include <hip/hip_runtime.h>
#include "../kernel_params.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned long long u64;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));

/* 16-byte weight load marked non-temporal: weights are read once per chunk, so they should not
 * displace activations and caches from L2 / MALL. */
__device__ __forceinline__ uint4 ld_nt16(const u16 *p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
/* 16 bytes with the default cache policy: weights read again by every step of a loop */
__device__ __forceinline__ uint4 ld_c16(const u16 *p) {
    const u32x4 v = *(const u32x4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

/* float4 i of an n-float4 array, or zeros for i >= n (n >= 1).  The load itself is unconditional
 * (index clamped into the array) and only the result is selected: written as `i < n ? p[i] : 0`,
 * the compiler splits the 16-byte load into four exec-masked 4-byte loads, each behind a branch. */
__device__ __forceinline__ float4 ld4z(const float4 *p, u32 i, u32 n) {
    const float4 v = p[min(i, n - 1)];
    return i < n ? v : make_float4(0.f, 0.f, 0.f, 0.f);
}

/* bf16 bits -> f32: the upper half of the f32 pattern (exact). */
__device__ __forceinline__ float bf2f(u32 bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float bf_lo(u32 pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf_hi(u32 pair) { return __uint_as_float(pair & 0xffff0000u); }

/* f32 -> bf16 bits, round to nearest even (finite inputs). */
__device__ __forceinline__ u32 f2bf(float f) {
    u32 u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

/* The reference's activation forms (src/kernels.metal:6-7): a division, IEEE expf. */
__device__ __forceinline__ float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }
__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

/* Butterfly sum over the 64 lanes of a wavefront; every lane ends with the same total. */
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
#define DPP_QUAD_1032 0xB1 /* quad_perm(1,0,3,2) */
#define DPP_QUAD_2301 0x4E /* quad_perm(2,3,0,1) */
#define DPP_QUAD_0000 0x00 /* quad_perm(0,0,0,0): lane 0 of the quad to all four */
#define DPP_QUAD_1111 0x55
#define DPP_QUAD_2222 0xAA
#define DPP_QUAD_3333 0xFF
#define DPP_ROW_ROR4 0x124
#define DPP_ROW_ROR8 0x128

/* Sum over the 64 lanes of a wavefront, returned wave-uniform; fixed combination order
 * (DPP within each 16-lane row, then the four row totals read from lanes 0, 16, 32, 48). */
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

/* Maximum over the 64 lanes of a wavefront, returned wave-uniform (DPP rows, then four lanes). */
__device__ __forceinline__ float wmax(float v) {
    v = fmaxf(v, dpp_f<DPP_QUAD_1032>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_2301>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_ROR4>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_ROR8>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

/* Workgroup barrier for data exchanged through LDS only: waits for this wavefront's LDS
 * operations but not for its outstanding global loads (a __syncthreads() would also wait for
 * every weight load in flight).  The "memory" clobber keeps the compiler from moving memory
 * accesses across it. */
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

/* Dot of 8 f32 activations with 8 bf16 weights packed in a uint4, summed in index order. */
__device__ __forceinline__ float dot8(const float *a, uint4 w, float acc) {
    acc += a[0] * bf_lo(w.x);
    acc += a[1] * bf_hi(w.x);
    acc += a[2] * bf_lo(w.y);
    acc += a[3] * bf_hi(w.y);
    acc += a[4] * bf_lo(w.z);
    acc += a[5] * bf_hi(w.z);
    acc += a[6] * bf_lo(w.w);
    acc += a[7] * bf_hi(w.w);
    return acc;
}

/* GEMM epilogue of one output element (reference src/kernels.metal:106-116). */
__device__ __forceinline__ void epi_store(const NkGemmArgs &a, u32 m, u32 n, float s) {
    float v = s + (a.bias ? a.bias[n] : 0.0f);
    if (a.act == NK_ACT_SILU) v = silu_f(v);
    else if (a.act == NK_ACT_RELU) v = fmaxf(v, 0.0f);
    v *= a.alpha;
    const u32 row = a.crow ? (u32)a.crow[m] : m;
    float *c = a.C + (u64)row * a.ldc + n;
    *c = a.accumulate ? (*c + v) : v;
}

/* GLU epilogue: output column j pairs weight rows j and j + N/2 (src/kernels.metal:96-104). */
__device__ __forceinline__ void epi_store_glu(const NkGemmArgs &a, u32 m, u32 j, float sa, float sb) {
    const float va = sa + (a.bias ? a.bias[j] : 0.0f);
    const float vb = sb + (a.bias ? a.bias[j + a.N / 2] : 0.0f);
    const float v = va * sigmoid_f(vb) * a.alpha;
    const u32 row = a.crow ? (u32)a.crow[m] : m;
    float *c = a.C + (u64)row * a.ldc + j;
    *c = a.accumulate ? (*c + v) : v;
}

/* Split one f32 into bf16 hi + bf16 lo so that hi + lo carries 16 significant bits. */
__device__ __forceinline__ void split_bf16(float v, u32 &hi, u32 &lo) {
    hi = f2bf(v);
    lo = f2bf(v - __uint_as_float(hi << 16));
}

/* 8 f32 -> bf16 hi (round to nearest even, v_cvt_pk_bf16_f32) and bf16 lo = bf16(x - hi), packed
 * in pairs (element 2p in the low half of word p). */
__device__ __forceinline__ void split8(const float (&x)[8], uint4 &hi, uint4 &lo) {
    u32 h[4], l[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const floatx2 v = { x[2 * p], x[2 * p + 1] };
        const u32 hb = __builtin_bit_cast(u32, __builtin_convertvector(v, bf16x2));
        const floatx2 hv = { __uint_as_float(hb << 16), __uint_as_float(hb & 0xffff0000u) };
        h[p] = hb;
        l[p] = __builtin_bit_cast(u32, __builtin_convertvector(v - hv, bf16x2));
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

/* two f32 -> their bf16 hi (RNE) and lo = RNE(x - hi), each pair packed element 0 in the low half:
 * the same rounding as split8 */
__device__ __forceinline__ void split2(float x0, float x1, u32 &hi, u32 &lo) {
    const floatx2 v = { x0, x1 };
    hi = __builtin_bit_cast(u32, __builtin_convertvector(v, bf16x2));
    const floatx2 hv = { __uint_as_float(hi << 16), __uint_as_float(hi & 0xffff0000u) };
    lo = __builtin_bit_cast(u32, __builtin_convertvector(v - hv, bf16x2));
}

/* Split-row stores: element i of a row of D values goes to row[i] (hi) and row[D + i] (lo). */
__device__ __forceinline__ void store_split4(u16 *row, u32 D, u32 i, float4 v) {
    uint2 h, l;
    split2(v.x, v.y, h.x, l.x);
    split2(v.z, v.w, h.y, l.y);
    *(uint2 *)(row + i) = h;
    *(uint2 *)(row + D + i) = l;
}
__device__ __forceinline__ void store_split1(u16 *row, u32 D, u32 i, float v) {
    u32 h, l;
    split2(v, 0.0f, h, l);
    row[i] = (u16)h;
    row[D + i] = (u16)l;
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
    union { uint4 u; bf16x8 b; } c;
    c.u = v;
    return c.b;
}

__device__ __forceinline__ floatx4 mfma_bf16(uint4 a, uint4 b, floatx4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), acc, 0, 0, 0);
}

/* (score, index) -> 64-bit key whose unsigned order is: higher score first, then lower index */
__device__ __forceinline__ unsigned long long dec_key(float v, u32 n) {
    v += 0.0f; /* -0 -> +0 so that equal scores compare equal */
    const u32 b = __float_as_uint(v);
    const u32 ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (0xffffffffu - n);
}
__device__ __forceinline__ u32 dec_key_index(unsigned long long k) { return 0xffffffffu - (u32)(k & 0xffffffffu); }

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int m) {
    const u32 lo = (u32)__shfl_xor((int)(u32)v, m, 64), hi = (u32)__shfl_xor((int)(u32)(v >> 32), m, 64);
    return ((unsigned long long)hi << 32) | lo;
}

typedef __attribute__((address_space(3))) char lds_char_t;

/* 16 bytes per lane from global memory straight into LDS: lane i writes LDS bytes
 * [lds + 16 i, +16) of the wavefront-uniform base `lds`.  Issued as inline assembly, so the
 * compiler does not track these loads: a kernel waits for them itself (wait_vm_lgkm) before the
 * barrier that publishes the data, and drains them all before it can end. */
__device__ __forceinline__ void dma16(const void *g, lds_char_t *lds) {
    const u32 base = __builtin_amdgcn_readfirstlane((u32)(size_t)lds);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(base) : "memory");
}

/* s_waitcnt vmcnt(N) lgkmcnt(0) */
template <int N> __device__ __forceinline__ void wait_vm_lgkm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void barrier_mem() { asm volatile("s_barrier" ::: "memory"); }

#endif
