/* Kernels served only through the reference-shaped dispatch (include/nemo_gpu.h): the reference
 * has them as separate dispatches, this library's own path fuses them (GLU into the GEMM
 * epilogue, the LSTM cell and the joint argmax into the device-resident greedy loop). */
#include "nk_common.h"

/* Y[m][d] = X[m][d] * sigmoid(X[m][D + d]), src/kernels.metal:349-356 */
extern "C" __global__ __launch_bounds__(256) void glu_rows(const NkGluArgs a) {
    const u32 m = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x;
    if (m >= a.M || d >= a.D) return;
    const float *x = a.X + (u64)m * 2 * a.D;
    a.Y[(u64)m * a.D + d] = x[d] * sigmoid_f(x[a.D + d]);
}

/* one LSTM cell over H units, gates in i, f, g, o order: src/kernels.metal:474-486 */
extern "C" __global__ __launch_bounds__(256) void lstm_cell_vec(const NkLstmCellArgs a) {
    const u32 i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.H) return;
    const float ig = sigmoid_f(a.gates[i]), fg = sigmoid_f(a.gates[a.H + i]);
    const float gg = tanhf(a.gates[2 * a.H + i]), og = sigmoid_f(a.gates[3 * a.H + i]);
    const float c = fg * a.c_in[i] + ig * gg;
    a.c_out[i] = c;
    a.h_out[i] = og * tanhf(c);
}

/* Joint stage 1 (src/kernels.metal:488-519): workgroup (g, r) has eight wavefronts; wavefront w owns
 * slot s = 8 g + w of row r and scores n = s, s + 8 G, ... of W . relu(enc[enc_row + r] + pred) + b,
 * keeping the best (lowest index on ties) in part_v / part_i[r][s].  H % 4 == 0, H <= 1024. */
extern "C" __global__ __launch_bounds__(512) void joint_partial_groups(const NkJointPartArgs a) {
    __shared__ float4 r4[NK_JOINT_MAX_H / 4];
    const u32 g = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float *e = a.enc + (u64)(a.enc_row + row) * a.enc_ld;
    float *r = (float *)r4;
    for (u32 i = tid; i < a.H; i += 512) r[i] = fmaxf(e[i] + a.pred[i], 0.0f);
    __syncthreads();
    const u32 H4 = a.H / 4, slots = a.groups * 8, s = g * 8 + w;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (u32 n = s; n < a.V; n += slots) {
        const ushort4 *w4 = (const ushort4 *)(a.W + (u64)n * a.H);
        float acc = 0.0f;
        for (u32 k4 = lane; k4 < H4; k4 += 64) {
            const ushort4 q = w4[k4];
            const float4 x = r4[k4];
            acc += x.x * bf2f(q.x) + x.y * bf2f(q.y) + x.z * bf2f(q.z) + x.w * bf2f(q.w);
        }
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) acc += __shfl_xor(acc, m, 64);
        acc += a.bias[n];
        if (acc > bv || (acc == bv && (int)n < bi)) { bv = acc; bi = (int)n; }
    }
    if (lane == 0) {
        a.part_v[(u64)row * slots + s] = bv;
        a.part_i[(u64)row * slots + s] = bi;
    }
}

/* Joint stage 2 (src/kernels.metal:521-550): best of a row's n partials, lowest index on ties;
 * out[2 r] = index, out[2 r + 1] = the value's bits.  One workgroup of 256 per row. */
extern "C" __global__ __launch_bounds__(256) void argmax_partials(const NkArgmaxPartArgs a) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    const u32 row = blockIdx.x, tid = threadIdx.x;
    const float *pv = a.part_v + (u64)row * a.n;
    const int *pi = a.part_i + (u64)row * a.n;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (u32 i = tid; i < a.n; i += 256)
        if (pv[i] > best || (pv[i] == best && pi[i] < bidx)) { best = pv[i]; bidx = pi[i]; }
    bv[tid] = best;
    bi[tid] = bidx;
    __syncthreads();
    for (u32 st = 128; st > 0; st >>= 1) {
        if (tid < st) {
            const float ov = bv[tid + st];
            const int oi = bi[tid + st];
            if (ov > bv[tid] || (ov == bv[tid] && oi < bi[tid])) { bv[tid] = ov; bi[tid] = oi; }
        }
        __syncthreads();
    }
    if (tid == 0) {
        a.out[2 * row] = bi[0];
        a.out[2 * row + 1] = __float_as_int(bv[0]);
    }
}
