/* Streaming-chunk kernels for gfx950 besides the GEMMs and the per-row kernels of nk_seq.hip:
 * the subsampling convs, copies, cache compaction, and the
 * RNNT decoder's LSTM cell and joint argmax.  Each states the reference kernel it replaces. */
#include "nk_common.h"

/* The two stride-2 3x3 convolutions of the subsampling, same causal padding (2 rows/columns
 * before, reference src/kernels.metal:411-454).  Workgroup = one output row t1 and 8 output
 * columns f1 (grid.x = T1 * ceil(F1/8), grid.y = windows of one size back to back, X and Y strides
 * xs / ys); thread = output channel, holding its 9 taps and bias in registers for the 8 columns.
 * Each output sums bias, then taps in (kh, kw) order. */
/* 1 input channel -> C channels + ReLU: X [T][F] -> Y [T1][F1][C] */
extern "C" __global__ __launch_bounds__(256) void conv2d_c1_s2_relu(NkConvArgs a) {
    const u32 nfb = (a.F1 + a.fb - 1) / a.fb;
    const u32 t1 = blockIdx.x / nfb, f0 = (blockIdx.x % nfb) * a.fb;
    const float *X = a.X + (u64)blockIdx.y * a.xs;
    float *Y = a.Y + (u64)blockIdx.y * a.ys;
    const u32 fe = min(f0 + a.fb, a.F1);
    for (u32 o = threadIdx.x; o < a.C; o += 256) {
        float w[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) w[k] = a.W[o * 9 + k];
        const float bo = a.bias[o];
        for (u32 f1 = f0; f1 < fe; ++f1) {
            float acc = bo;
#pragma unroll
            for (int kh = 0; kh < 3; ++kh) {
                const int ti = (int)(2 * t1 + kh) - 2;
                if (ti < 0 || ti >= (int)a.T) continue;
#pragma unroll
                for (int kw = 0; kw < 3; ++kw) {
                    const int fi = (int)(2 * f1 + kw) - 2;
                    if (fi < 0 || fi >= (int)a.F) continue;
                    acc += w[kh * 3 + kw] * X[(u64)ti * a.F + fi];
                }
            }
            Y[((u64)t1 * a.F1 + f1) * a.C + o] = fmaxf(acc, 0.0f);
        }
    }
}

/* depthwise, + bias, no activation: X [T][F][C] -> Y [T1][F1][C] */
extern "C" __global__ __launch_bounds__(256) void dwconv2d_s2(NkConvArgs a) {
    const u32 nfb = (a.F1 + a.fb - 1) / a.fb;
    const u32 t1 = blockIdx.x / nfb, f0 = (blockIdx.x % nfb) * a.fb;
    const float *X = a.X + (u64)blockIdx.y * a.xs;
    float *Y = a.Y + (u64)blockIdx.y * a.ys;
    const u32 fe = min(f0 + a.fb, a.F1);
    for (u32 c = threadIdx.x; c < a.C; c += 256) {
        float w[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) w[k] = a.W[c * 9 + k];
        const float bc = a.bias[c];
        for (u32 f1 = f0; f1 < fe; ++f1) {
            float acc = bc;
#pragma unroll
            for (int kh = 0; kh < 3; ++kh) {
                const int ti = (int)(2 * t1 + kh) - 2;
                if (ti < 0 || ti >= (int)a.T) continue;
#pragma unroll
                for (int kw = 0; kw < 3; ++kw) {
                    const int fi = (int)(2 * f1 + kw) - 2;
                    if (fi < 0 || fi >= (int)a.F) continue;
                    acc += w[kh * 3 + kw] * X[((u64)ti * a.F + fi) * a.C + c];
                }
            }
            Y[((u64)t1 * a.F1 + f1) * a.C + c] = acc;
        }
    }
}

/* conv 0 (1 -> C channels + ReLU) followed by conv 2 (depthwise, + bias) without storing conv 0's
 * output: X [T][F] -> Y [T2][F2][C].  Workgroup = one output row t2 and fb output columns of one
 * window; thread = channel.  The seven X rows the output row reads (4 t2 - 6 .. 4 t2) are staged
 * in LDS.  Every conv 0 value is computed exactly as conv2d_c1_s2_relu computes it (bias, then the
 * taps in (kh, kw) order, taps outside X skipped, ReLU) and every output exactly as dwconv2d_s2
 * computes it (bias, then the taps in order, positions outside conv 0's T1 x F1 skipped), so the
 * result equals the two kernels' bit for bit.  A thread walks its columns left to right; for each
 * it reads the 7 x 7 mel values its conv 0 taps can touch (columns 4 f2 - 6 .. 4 f2) from LDS
 * into registers once (a third fewer LDS reads than per tap: 8.6 -> 5.7 us for one 24-row window,
 * 564 -> 386 us for 256 windows of 121 rows), and the conv 0 column 2 f2 of output f2, which is
 * column 2 (f2 + 1) - 2 of the next, is kept. */
extern "C" __global__ __launch_bounds__(256) void conv2d_c1_dw_s2(NkConv02Args a) {
    __shared__ float xs[7][NK_CONV02_FMAX];
    const u32 nfb = (a.F2 + a.fb - 1) / a.fb;
    const u32 t2 = blockIdx.x / nfb, f0 = (blockIdx.x % nfb) * a.fb;
    const float *X = a.X + (u64)blockIdx.y * a.xs;
    float *Y = a.Y + (u64)blockIdx.y * a.ys;
    const u32 fe = min(f0 + a.fb, a.F2);
    const int ti0 = 4 * (int)t2 - 6; /* X row of LDS row 0 */
    for (u32 i = threadIdx.x; i < 7 * a.F; i += 256) {
        const int r = (int)(i / a.F), ti = ti0 + r;
        xs[r][i % a.F] = (ti >= 0 && ti < (int)a.T) ? X[(u64)ti * a.F + i % a.F] : 0.0f;
    }
    __syncthreads();
    for (u32 c = threadIdx.x; c < a.C; c += 256) {
        float w0[9], w2[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) { w0[k] = a.W0[c * 9 + k]; w2[k] = a.W2[c * 9 + k]; }
        const float bias0 = a.b0[c], bias2 = a.b2[c];
        float keep[3];
        bool keep_ok[3];
        for (u32 f2 = f0; f2 < fe; ++f2) {
            /* mel columns 4 f2 - 6 .. 4 f2 of the 7 rows (reads clamped into the row; taps outside
             * the mel window are skipped below, as in conv2d_c1_s2_relu) */
            float xv[7][7];
            const int cb = 4 * (int)f2 - 6;
#pragma unroll
            for (int r = 0; r < 7; ++r)
#pragma unroll
                for (int q = 0; q < 7; ++q) xv[r][q] = xs[r][min(max(cb + q, 0), (int)a.F - 1)];
            /* conv 0 at row 2 t2 + kh2 - 2, column 2 f2 - 2 + cs: mel row 2 kh2 + kh of xv, column 2 cs + kw */
            auto conv0 = [&](const int kh2, const int cs, bool &ok) -> float {
                const int t1 = 2 * (int)t2 + kh2 - 2, f1 = 2 * (int)f2 - 2 + cs;
                ok = t1 >= 0 && t1 < (int)a.T1 && f1 >= 0 && f1 < (int)a.F1;
                if (!ok) return 0.0f;
                float acc = bias0;
#pragma unroll
                for (int kh = 0; kh < 3; ++kh) {
                    const int ti = 2 * t1 + kh - 2;
                    if (ti < 0 || ti >= (int)a.T) continue;
#pragma unroll
                    for (int kw = 0; kw < 3; ++kw) {
                        const int fi = 2 * f1 + kw - 2;
                        if (fi < 0 || fi >= (int)a.F) continue;
                        acc += w0[kh * 3 + kw] * xv[2 * kh2 + kh][2 * cs + kw];
                    }
                }
                return fmaxf(acc, 0.0f);
            };
            float v[3][3];
            bool ok[3][3];
#pragma unroll
            for (int kh2 = 0; kh2 < 3; ++kh2) {
                if (f2 == f0) v[kh2][0] = conv0(kh2, 0, ok[kh2][0]);
                else { v[kh2][0] = keep[kh2]; ok[kh2][0] = keep_ok[kh2]; }
                v[kh2][1] = conv0(kh2, 1, ok[kh2][1]);
                v[kh2][2] = conv0(kh2, 2, ok[kh2][2]);
                keep[kh2] = v[kh2][2];
                keep_ok[kh2] = ok[kh2][2];
            }
            float acc = bias2;
#pragma unroll
            for (int kh2 = 0; kh2 < 3; ++kh2)
#pragma unroll
                for (int kw2 = 0; kw2 < 3; ++kw2)
                    if (ok[kh2][kw2]) acc += w2[kh2 * 3 + kw2] * v[kh2][kw2];
            Y[((u64)t2 * a.F2 + f2) * a.C + c] = acc;
        }
    }
}

/* Log-mel of one 512-sample frame per workgroup (reference src/mel.c:115-173, the host front end's
 * computation step for step): window, radix-2 decimation-in-time FFT in double (bit-reversed load,
 * nine stages of 256 butterflies, one per thread, with the host's twiddle table and operation
 * order), power in double rounded to float, each filter's sum over its bins in ascending order in
 * float, log(x + 2^-24).  Floating-point contraction is off, so the spectrum equals the host's. */
extern "C" __global__ __launch_bounds__(256) void mel_frames(const NkMelArgs a) {
#pragma clang fp contract(off)
    __shared__ double re[512], im[512];
    __shared__ float pw[257];
    const u32 f = blockIdx.x, t = threadIdx.x;
    const float *fr = a.span + a.tab[2 * f];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const u32 k = t + 256 * h, j = a.rev[k];
        re[j] = (double)(fr[k] * a.win[k]);
        im[j] = 0.0;
    }
    __syncthreads();
    for (u32 len = 2; len <= 512; len <<= 1) {
        const u32 hl = len >> 1, stride = 512 / len, k = t % hl, ia = (t / hl) * len + k, ib = ia + hl;
        const double wr = a.tw_re[k * stride], wi = a.tw_im[k * stride];
        const double br = re[ib], bi = im[ib], ar = re[ia], ai = im[ia];
        const double xr = br * wr - bi * wi, xi = br * wi + bi * wr;
        re[ib] = ar - xr;
        im[ib] = ai - xi;
        re[ia] = ar + xr;
        im[ia] = ai + xi;
        __syncthreads();
    }
    pw[t] = (float)(re[t] * re[t] + im[t] * im[t]);
    if (t == 0) pw[256] = (float)(re[256] * re[256] + im[256] * im[256]);
    __syncthreads();
    if (t < 128) {
        float acc = 0.0f;
        const float *w = a.fb + (u64)t * 257;
        for (int k = a.fb_lo[t]; k < a.fb_hi[t]; ++k) acc += w[k] * pw[k];
        a.out[(u64)(u32)a.tab[2 * f + 1] * 128 + t] = logf(acc + 5.9604644775390625e-08f);
    }
}

/* [T][F][C] -> [T][C*F] channel-major flatten: reference src/kernels.metal:456-462.
 * One thread per output element (reads gather, writes are coalesced). */
extern "C" __global__ __launch_bounds__(256) void flatten_cf(NkFlatArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    const u64 total = (u64)a.T * a.C * a.F;
    if (idx >= total) return;
    a.X += (u64)blockIdx.y * total; /* grid.y: windows of the same size, back to back */
    a.Y += (u64)blockIdx.y * total;
    const u32 f = (u32)(idx % a.F), c = (u32)((idx / a.F) % a.C), t = (u32)(idx / ((u64)a.F * a.C));
    a.Y[idx] = a.X[((u64)t * a.F + f) * a.C + c];
}

extern "C" __global__ __launch_bounds__(256) void copy_f32(const NkCopyArgs a) {
    const u32 i = blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.dst[i] = a.src[i];
}

/* Pending residual update of the many-row GEMM (NkFoldArgs): one thread per 4 consecutive values
 * of a row, the parts added in order from zero, then C + alpha * sum. */
extern "C" __global__ __launch_bounds__(256) void resid_fold(const NkFoldArgs a) {
    const u32 n4 = a.N >> 2, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.M * n4) return;
    const u32 r = i / n4, c = 4 * (i % n4);
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
    for (u32 b = 0; b < a.nparts; ++b) {
        const float4 q = *(const float4 *)(a.P + ((u64)b * a.M + r) * a.N + c);
        t.x += q.x; t.y += q.y; t.z += q.z; t.w += q.w;
    }
    float4 *dst = (float4 *)(a.C + (u64)r * a.ldc + c);
    float4 v = *dst;
    v.x = v.x + t.x * a.alpha; v.y = v.y + t.y * a.alpha; v.z = v.z + t.z * a.alpha; v.w = v.w + t.w * a.alpha;
    *dst = v;
}

extern "C" __global__ __launch_bounds__(256) void fill_f32(const NkFillArgs a) {
    const u32 i = blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.dst[i] = a.value;
}

/* Epoch compaction of the per-layer caches in one launch (reference src/encoder.c:199-211 issues
 * one copy per layer and cache).  grid = (ceil(rows*cols/256), nbuf).  Source and destination rows
 * never overlap (the host checks src_row >= dst_row + rows). */
extern "C" __global__ __launch_bounds__(256) void compact_rows(const NkCompactArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (u64)a.rows * a.cols) return;
    float *b = a.base + (u64)blockIdx.y * a.stride;
    b[(u64)a.dst_row * a.cols + idx] = b[(u64)a.src_row * a.cols + idx];
}
/* The same copy 16 bytes per thread, when cols, the buffer stride and the base are multiples of 4
 * floats (every cache of the model: rows of 1024 or 3072 floats).  grid = (ceil(rows*cols/1024), nbuf). */
extern "C" __global__ __launch_bounds__(256) void compact_rows4(const NkCompactArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x, n4 = (u64)a.rows * a.cols / 4;
    if (idx >= n4) return;
    float4 *b = (float4 *)(a.base + (u64)blockIdx.y * a.stride);
    b[(u64)a.dst_row * (a.cols / 4) + idx] = b[(u64)a.src_row * (a.cols / 4) + idx];
}

/* Strided row copy: rows x cols floats from src (row stride src_ld) to dst (row stride dst_ld).
 * Used for the row select of the subsampled window and for activation dumps. */
extern "C" __global__ __launch_bounds__(256) void copy2d_f32(const NkCopy2dArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (u64)a.rows * a.cols) return;
    const u32 r = (u32)(idx / a.cols), c = (u32)(idx % a.cols);
    a.dst[(u64)r * a.dst_ld + c] = a.src[(u64)r * a.src_ld + c];
}

/* ---- batched streams ------------------------------------------------------------------------ */

/* dst[m] = src[map[m]] row gather (the batched row select of the subsampled windows) */
extern "C" __global__ __launch_bounds__(256) void gather_rows(const NkGatherArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (u64)a.rows * a.cols) return;
    const u32 m = (u32)(idx / a.cols), k = (u32)(idx % a.cols);
    a.dst[(u64)m * a.dst_ld + k] = a.src[(u64)(u32)a.map[m] * a.src_ld + k];
}

/* dst row map[m] = src row m (rows of `cols` floats; the map's targets are distinct) */
extern "C" __global__ __launch_bounds__(256) void scatter_rows(const NkGatherArgs a) {
    const u64 idx = (u64)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (u64)a.rows * a.cols) return;
    const u32 m = (u32)(idx / a.cols), k = (u32)(idx % a.cols);
    a.dst[(u64)(u32)a.map[m] * a.dst_ld + k] = a.src[(u64)m * a.src_ld + k];
}

/* LSTM input rows [x | h] of the batched decoder (one thread per element; grid.y = row) */
extern "C" __global__ __launch_bounds__(256) void lstm_input_rows(const NkLstmInArgs a) {
    const u32 n = blockIdx.y, k = blockIdx.x * 256 + threadIdx.x;
    if (n >= a.n || k >= 2 * a.P) return;
    float v;
    if (k < a.P) {
        if (a.tok) {
            const int t = a.tok[n];
            v = (t < 0 || (u32)t == a.blank) ? 0.0f : bf2f(a.embed[(u64)t * a.P + k]);
        } else {
            v = a.xsrc[(u64)n * a.P + k];
        }
    } else {
        v = a.hc[(u64)(u32)a.hrow[n] * a.P + (k - a.P)];
    }
    a.A[(u64)n * 2 * a.P + k] = v;
}

/* LSTM cell on batched rows, reference src/kernels.metal:474-486 (c' = f*c + i*g, h' = o*tanh(c')) */
extern "C" __global__ __launch_bounds__(256) void lstm_cell_rows(const NkLstmRowsArgs a) {
    const u32 n = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x;
    if (n >= a.n || j >= a.P) return;
    const float *gt = a.gates + (u64)n * 4 * a.P;
    const float ig = sigmoid_f(gt[j]), fg = sigmoid_f(gt[a.P + j]), gg = tanhf(gt[2 * a.P + j]), og = sigmoid_f(gt[3 * a.P + j]);
    const float c = fg * a.hc[(u64)(u32)a.crow_in[n] * a.P + j] + ig * gg;
    const float h = og * tanhf(c);
    a.hc[(u64)(u32)a.crow_out[n] * a.P + j] = c;
    a.hc[(u64)(u32)a.hrow_out[n] * a.P + j] = h;
    a.hout[(u64)n * a.P + j] = h;
}

/* joint input rows relu(enc + pred), reference src/kernels.metal:488-519 (the r vector) */
extern "C" __global__ __launch_bounds__(256) void joint_in_rows(const NkJointInArgs a) {
    const u32 r = blockIdx.y, k = blockIdx.x * 256 + threadIdx.x;
    if (r >= a.rows || k >= a.J) return;
    a.jin[(u64)r * a.J + k] = fmaxf(a.enc[(u64)(u32)a.erow[r] * a.J + k] + a.pred[(u64)(u32)a.prow[r] * a.J + k], 0.0f);
}

/* argmax of each row of joint logits, lowest index on ties (src/kernels.metal:521-550) */
extern "C" __global__ __launch_bounds__(256) void argmax_rows(const NkArgmaxRowsArgs a) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    const u32 r = blockIdx.x, tid = threadIdx.x;
    const float *x = a.logits + (u64)r * a.ld;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (u32 n = tid; n < a.V; n += 256) {
        const float v = x[n];
        if (v > best || (v == best && (int)n < bidx)) { best = v; bidx = (int)n; }
    }
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
        a.out[2 * r] = bi[0];
        a.out[2 * r + 1] = __float_as_int(bv[0]);
    }
}
