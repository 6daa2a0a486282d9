/* The reference's kernel parameter blocks (src/kernel_params.h:9-32), the by-value argument of
 * each kernel dispatched through include/nemo_gpu.h.  Layouts are the reference's (plain 32-bit
 * fields in this order): they are the ABI a host built against the reference passes with
 * GPU_BYTES.  The constants are the reference's sizing values its host code reads. */
#ifndef NEMO_KERNEL_PARAMS_REF_H
#define NEMO_KERNEL_PARAMS_REF_H
#include <stdint.h>

#define GEMM_ROWS 16
#define GEMM_SIMDS 8
#define ATT_DH 128
#define JOINT_GROUPS 64
#define MMA_MIN_ROWS 16
#define CACHE_EPOCH_CHUNKS 8
#define DEC_MAX_BATCH 16
#define ATT_MAX_L 80
#define LN_THREADS 256
#define JOINT_MAX_H 640

/* act: 0 none, 1 SiLU, 2 ReLU, 3 GLU (N = 2 x output width) */
typedef struct { uint32_t M, N, K, lda, ldw, ldc, has_bias, act, accumulate; float alpha; } GemmParams;
typedef struct { uint32_t M, D; float eps; } LnParams;
typedef struct { uint32_t c, L, Lmax, H, dh, D, ldq, ldk; float scale; } AttnParams;
typedef struct { uint32_t M, D; } GluParams;
typedef struct { uint32_t c, D, taps; float eps; } DwParams;
typedef struct { uint32_t T, F, T1, F1, C; } Conv2dParams;
typedef struct { uint32_t T, F, C; } FlatParams;
typedef struct { uint32_t n; } CountParams;
typedef struct { uint32_t n; float value; } FillParams;
typedef struct { uint32_t H; } LstmParams;
typedef struct { uint32_t V, H, enc_row, enc_ld; } JointParams;

#endif
