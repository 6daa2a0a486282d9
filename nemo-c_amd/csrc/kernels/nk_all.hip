/* Single translation unit for the gfx950 code object loaded by the host (hipModuleLoadData). */
#include "nk_gemm.hip"
#include "nk_mm.hip"
#include "nk_mx.hip"
#include "nk_gemv.hip"
#include "nk_seq.hip"
#include "nk_ops.hip"
#include "nk_dec.hip"
#include "nk_bdec.hip"
