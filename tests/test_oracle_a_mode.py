"""The oracle's numerics study switch (or_set_gemm_a_mode, used by oracle/study_a_precision.py):
mode 0 is the reference's f32 GEMM, mode 2 (A as bf16 hi + lo) stays within the GEMM gate of it,
mode 1 (A as one bf16) equals a GEMM of the bf16-rounded A, and the switch resets."""
import numpy as np

import oracle


def test_gemm_a_modes():
    rng = np.random.default_rng(5)
    M, N, K = 5, 64, 512
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = oracle.f32_to_bf16((rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32))
    ref = oracle.gemm(A, W)
    L = oracle.lib()
    try:
        L.or_set_gemm_a_mode(2)
        hilo = oracle.gemm(A, W)
        L.or_set_gemm_a_mode(1)
        one = oracle.gemm(A, W)
    finally:
        L.or_set_gemm_a_mode(0)
    err = lambda x: float(np.max(np.abs(x - ref)) / np.max(np.abs(ref)))
    assert err(hilo) < 2e-5
    assert err(one) > 1e-4
    Ab = oracle.bf16_to_f32(oracle.f32_to_bf16(A))
    assert np.array_equal(one, oracle.gemm(Ab, W))
    assert np.array_equal(oracle.gemm(A, W), ref)
