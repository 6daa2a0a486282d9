"""The allocation-free entry point nk_gemm_split_noalloc (split-K scratch in a static device array)
against nk_gemm_split, through the C ABI: bit-identical outputs on two calls in a row, the second
with a smaller input, and a clear refusal (nothing launched) for a shape whose K split needs more
scratch than the array holds."""
import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu

NK_NOALLOC_WS_FLOATS = 4 << 20


def run(gpu, fn, A, W, C0, K_split, alpha=0.5):
    import nemoasr

    L = nemoasr.lib()
    M, K = A.shape
    N = W.shape[0]
    dA, dW, dC = gpu.put(A), gpu.put(W), gpu.put(C0)
    prev = L.nk_gemm_ksplit(K_split)
    try:
        gpu.begin()
        rc = getattr(L, fn)(gpu.h, dA.ptr, None, K, dW.ptr, K, None, dC.ptr, None, N, None, M, N, K, 0, 1, alpha)
        err = L.gpu_last_error(gpu.h).decode() if rc else None
        gpu.end()
    finally:
        L.nk_gemm_ksplit(prev)
    out = dC.read((M, N))
    for b in (dA, dW, dC):
        b.free()
    return rc, out, err


@pytest.mark.parametrize("ksplit", [1, 0, -1])
def test_noalloc_matches_gemm_split(gpu, ksplit):
    rng = np.random.default_rng([ksplit + 1, 77])
    W = oracle.f32_to_bf16((rng.standard_normal((1024, 4096)) / 64).astype(np.float32))
    for M in (448, 130):  # the second call smaller than the first
        A = rng.standard_normal((M, 4096)).astype(np.float32)
        C0 = rng.standard_normal((M, 1024)).astype(np.float32)
        rc1, ref, _ = run(gpu, "nk_gemm_split", A, W, C0.copy(), ksplit)
        rc2, got, err = run(gpu, "nk_gemm_split_noalloc", A, W, C0.copy(), ksplit)
        assert rc1 == 0 and rc2 == 0, err
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), M
        assert rel_err(got, oracle.gemm(A, W, None, 0, True, 0.5, C0=C0)) < 2e-5


def test_noalloc_unsplit_when_split_does_not_fit(gpu):
    """1536 x 1024 outputs with K = 4096 are split four ways by default below ~400 tiles (6M floats
    of partial rows, more than the array); the unsplit partial rows (1.5M floats) fit, so the call
    succeeds with the bits of nk_gemm_split."""
    rng = np.random.default_rng(1536)
    M, N, K = 1536, 1024, 4096
    W = oracle.f32_to_bf16((rng.standard_normal((N, K)) / 64).astype(np.float32))
    A = rng.standard_normal((M, K)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    rc1, ref, _ = run(gpu, "nk_gemm_split", A, W, C0.copy(), -1)
    rc2, got, err = run(gpu, "nk_gemm_split_noalloc", A, W, C0.copy(), -1)
    assert rc1 == 0 and rc2 == 0, err
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_noalloc_in_graph_capture(gpu):
    """The entry point recorded into a hipGraph (where the library could not grow its own scratch)
    and replayed three times, with eager launches of the allocating form and host synchronisation
    between the replays: every replay gives the allocating form's bits."""
    import nemoasr

    L = nemoasr.lib()
    rng = np.random.default_rng(4481)
    M, N, K = 448, 1024, 4096
    W = oracle.f32_to_bf16((rng.standard_normal((N, K)) / 64).astype(np.float32))
    A = rng.standard_normal((M, K)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    rc, ref, err = run(gpu, "nk_gemm_split", A, W, C0.copy(), 1)
    assert rc == 0, err
    dA, dW, dC = gpu.put(A), gpu.put(W), gpu.put(C0)
    prev = L.nk_gemm_ksplit(1)
    graph = None
    try:
        gpu.begin()
        gpu.check(L.gpu_capture_begin(gpu.h))
        rc = L.nk_gemm_split_noalloc(gpu.h, dA.ptr, None, K, dW.ptr, K, None, dC.ptr, None, N, None, M, N, K, 0, 1, 0.5)
        graph = L.gpu_capture_end(gpu.h)
        gpu.end()
        assert rc == 0 and graph, L.gpu_last_error(gpu.h).decode()
        for rep in range(3):
            dC.write(C0)
            gpu.begin()
            gpu.check(L.gpu_graph_launch(gpu.h, graph))
            gpu.end()
            got = dC.read((M, N))
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), rep
            rc_e, ref_e, _ = run(gpu, "nk_gemm_split", A, W, C0.copy(), 1)  # eager work between replays
            assert rc_e == 0 and np.array_equal(ref_e.view(np.uint32), ref.view(np.uint32))
    finally:
        L.nk_gemm_ksplit(prev)
        if graph:
            L.gpu_graph_free(graph)
        for b in (dA, dW, dC):
            b.free()


def test_noalloc_refuses_oversized_split(gpu):
    """448 x 16384 outputs split four ways over K need 29M floats of partial rows, more than the
    array: the call fails with a message before launching anything."""
    import nemoasr

    L = nemoasr.lib()
    M, N, K = 448, 16384, 4096
    need = 4 * M * N
    assert need > NK_NOALLOC_WS_FLOATS
    dA, dW, dC = gpu.alloc(M * K * 4), gpu.alloc(N * K * 2), gpu.alloc(M * N * 4)
    prev = L.nk_gemm_ksplit(1)
    launches = L.gpu_launch_count(gpu.h)
    try:
        gpu.begin()
        rc = L.nk_gemm_split_noalloc(gpu.h, dA.ptr, None, K, dW.ptr, K, None, dC.ptr, None, N, None, M, N, K, 0, 1, 1.0)
        msg = L.gpu_last_error(gpu.h).decode()
        with pytest.raises(RuntimeError):
            gpu.end()
    finally:
        L.nk_gemm_ksplit(prev)
    assert rc != 0 and "scratch" in msg, msg
    assert L.gpu_launch_count(gpu.h) == launches
    for b in (dA, dW, dC):
        b.free()
