"""Per-kernel parity of the gfx950 kernels against the oracle, at the model's real shapes.

Each test uploads seeded inputs, launches through the kernel-level C ABI
(include/nemo_kernels.h) and compares with the oracle's CPU restatement on the same inputs.
Tolerances: relative to the largest reference magnitude (tools/compare.py:30-32 style); the GPU
sums in a different order than the oracle (and the MFMA kernels split activations into bf16
hi + lo), so results agree to f32 rounding, not bit for bit.  Index outputs (argmax) are exact.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu

GEMM_TOL = 2e-5


def _w(rng, n, k, scale=None):
    s = scale if scale is not None else 1.0 / np.sqrt(k)
    return oracle.f32_to_bf16(rng.standard_normal((n, k)).astype(np.float32) * s)


def run_gemm(gpu, A, W, bias, act, acc, alpha, C0=None, ldw=None, K=None, kind=0, rows=None, ldc=None):
    import nemoasr

    L = nemoasr.lib()
    M = A.shape[0]
    N = W.shape[0]
    K = A.shape[1] if K is None else K
    ldw = W.shape[1] if ldw is None else ldw
    nout = N // 2 if act == 3 else N
    ldc = nout if ldc is None else ldc
    crows = M if rows is None else int(max(rows)) + 1
    C0 = np.zeros((crows, ldc), np.float32) if C0 is None else C0
    crows = C0.shape[0]
    dA, dW, dC = gpu.put(A), gpu.put(W), gpu.put(C0)
    dB = gpu.put(bias) if bias is not None else None
    dR = gpu.put(np.asarray(rows, np.int32)) if rows is not None else None
    prev = L.nk_gemm_force(kind)
    try:
        gpu.begin()
        gpu.check(L.nk_gemm_rows(gpu.h, dA.ptr, A.shape[1], dW.ptr, ldw, dB.ptr if dB else None, dC.ptr, ldc,
                                 dR.ptr if dR else None, M, N, K, act, int(acc), alpha))
        gpu.end()
    finally:
        L.nk_gemm_force(prev)
    out = dC.read((crows, ldc))
    for b in (dA, dW, dC, dB, dR):
        if b is not None:
            b.free()
    return out


# (N, K, act, accumulate, alpha, bias, ldw) at the model's shapes (src/encoder.c:120-194, decoder.c:69-76)
SHAPES = [
    (4096, 1024, 1, 0, 1.0, False, None),   # FF up + SiLU
    (1024, 4096, 0, 1, 0.5, False, None),   # FF down, half-step residual
    (3072, 1024, 0, 0, 1.0, False, None),   # fused QKV
    (2048, 1024, 3, 0, 1.0, False, None),   # pointwise conv 1 + GLU
    (1024, 1024, 0, 1, 1.0, False, None),   # out proj / pointwise conv 2
    (2048, 1024, 2, 0, 1.0, True, 1152),    # prompt W0 (ldw 1152) + ReLU
    (1024, 2048, 0, 0, 1.0, True, None),    # prompt W2
    (640, 1024, 0, 0, 1.0, True, None),     # joint.enc
    (1024, 4352, 0, 0, 1.0, True, None),    # pre-encode out
]


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 7, 10, 14, 16])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}a{s[2]}")
def test_gemm_few_rows(gpu, M, shape):
    N, K, act, acc, alpha, has_bias, ldw = shape
    rng = np.random.default_rng([M, N, K, act])
    ldw_ = ldw or K
    W = _w(rng, N, ldw_)
    A = rng.standard_normal((M, K)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32) if has_bias else None
    nout = N // 2 if act == 3 else N
    C0 = rng.standard_normal((M, nout)).astype(np.float32) if acc else None
    got = run_gemm(gpu, A, W, bias, act, acc, alpha, C0=C0, ldw=ldw_, K=K)
    ref = oracle.gemm(A, W, bias, act, acc, alpha, C0=C0, ldw=ldw_, K=K)
    assert rel_err(got, ref) < GEMM_TOL, (M, shape)


@pytest.mark.parametrize("M,N,K,act", [(231, 256, 256, 2), (627, 256, 256, 2), (1089, 256, 256, 2),
                                       (68, 256, 256, 2), (170, 256, 256, 2), (289, 256, 256, 2),
                                       (17, 1024, 4352, 0), (143, 1024, 1024, 0), (448, 4096, 1024, 1)])
def test_gemm_many_rows(gpu, M, N, K, act):
    rng = np.random.default_rng([M, N, K])
    W = _w(rng, N, K)
    A = np.abs(rng.standard_normal((M, K))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    got = run_gemm(gpu, A, W, bias, act, False, 1.0)
    ref = oracle.gemm(A, W, bias, act, False, 1.0)
    assert rel_err(got, ref) < GEMM_TOL


# batched multi-stream shapes (64 streams x 7 rows, 256 x 14) through the many-row MFMA kernels:
# each tile shape (128x128, 64x128, 64x64, plain and GLU), the residual updates' K split over
# workgroups (by tile count, never, always), row counts that are not tile multiples, K of one or
# two steps, row maps
@pytest.mark.parametrize("M,N,K,act,acc,bias", [
    (448, 4096, 1024, 1, 0, False), (448, 1024, 4096, 0, 1, False), (448, 3072, 1024, 0, 0, False),
    (448, 2048, 1024, 3, 0, False), (448, 1024, 1024, 0, 1, False), (448, 640, 1024, 0, 0, True),
    (3584, 4096, 1024, 1, 0, False), (3584, 2048, 1024, 3, 0, False), (3584, 1024, 4096, 0, 1, False),
    (100, 2048, 1024, 2, 0, True), (37, 1024, 2048, 0, 0, True),
    (445, 4096, 1024, 1, 0, False), (1000, 2048, 1024, 3, 0, False), (3584, 1024, 1024, 0, 1, False),
    (20, 3072, 1024, 0, 0, False), (448, 2560, 1280, 0, 0, True), (1024, 1088, 640, 0, 0, True),
    (64, 256, 32, 2, 0, True), (96, 128, 64, 0, 1, False), (64, 1024, 1024, 0, 1, False),
    (64, 2560, 1280, 0, 1, False), (224, 1024, 1024, 0, 1, False), (896, 1024, 4096, 0, 1, False)])
@pytest.mark.parametrize("split", [-1, 0, 1])
def test_gemm_batched_rows(gpu, M, N, K, act, acc, bias, split):
    import nemoasr

    prev = nemoasr.lib().nk_gemm_ksplit(split)
    rng = np.random.default_rng([M, N, K, act])
    W = _w(rng, N, K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    b = (0.1 * rng.standard_normal(N)).astype(np.float32) if bias else None
    nout = N // 2 if act == 3 else N
    C0 = rng.standard_normal((M, nout)).astype(np.float32) if acc else None
    try:
        got = run_gemm(gpu, A, W, b, act, acc, 0.5 if acc else 1.0, C0=C0)
    finally:
        nemoasr.lib().nk_gemm_ksplit(prev)
    ref = oracle.gemm(A, W, b, act, acc, 0.5 if acc else 1.0, C0=C0)
    assert rel_err(got, ref) < GEMM_TOL, (M, N, K, act)


@pytest.mark.parametrize("N,K", [(1024, 1024), (1024, 4096), (1024, 2048)])
def test_gemm_residual_bits(gpu, N, K):
    """The many-row residual update (C += alpha A W^T) gives the same bits whether its K is split
    over workgroups or not, from one launch to the next, and whatever the number of rows in the
    launch (a row computed alone equals the same row in a launch of 3584): the property that makes
    a stream's results independent of the other streams of a batch step."""
    import nemoasr

    L = nemoasr.lib()
    rng = np.random.default_rng([N, K])
    W = _w(rng, N, K)
    A = rng.standard_normal((3584, K)).astype(np.float32)
    C0 = rng.standard_normal((3584, N)).astype(np.float32)
    outs = {}
    try:
        for M in (3584, 448, 64, 17):
            for split in (0, 1, -1, -1):
                L.nk_gemm_ksplit(split)
                outs.setdefault(M, []).append(run_gemm(gpu, A[:M], W, None, 0, True, 0.5, C0=C0[:M].copy()))
    finally:
        L.nk_gemm_ksplit(-1)
    for M, runs in outs.items():
        for r in runs[1:]:
            assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32)), M
        assert np.array_equal(runs[0].view(np.uint32), outs[3584][0][:M].view(np.uint32)), M
    ref = oracle.gemm(A[:448], W, None, 0, True, 0.5, C0=C0[:448])
    assert rel_err(outs[448][0], ref) < GEMM_TOL


@pytest.mark.parametrize("M,N,K", [(7, 1024, 4096), (14, 1024, 1024), (10, 1024, 4096)])
def test_gemm_few_rows_split_repeatable(gpu, M, N, K):
    """The few-row residual update splits K over four workgroups; their partials are combined in a
    fixed order, so repeated launches give the same bits (and the oracle's values)."""
    rng = np.random.default_rng([M, N, K, 5])
    W = _w(rng, N, K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    runs = [run_gemm(gpu, A, W, None, 0, True, 0.5, C0=C0.copy()) for _ in range(4)]
    for r in runs[1:]:
        assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32))
    assert rel_err(runs[0], oracle.gemm(A, W, None, 0, True, 0.5, C0=C0)) < GEMM_TOL


@pytest.mark.parametrize("M,V", [(576, 1025), (64, 1025), (100, 97), (4096, 1025)])
def test_gemm_argmax_keys(gpu, M, V):
    """Row argmax of the joint scores from the GEMM's key epilogue: the best key over a row's column
    parts names the oracle's argmax (lowest index on ties), padding columns never win."""
    import nemoasr

    L = nemoasr.lib()
    rng = np.random.default_rng([M, V])
    J, N = 640, ((V + 63) // 64) * 64
    W = np.zeros((N, J), np.uint16)
    W[:V] = _w(rng, V, J)
    bias = np.zeros(N, np.float32)
    bias[:V] = rng.standard_normal(V).astype(np.float32)
    A = np.maximum(rng.standard_normal((M, J)), 0).astype(np.float32)
    A[1] = A[0]  # identical rows
    nk = N // 32
    dA, dW, dB, dK = gpu.put(A), gpu.put(W), gpu.put(bias), gpu.alloc(M * nk * 8)
    gpu.begin()
    gpu.check(L.nk_gemm_argmax(gpu.h, dA.ptr, J, dW.ptr, J, dB.ptr, dK.ptr, nk, M, N, J, V))
    gpu.end()
    keys = dK.read((M, nk), np.uint64)
    got = (0xFFFFFFFF - (keys.max(axis=1) & 0xFFFFFFFF)).astype(np.int64)
    scores = oracle.gemm(A, W[:V], bias[:V], 0, False, 1.0)
    ref = scores.argmax(axis=1)
    # the GPU sums in another order: accept a different winner only on a near tie
    bad = np.nonzero(got != ref)[0]
    for r in bad:
        assert abs(scores[r, got[r]] - scores[r, ref[r]]) < 1e-4 * max(1.0, abs(scores[r, ref[r]])), r
    assert len(bad) <= max(1, M // 500)
    assert got[0] == got[1]


def test_gemm_batched_row_map(gpu):
    """Output row m lands in row crow[m] (the per-stream cache scatter of the batched QKV / pw1)."""
    rng = np.random.default_rng(7)
    M, N, K = 96, 2048, 1024
    W = _w(rng, N, K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    rows = rng.permutation(300)[:M]
    got = run_gemm(gpu, A, W, None, 3, False, 1.0, rows=rows)
    ref = oracle.gemm(A, W, None, 3, False, 1.0)
    assert rel_err(got[rows], ref) < GEMM_TOL


@pytest.mark.parametrize("M,ldc", [(17, 1024), (96, 1024), (448, 1026)])
def test_gemm_batched_row_map_accumulate(gpu, M, ldc):
    """A residual update (accumulate, no bias or activation) above 16 rows with a row map, or on a
    row stride the partial-row fold does not take, adds into the mapped rows of C and leaves every
    other row untouched."""
    rng = np.random.default_rng([M, ldc])
    N, K = 1024, 4096
    W = _w(rng, N, K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    rows = rng.permutation(M + 40)[:M] if ldc == 1024 else None
    crows = M + 40 if rows is not None else M
    C0 = rng.standard_normal((crows, ldc)).astype(np.float32)
    got = run_gemm(gpu, A, W, None, 0, True, 0.5, C0=C0.copy(), rows=rows, ldc=ldc)
    sel = rows if rows is not None else np.arange(M)
    ref = oracle.gemm(A, W, None, 0, True, 0.5, C0=C0[sel, :N].copy())
    assert rel_err(got[sel, :N], ref) < GEMM_TOL
    untouched = np.setdiff1d(np.arange(crows), sel)
    assert np.array_equal(got[untouched], C0[untouched])
    assert np.array_equal(got[:, N:], C0[:, N:])


@pytest.mark.parametrize("kind,M", [(4, 1), (4, 4), (2, 1), (2, 4), (2, 16), (3, 5), (3, 16), (3, 100), (5, 16), (5, 100)])
def test_gemm_variants_agree(gpu, kind, M):
    """Every kernel the policy can pick computes the same GEMM (the reference's kbench.c:196-230
    cross-check, with a threshold)."""
    rng = np.random.default_rng([kind, M])
    N, K = 1024, 1024
    W = _w(rng, N, K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    got = run_gemm(gpu, A, W, bias, 1, False, 1.0, kind=kind)
    ref = oracle.gemm(A, W, bias, 1, False, 1.0)
    assert rel_err(got, ref) < GEMM_TOL


@pytest.mark.parametrize("kind", [4])
@pytest.mark.parametrize("M,N,K,act", [(1, 2560, 640, 0), (2, 1024, 4096, 0), (1, 1024, 4352, 0), (2, 640, 640, 2),
                                       (3, 2048, 1024, 3), (4, 4096, 1024, 1)])
def test_gemv_kinds(gpu, kind, M, N, K, act):
    rng = np.random.default_rng([kind, M, N, K])
    W = _w(rng, N, K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    nout = N // 2 if act == 3 else N
    C0 = rng.standard_normal((M, nout)).astype(np.float32)
    got = run_gemm(gpu, A, W, bias, act, True, 0.5, C0=C0, kind=kind)
    ref = oracle.gemm(A, W, bias, act, True, 0.5, C0=C0)
    assert rel_err(got, ref) < GEMM_TOL


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 7])
@pytest.mark.parametrize("N,act", [(4096, 1), (2048, 3), (3072, 0)])
def test_gemm_layernorm_prologue(gpu, mode, M, N, act):
    """GEMM on LN(A) (mode 1) or LN(LN(A)) (mode 2, the paired output / FF1 norm), with the first
    LayerNorm's output written to ln_out: equals the oracle's layernorm(2) followed by its GEMM."""
    import nemoasr

    L = nemoasr.lib()
    D = 1024
    rng = np.random.default_rng([mode, M, N])
    X = (2 * rng.standard_normal((M, D)) + 0.5).astype(np.float32)
    g1, g2 = [(1 + 0.1 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    b1, b2 = [(0.1 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    W = _w(rng, N, D)
    if mode == 1:
        y1 = oracle.layernorm(X, g1, b1)
        xin = y1
    else:
        y1, xin = oracle.layernorm2(X, g1, b1, g2, b2)
    ref = oracle.gemm(xin, W, None, act, False, 1.0)
    nout = N // 2 if act == 3 else N
    dX, dW, dC = gpu.put(X), gpu.put(W), gpu.alloc(M * nout * 4)
    dg1, db1, dg2, db2 = gpu.put(g1), gpu.put(b1), gpu.put(g2), gpu.put(b2)
    dout, dtmp = gpu.alloc(M * D * 4), gpu.alloc(M * D * 4)
    gpu.begin()
    gpu.check(L.nk_gemm_ln(gpu.h, dX.ptr, D, dW.ptr, D, None, dC.ptr, nout, None, M, N, D, act, 0, 1.0, mode,
                           dg1.ptr, db1.ptr, dg2.ptr, db2.ptr, dout.ptr, dtmp.ptr, 1e-5))
    gpu.end()
    assert rel_err(dC.read((M, nout)), ref) < GEMM_TOL
    assert rel_err(dout.read((M, D)), y1) < 1e-5


@pytest.mark.parametrize("M", [1, 7, 14])
def test_gemm_row_scatter(gpu, M):
    """Output row m lands in row crow[m] (the QKV / GLU write into the cache at pos)."""
    rng = np.random.default_rng(M)
    W = _w(rng, 2048, 1024)
    A = rng.standard_normal((M, 1024)).astype(np.float32)
    rows = list(range(40, 40 + M))
    C0 = rng.standard_normal((40 + M + 3, 1024)).astype(np.float32)
    got = run_gemm(gpu, A, W, None, 3, False, 1.0, C0=C0.copy(), rows=rows, ldc=1024)
    ref = oracle.gemm(A, W, None, 3, False, 1.0)
    assert rel_err(got[40:40 + M], ref) < GEMM_TOL
    np.testing.assert_array_equal(got[:40], C0[:40])
    np.testing.assert_array_equal(got[40 + M:], C0[40 + M:])


@pytest.mark.parametrize("M,D", [(1, 1024), (7, 1024), (16, 1024), (3, 256), (17, 1024), (448, 1024), (1101, 1024),
                                 (2050, 1024), (2049, 640), (3585, 1024),
                                 (50, 640), (33, 64)])
def test_layernorm_and_pair(gpu, M, D):
    import nemoasr

    L = nemoasr.lib()
    rng = np.random.default_rng([M, D])
    X = (3 * rng.standard_normal((M, D)) + 1).astype(np.float32)
    g1, b1, g2, b2 = [(1 + 0.1 * rng.standard_normal(D)).astype(np.float32) if i % 2 == 0 else
                      (0.1 * rng.standard_normal(D)).astype(np.float32) for i in range(4)]
    dX, dY1, dY2 = gpu.put(X), gpu.alloc(X.nbytes), gpu.alloc(X.nbytes)
    dg1, db1, dg2, db2 = gpu.put(g1), gpu.put(b1), gpu.put(g2), gpu.put(b2)
    gpu.begin()
    gpu.check(L.nk_layernorm2(gpu.h, dX.ptr, dg1.ptr, db1.ptr, dg2.ptr, db2.ptr, dY1.ptr, dY2.ptr, M, D, 1e-5))
    gpu.end()
    r1, r2 = oracle.layernorm2(X, g1, b1, g2, b2)
    assert rel_err(dY1.read((M, D)), r1) < 1e-5
    assert rel_err(dY2.read((M, D)), r2) < 1e-5
    gpu.begin()
    gpu.check(L.nk_layernorm(gpu.h, dX.ptr, dg2.ptr, db2.ptr, dY1.ptr, M, D, 1e-5))
    gpu.end()
    assert rel_err(dY1.read((M, D)), oracle.layernorm(X, g2, b2)) < 1e-5


@pytest.mark.parametrize("c,cache", [(1, 0), (1, 56), (7, 0), (7, 56), (14, 56), (16, 56), (7, 23)])
def test_attention_rel(gpu, c, cache):
    import nemoasr

    lib = nemoasr.lib()
    H, dh, D, Lmax = 8, 128, 1024, 72
    L = cache + c
    rng = np.random.default_rng([c, cache])
    pos = cache + 5
    kv = rng.standard_normal((pos + c + 2, 3 * D)).astype(np.float32)
    P = rng.standard_normal((2 * Lmax - 1, D)).astype(np.float32)
    bu = (0.1 * rng.standard_normal(D)).astype(np.float32)
    bv = (0.1 * rng.standard_normal(D)).astype(np.float32)
    Q = kv[pos:pos + c, :]
    K = kv[pos - cache:pos + c, D:2 * D]
    V = kv[pos - cache:pos + c, 2 * D:]
    ref = oracle.attention_rel(Q, K, V, P, bu, bv, c, L, Lmax, H, dh)
    dkv, dP, dbu, dbv, dO = gpu.put(kv), gpu.put(P), gpu.put(bu), gpu.put(bv), gpu.alloc(c * D * 4)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dh)))
    gpu.begin()
    row = 3 * D * 4
    gpu.check(lib.nk_attention_rel(gpu.h, dkv.at(pos * row), 3 * D, dkv.at((pos - cache) * row + D * 4),
                                   dkv.at((pos - cache) * row + 2 * D * 4), 3 * D, dP.ptr, dbu.ptr, dbv.ptr, dO.ptr,
                                   c, L, Lmax, H, dh, D, scale))
    gpu.end()
    assert rel_err(dO.read((c, D)), ref) < 1e-5
    desc = np.zeros(20, np.int32)
    desc[:4] = [pos, cache, L, c]
    ddesc = gpu.put(desc)
    gpu.begin()
    gpu.check(lib.nk_attention_rel_desc(gpu.h, dkv.ptr, 3 * D, ddesc.ptr, dP.ptr, dbu.ptr, dbv.ptr, dO.ptr, c, Lmax,
                                        H, dh, D, scale))
    gpu.end()
    assert rel_err(dO.read((c, D)), ref) < 1e-5


@pytest.mark.parametrize("Lmax", [72, 73])
def test_attention_batched_streams(gpu, Lmax):
    """Several streams' chunks in one launch, each at its own cache position and fill level: the
    per-row table kernel and the whole-chunk kernel against the oracle chunk by chunk."""
    import nemoasr

    lib = nemoasr.lib()
    H, dh, D = 8, 128, 1024
    rng = np.random.default_rng([Lmax, 5])
    chunks_spec = [(7, 56), (7, 0), (1, 56), (14, 56), (16, 56), (9, 23), (7, 49), (3, 1)]
    cap = 96
    kv = rng.standard_normal((len(chunks_spec) * cap, 3 * D)).astype(np.float32)
    P = rng.standard_normal((2 * Lmax - 1, D)).astype(np.float32)
    bu = (0.1 * rng.standard_normal(D)).astype(np.float32)
    bv = (0.1 * rng.standard_normal(D)).astype(np.float32)
    rows, chunks, refs, m = [], [], [], 0
    for s, (c, cache) in enumerate(chunks_spec):
        pos = s * cap + cache + 3 + s  # first cache row of the chunk inside stream s's region
        L = cache + c
        Q = kv[pos:pos + c, :]
        K = kv[pos - cache:pos + c, D:2 * D]
        V = kv[pos - cache:pos + c, 2 * D:]
        refs.append(oracle.attention_rel(Q, K, V, P, bu, bv, c, L, Lmax, H, dh))
        for i in range(c):
            rows += [pos + i, i, c, cache]
        chunks += [pos, m, c, cache]
        m += c
    ref = np.concatenate(refs)
    dkv, dP, dbu, dbv = gpu.put(kv), gpu.put(P), gpu.put(bu), gpu.put(bv)
    drows, dch = gpu.put(np.asarray(rows, np.int32)), gpu.put(np.asarray(chunks, np.int32))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dh)))
    for which in ("rows", "chunks"):
        dO = gpu.alloc(m * D * 4)
        gpu.begin()
        if which == "rows":
            gpu.check(lib.nk_attention_rel_rows(gpu.h, dkv.ptr, 3 * D, drows.ptr, m, dP.ptr, dbu.ptr, dbv.ptr, dO.ptr,
                                                Lmax, H, dh, D, scale))
        else:
            gpu.check(lib.nk_attention_rel_chunks(gpu.h, dkv.ptr, 3 * D, dch.ptr, len(chunks_spec), dP.ptr, dbu.ptr,
                                                  dbv.ptr, dO.ptr, Lmax, H, dh, D, scale))
        gpu.end()
        assert rel_err(dO.read((m, D)), ref) < 1e-5, which
        dO.free()


@pytest.mark.parametrize("c", [1, 7, 14])
def test_dwconv_ln_silu(gpu, c):
    import nemoasr

    lib = nemoasr.lib()
    D, taps = 1024, 9
    rng = np.random.default_rng(c)
    din = rng.standard_normal((taps - 1 + c, D)).astype(np.float32)
    W = (rng.standard_normal((D, taps)) / 3).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b = (0.1 * rng.standard_normal(D)).astype(np.float32)
    ref = oracle.dwconv_ln_silu(din, W, g, b, c)
    ddin, dW, dg, db, dY = gpu.put(din), gpu.put(W), gpu.put(g), gpu.put(b), gpu.alloc(c * D * 4)
    gpu.begin()
    gpu.check(lib.nk_dwconv_ln_silu(gpu.h, ddin.ptr, dW.ptr, dg.ptr, db.ptr, dY.ptr, c, D, taps, 1e-5))
    gpu.end()
    assert rel_err(dY.read((c, D)), ref) < 1e-5


@pytest.mark.parametrize("c,cache,cpw", [(1, 56, 16), (1, 56, 8), (1, 56, 4), (1, 0, 16), (2, 56, 16), (4, 40, 8)])
def test_attention_out_fused(gpu, c, cache, cpw):
    """Attention fused with its output projection: residual += attention . Wo^T against the
    oracle's attention times the same bf16 weights (float64 product), and against the two
    separate launches.  Each head writes its share of the projection as a partial row and the shares
    are added to the residual in head order (no atomics); the float64 reference sums in another
    order, so float tolerance applies against it."""
    import nemoasr

    lib = nemoasr.lib()
    H, dh, D, Lmax = 8, 128, 1024, 72
    L = cache + c
    rng = np.random.default_rng([c, cache, cpw])
    pos = cache + 5
    kv = rng.standard_normal((pos + c + 2, 3 * D)).astype(np.float32)
    P = rng.standard_normal((2 * Lmax - 1, D)).astype(np.float32)
    bu = (0.1 * rng.standard_normal(D)).astype(np.float32)
    bv = (0.1 * rng.standard_normal(D)).astype(np.float32)
    Wo = _w(rng, D, D)
    res0 = rng.standard_normal((c, D)).astype(np.float32)
    att = oracle.attention_rel(kv[pos:pos + c, :], kv[pos - cache:pos + c, D:2 * D], kv[pos - cache:pos + c, 2 * D:],
                               P, bu, bv, c, L, Lmax, H, dh)
    ref = res0 + (att.astype(np.float64) @ oracle.bf16_to_f32(Wo).astype(np.float64).T)
    desc = np.zeros(20, np.int32)
    desc[:4] = [pos, cache, L, c]
    dkv, dP, dbu, dbv, dW = gpu.put(kv), gpu.put(P), gpu.put(bu), gpu.put(bv), gpu.put(Wo)
    ddesc, dres, dO, dres2 = gpu.put(desc), gpu.put(res0), gpu.alloc(c * D * 4), gpu.put(res0)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dh)))
    prev = lib.nk_fuse_shape(cpw, 0)
    try:
        gpu.begin()
        gpu.check(lib.nk_attention_out_desc(gpu.h, dkv.ptr, 3 * D, ddesc.ptr, dP.ptr, dbu.ptr, dbv.ptr, c, Lmax, H, dh,
                                            D, scale, dW.ptr, D, dres.ptr, D, 1.0))
        gpu.check(lib.nk_attention_rel_desc(gpu.h, dkv.ptr, 3 * D, ddesc.ptr, dP.ptr, dbu.ptr, dbv.ptr, dO.ptr, c, Lmax,
                                            H, dh, D, scale))
        gpu.check(lib.nk_gemm(gpu.h, dO.ptr, D, dW.ptr, D, None, dres2.ptr, D, c, D, D, 0, 1, 1.0))
        gpu.end()
    finally:
        lib.nk_fuse_shape(prev // 16, prev % 16)
    got, sep = dres.read((c, D)), dres2.read((c, D))
    assert rel_err(got, ref) < 1e-5
    assert rel_err(got, sep) < 1e-6


@pytest.mark.parametrize("c,D,N,nc,acc", [(1, 1024, 1024, 2, 1), (1, 1024, 1024, 1, 1), (1, 1024, 1024, 4, 0),
                                          (2, 1024, 1024, 2, 1), (2, 1024, 1000, 4, 1), (1, 256, 192, 2, 1),
                                          (2, 64, 64, 1, 0)])
def test_dwconv_pw_fused(gpu, c, D, N, nc, acc):
    """Depthwise conv + LN + SiLU as the prologue of the pointwise GEMV: bit-identical to the two
    separate launches (same per-thread conv, reductions and dot-product order), and against the
    oracle's conv times the same bf16 weights."""
    import nemoasr

    lib = nemoasr.lib()
    taps, eps, pos = 9, 1e-5, 20
    rng = np.random.default_rng([c, D, N, nc])
    din = rng.standard_normal((pos + c + 3, D)).astype(np.float32)
    Wd = (rng.standard_normal((D, taps)) / 3).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b = (0.1 * rng.standard_normal(D)).astype(np.float32)
    Wp = _w(rng, N, D)
    C0 = rng.standard_normal((c, N)).astype(np.float32)
    y = oracle.dwconv_ln_silu(din[pos - (taps - 1):pos + c], Wd, g, b, c)
    ref = (C0 if acc else 0) + y.astype(np.float64) @ oracle.bf16_to_f32(Wp).astype(np.float64).T
    desc = np.zeros(20, np.int32)
    desc[:4] = [pos, 0, c, c]
    ddin, dWd, dg, db, dWp, ddesc = gpu.put(din), gpu.put(Wd), gpu.put(g), gpu.put(b), gpu.put(Wp), gpu.put(desc)
    dC, dC2, dY = gpu.put(C0), gpu.put(C0), gpu.alloc(c * D * 4)
    prev = lib.nk_fuse_shape(0, nc)
    try:
        gpu.begin()
        gpu.check(lib.nk_dwconv_pw_desc(gpu.h, ddin.ptr, ddesc.ptr, dWd.ptr, dg.ptr, db.ptr, eps, dWp.ptr, D, dC.ptr, N,
                                        c, D, N, acc, 1.0))
        gpu.check(lib.nk_dwconv_ln_silu_desc(gpu.h, ddin.ptr, ddesc.ptr, dWd.ptr, dg.ptr, db.ptr, dY.ptr, c, D, taps,
                                             eps))
        gpu.check(lib.nk_gemm(gpu.h, dY.ptr, D, dWp.ptr, D, None, dC2.ptr, N, c, N, D, 0, acc, 1.0))
        gpu.end()
    finally:
        lib.nk_fuse_shape(0, prev % 16)
    got = dC.read((c, N))
    np.testing.assert_array_equal(got, dC2.read((c, N)))
    assert rel_err(got, ref) < 1e-5


class _MelTables(C.Structure):
    _fields_ = [("win", C.POINTER(C.c_float)), ("fb", C.POINTER(C.c_float)), ("fb_lo", C.POINTER(C.c_int)),
                ("fb_hi", C.POINTER(C.c_int)), ("tw_re", C.POINTER(C.c_double)), ("tw_im", C.POINTER(C.c_double)),
                ("rev", C.POINTER(C.c_ushort))]


@pytest.mark.parametrize("seconds,seed", [(0.5, 1), (1.37, 2), (0.02, 3)])
def test_mel_frames(gpu, seconds, seed):
    """GPU log-mel frames against the host front end's own computation on the same sample spans
    (the first frames read reflected samples at the start, the last ones at the final end): the
    spectra are computed identically in double; the device log and the host's libm log round
    differently in about half the values, by at most two ulp."""
    import nemoasr

    L = nemoasr.lib()
    f32p = C.POINTER(C.c_float)
    L.melfe_create.restype = C.c_void_p
    L.melfe_destroy.argtypes = [C.c_void_p]
    L.melfe_append.restype = C.c_size_t
    L.melfe_append.argtypes = [C.c_void_p, f32p, C.c_size_t, C.c_int]
    L.melfe_span_len.restype = C.c_size_t
    L.melfe_span_len.argtypes = [C.c_size_t]
    L.melfe_take.restype = C.c_size_t
    L.melfe_take.argtypes = [C.c_void_p, f32p, C.c_size_t]
    L.melfe_compute.argtypes = [C.c_void_p, f32p, C.c_size_t, f32p]
    L.melfe_tables.argtypes = [C.c_void_p, C.POINTER(_MelTables)]
    x = (0.1 * synth.make_audio(seconds, seed=seed)).astype(np.float32)
    m = L.melfe_create()
    try:
        cnt = L.melfe_append(m, x.ctypes.data_as(f32p), x.size, 1)
        span = np.zeros(L.melfe_span_len(cnt), np.float32)
        assert L.melfe_take(m, span.ctypes.data_as(f32p), cnt) == cnt
        ref = np.zeros((cnt, 128), np.float32)
        L.melfe_compute(m, span.ctypes.data_as(f32p), cnt, ref.ctypes.data_as(f32p))
        t = _MelTables()
        L.melfe_tables(m, C.byref(t))
        win = np.ctypeslib.as_array(t.win, (512,)).copy()
        fb = np.ctypeslib.as_array(t.fb, (128 * 257,)).copy()
        lo = np.ctypeslib.as_array(t.fb_lo, (128,)).copy()
        hi = np.ctypeslib.as_array(t.fb_hi, (128,)).copy()
        twr = np.ctypeslib.as_array(t.tw_re, (256,)).copy()
        twi = np.ctypeslib.as_array(t.tw_im, (256,)).copy()
        rev = np.ctypeslib.as_array(t.rev, (512,)).copy()
    finally:
        L.melfe_destroy(m)
    # frames written to shuffled output rows, to check the row table
    perm = np.random.default_rng(seed).permutation(cnt).astype(np.int32)
    tab = np.stack([np.arange(cnt, dtype=np.int32) * 160, perm], axis=1).astype(np.int32)
    bufs = [gpu.put(a) for a in (span, tab, win, fb, lo, hi, twr, twi, rev)]
    dout = gpu.alloc(cnt * 128 * 4)
    gpu.begin()
    gpu.check(L.nk_mel_frames(gpu.h, bufs[0].ptr, bufs[1].ptr, cnt, *[b.ptr for b in bufs[2:]], dout.ptr))
    gpu.end()
    got = dout.read((cnt, 128))[perm]
    assert np.abs(got - ref).max() <= 4e-6, np.abs(got - ref).max()
    ulps = np.abs(got - ref) / np.spacing(np.abs(ref))
    assert ulps.max() <= 2, ulps.max()


@pytest.mark.parametrize("nwin", [8, 24, 72, 128, 33])
def test_subsampling_convs(gpu, nwin):
    import nemoasr

    lib = nemoasr.lib()
    rng = np.random.default_rng(nwin)
    F, C = 128, 256
    X = rng.standard_normal((nwin, F)).astype(np.float32)
    W0 = (rng.standard_normal((C, 9)) / 3).astype(np.float32)
    b0 = (0.1 * rng.standard_normal(C)).astype(np.float32)
    W2 = (rng.standard_normal((C, 9)) / 3).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(C)).astype(np.float32)
    y0 = oracle.conv2d_c1_s2_relu(X, W0, b0)
    y1 = oracle.dwconv2d_s2(y0, W2, b2)
    fl = oracle.flatten_cf(y1)
    T1, F1 = y0.shape[:2]
    T2, F2 = y1.shape[:2]
    dX, dW0, db0, dW2, db2 = gpu.put(X), gpu.put(W0), gpu.put(b0), gpu.put(W2), gpu.put(b2)
    dy0, dy1, dfl = gpu.alloc(y0.nbytes), gpu.alloc(y1.nbytes), gpu.alloc(fl.nbytes)
    gpu.begin()
    gpu.check(lib.nk_conv2d_c1_s2_relu(gpu.h, dX.ptr, dW0.ptr, db0.ptr, dy0.ptr, nwin, F, T1, F1, C))
    gpu.check(lib.nk_dwconv2d_s2(gpu.h, dy0.ptr, dW2.ptr, db2.ptr, dy1.ptr, T1, F1, T2, F2, C))
    gpu.check(lib.nk_flatten_cf(gpu.h, dy1.ptr, dfl.ptr, T2, F2, C))
    gpu.end()
    assert rel_err(dy0.read(y0.shape), y0) < 1e-6
    assert rel_err(dy1.read(y1.shape), y1) < 1e-6
    np.testing.assert_array_equal(dfl.read(fl.shape), oracle.flatten_cf(dy1.read(y1.shape)))


@pytest.mark.parametrize("nwin,batch,F,C", [(9, 1, 128, 256), (23, 3, 128, 256), (61, 2, 128, 256),
                                          (121, 40, 128, 256), (128, 9, 128, 256), (121, 12, 128, 256),
                                          (17, 2, 80, 96)])
def test_subsampling_conv02_fused(gpu, nwin, batch, F, C):
    """conv 0 + conv 2 in one launch equals the two launches bit for bit (and the oracle), with
    whole-row, 4-column and 1-column workgroups (the launcher picks by rows x windows)."""
    import nemoasr

    lib = nemoasr.lib()
    rng = np.random.default_rng(nwin * 7 + batch)
    X = rng.standard_normal((batch, nwin, F)).astype(np.float32)
    W0 = (rng.standard_normal((C, 9)) / 3).astype(np.float32)
    b0 = (0.1 * rng.standard_normal(C)).astype(np.float32)
    W2 = (rng.standard_normal((C, 9)) / 3).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(C)).astype(np.float32)
    T1, F1 = nwin // 2 + 1, F // 2 + 1
    T2, F2 = T1 // 2 + 1, F1 // 2 + 1
    dX, dW0, db0, dW2, db2 = gpu.put(X), gpu.put(W0), gpu.put(b0), gpu.put(W2), gpu.put(b2)
    dy0 = gpu.alloc(batch * T1 * F1 * C * 4)
    dy1, dyf = gpu.alloc(batch * T2 * F2 * C * 4), gpu.alloc(batch * T2 * F2 * C * 4)
    gpu.begin()
    gpu.check(lib.nk_conv2d_c1_s2_relu_b(gpu.h, dX.ptr, dW0.ptr, db0.ptr, dy0.ptr, nwin, F, T1, F1, C, batch))
    gpu.check(lib.nk_dwconv2d_s2_b(gpu.h, dy0.ptr, dW2.ptr, db2.ptr, dy1.ptr, T1, F1, T2, F2, C, batch))
    gpu.check(lib.nk_conv2d_c1_dw_s2_b(gpu.h, dX.ptr, dW0.ptr, db0.ptr, dW2.ptr, db2.ptr, dyf.ptr, nwin, F, T1, F1,
                                       T2, F2, C, batch))
    gpu.end()
    sep, fused = dy1.read((batch, T2, F2, C)), dyf.read((batch, T2, F2, C))
    np.testing.assert_array_equal(fused, sep)
    for w in range(batch):
        ref = oracle.dwconv2d_s2(oracle.conv2d_c1_s2_relu(X[w], W0, b0), W2, b2)
        assert ref.shape == (T2, F2, C)
        assert rel_err(fused[w], ref) < 1e-6


def test_lstm_cell_rows(gpu):
    from conftest import lstm_cell_rows

    H = 640
    rng = np.random.default_rng(7)
    gates = (2 * rng.standard_normal(4 * H)).astype(np.float32)
    c_in = rng.standard_normal(H).astype(np.float32)
    rc, rh = oracle.lstm_cell(gates, c_in)
    co, ho = lstm_cell_rows(gpu, gates, c_in)
    assert rel_err(co, rc) < 1e-6
    assert rel_err(ho, rh) < 1e-6


@pytest.mark.parametrize("device_loop", [True, False])
@pytest.mark.parametrize("rows", [1, 5, 16])
def test_joint_argmax(gpu, rows, device_loop):
    """The full-size joint (V = 1025 classes, 640 wide) through the batched loop's kernels."""
    from conftest import joint_argmax_rows

    V, H = 1025, 640
    rng = np.random.default_rng(rows)
    W = _w(rng, V, H)
    bias = (0.1 * rng.standard_normal(V)).astype(np.float32)
    enc = rng.standard_normal((rows, H)).astype(np.float32)
    pred = rng.standard_normal(H).astype(np.float32)
    got = joint_argmax_rows(gpu, enc, pred, W, bias, device_loop)
    for r in range(rows):
        i, v, logits = oracle.joint_argmax(enc[r], pred, W, bias)
        assert got[r][0] == i
        assert abs(got[r][1] - v) <= 1e-5 * max(1.0, abs(v))


@pytest.mark.parametrize("device_loop", [True, False])
def test_joint_argmax_tie_lowest_index(gpu, device_loop):
    """Exact ties resolve to the lowest class index (src/kernels.metal:516, :545)."""
    from conftest import joint_argmax_rows

    V, H = 1025, 640
    W = np.zeros((V, H), np.uint16)
    bias = np.zeros(V, np.float32)
    bias[[17, 300, 999]] = 1.0
    enc = np.ones((1, H), np.float32)
    pred = np.zeros(H, np.float32)
    assert joint_argmax_rows(gpu, enc, pred, W, bias, device_loop)[0][0] == 17


@pytest.mark.parametrize("cols", [96, 97])  # 16-byte rows (compact_rows4) and the 4-byte fallback
def test_compact_rows(gpu, cols):
    import nemoasr

    lib = nemoasr.lib()
    nbuf, rows_total = 3, 40
    rng = np.random.default_rng(3)
    X = rng.standard_normal((nbuf, rows_total, cols)).astype(np.float32)
    d = gpu.put(X)
    gpu.begin()
    gpu.check(lib.nk_compact(gpu.h, d.ptr, rows_total * cols, nbuf, 10, cols, 25, 2))
    gpu.end()
    Y = X.copy()
    Y[:, 2:12] = X[:, 25:35]
    np.testing.assert_array_equal(d.read(X.shape), Y)
