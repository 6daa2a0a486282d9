"""Split rows: activations stored as bf16 hi = RNE(a), lo = RNE(a - hi) by their producer.

The many-row MFMA kernels multiply A as hi and lo bf16 halves either way; with split rows the
producer forms them once instead of every consumer workgroup forming them in its K loop.  The
split must be invisible: every split-row kernel is checked bit for bit against its f32 form, with
the split done here in numpy (round to nearest even, the rounding the kernels use), and the GEMMs
against the oracle.
"""
import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu


def split_rows(x):
    """[M][K] f32 -> [M][2K] bf16 bits: K hi then K lo per row."""
    x = np.ascontiguousarray(x, np.float32)
    hi = oracle.f32_to_bf16(x)
    lo = oracle.f32_to_bf16(x - oracle.bf16_to_f32(hi))
    return np.concatenate([hi, lo], axis=1)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else np.uint16)


def w_bf16(rng, n, k):
    return oracle.f32_to_bf16(rng.standard_normal((n, k)).astype(np.float32) / np.sqrt(k))


def gemm_split(gpu, A, W, bias, act, acc, alpha, split_in, split_out, C0=None, crow=None, ksplit=-1):
    import nemoasr

    L = nemoasr.lib()
    M, K = A.shape
    N = W.shape[0]
    nout = N // 2 if act == 3 else N
    dA = gpu.put(split_rows(A) if split_in else A)
    dW = gpu.put(W)
    dB = gpu.put(bias) if bias is not None else None
    rows = M if crow is None else int(max(crow)) + 1
    C0 = np.zeros((rows, nout), np.float32) if C0 is None else C0
    dC = gpu.alloc(M * 2 * nout * 2) if split_out else gpu.put(C0)
    dR = gpu.put(np.asarray(crow, np.int32)) if crow is not None else None
    prev = L.nk_gemm_ksplit(ksplit)
    try:
        gpu.begin()
        gpu.check(L.nk_gemm_split(gpu.h, None if split_in else dA.ptr, dA.ptr if split_in else None, 2 * K if split_in else K,
                                  dW.ptr, K, dB.ptr if dB else None, None if split_out else dC.ptr,
                                  dC.ptr if split_out else None, 2 * nout if split_out else nout,
                                  dR.ptr if dR else None, M, N, K, act, int(acc), alpha))
        gpu.end()
    finally:
        L.nk_gemm_ksplit(prev)
    out = dC.read((M, 2 * nout), np.uint16) if split_out else dC.read((rows, nout))
    for b in (dA, dW, dB, dC, dR):
        if b is not None:
            b.free()
    return out


# the batched encoder's GEMMs at 64 x 7 and 256 x 14 rows and a ragged row count
@pytest.mark.parametrize("M", [448, 3584, 301])
@pytest.mark.parametrize("N,K,act,acc,bias", [
    (4096, 1024, 1, 0, False),   # FF up + SiLU
    (1024, 4096, 0, 1, False),   # FF down, residual update
    (3072, 1024, 0, 0, False),   # QKV (row map)
    (2048, 1024, 3, 0, False),   # pw1 + GLU (row map)
    (1024, 1024, 0, 1, False),   # out / pw2, residual update
    (2048, 1024, 2, 0, True),    # prompt W0 + ReLU
    (1024, 2048, 0, 0, True),    # prompt W2
])
def test_gemm_split_input_bits(gpu, M, N, K, act, acc, bias):
    """Split-row A gives the bits of f32 A (each residual update also with its K split forced on
    and off), and the oracle's values."""
    rng = np.random.default_rng([M, N, K, act])
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = w_bf16(rng, N, K)
    b = (0.1 * rng.standard_normal(N)).astype(np.float32) if bias else None
    nout = N // 2 if act == 3 else N
    C0 = rng.standard_normal((M, nout)).astype(np.float32) if acc else None
    crow = rng.permutation(M + 37)[:M] if N in (3072, 2048) and not bias else None
    alpha = 0.5 if acc else 1.0
    ref_f32 = gemm_split(gpu, A, W, b, act, acc, alpha, False, False, C0=None if C0 is None else C0.copy(), crow=crow)
    for ks in ((-1, 0, 1) if acc else (-1,)):
        got = gemm_split(gpu, A, W, b, act, acc, alpha, True, False, C0=None if C0 is None else C0.copy(), crow=crow,
                         ksplit=ks)
        assert np.array_equal(bits(got), bits(ref_f32)), ks
    ref = oracle.gemm(A, W, b, act, acc, alpha, C0=C0)
    assert rel_err(ref_f32[crow] if crow is not None else ref_f32, ref) < 2e-5


@pytest.mark.parametrize("M", [448, 3584, 77])
@pytest.mark.parametrize("split_in", [False, True])
@pytest.mark.parametrize("N,K,act,bias", [(4096, 1024, 1, False), (2048, 1024, 2, True)])
def test_gemm_split_output_bits(gpu, M, N, K, act, bias, split_in):
    """Split-row outputs (FF up + SiLU, prompt W0 + ReLU) are exactly the split of the f32 outputs."""
    rng = np.random.default_rng([M, N, K, 9])
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = w_bf16(rng, N, K)
    b = (0.1 * rng.standard_normal(N)).astype(np.float32) if bias else None
    f32 = gemm_split(gpu, A, W, b, act, False, 1.0, split_in, False)
    got = gemm_split(gpu, A, W, b, act, False, 1.0, split_in, True)
    assert np.array_equal(got, split_rows(f32))


@pytest.mark.parametrize("M,paired", [(448, False), (448, True), (3585, True), (1101, False), (2050, True), (20, True)])
def test_layernorm_split_bits(gpu, M, paired):
    import nemoasr

    L = nemoasr.lib()
    D = 1024
    rng = np.random.default_rng([M, 3])
    X = (3 * rng.standard_normal((M, D)) + 1).astype(np.float32)
    g1, g2 = [(1 + 0.1 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    b1, b2 = [(0.1 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    dX, dg1, db1, dg2, db2 = gpu.put(X), gpu.put(g1), gpu.put(b1), gpu.put(g2), gpu.put(b2)
    dY1, dY2, dYs, dZ = gpu.alloc(X.nbytes), gpu.alloc(X.nbytes), gpu.alloc(X.nbytes), gpu.alloc(X.nbytes)
    gpu.begin()
    if paired:
        gpu.check(L.nk_layernorm2(gpu.h, dX.ptr, dg1.ptr, db1.ptr, dg2.ptr, db2.ptr, dY1.ptr, dY2.ptr, M, D, 1e-5))
        gpu.check(L.nk_layernorm2_split(gpu.h, dX.ptr, None, dg1.ptr, db1.ptr, dg2.ptr, db2.ptr, dZ.ptr, dYs.ptr, M, D,
                                        1e-5))
    else:
        gpu.check(L.nk_layernorm2(gpu.h, dX.ptr, dg1.ptr, db1.ptr, None, None, dY2.ptr, None, M, D, 1e-5))
        gpu.check(L.nk_layernorm2_split(gpu.h, dX.ptr, None, dg1.ptr, db1.ptr, None, None, None, dYs.ptr, M, D, 1e-5))
    gpu.end()
    if paired:
        assert np.array_equal(bits(dZ.read((M, D))), bits(dY1.read((M, D))))
    y = dY2.read((M, D))
    assert np.array_equal(dYs.read((M, 2 * D), np.uint16), split_rows(y))
    ref = oracle.layernorm2(X, g1, b1, g2, b2)[1] if paired else oracle.layernorm(X, g1, b1)
    assert rel_err(y, ref) < 1e-5


def test_layernorm_zero_width_is_an_error(gpu):
    """Rows of zero floats are refused before any launch (the row kernels clamp their loads into the
    row, which needs at least one float4)."""
    import nemoasr

    L = nemoasr.lib()
    dX, dg, dYs = gpu.alloc(4096), gpu.alloc(4096), gpu.alloc(4096)
    for call in (lambda: L.nk_layernorm2_split(gpu.h, dX.ptr, None, dg.ptr, dg.ptr, None, None, None, dYs.ptr, 4, 0, 1e-5),
                 lambda: L.nk_layernorm2(gpu.h, dX.ptr, dg.ptr, dg.ptr, None, None, dYs.ptr, None, 4, 0, 1e-5)):
        gpu.begin()
        assert call() != 0
        with pytest.raises(RuntimeError, match="layernorm"):
            gpu.end()


def test_attention_chunks_split_bits(gpu):
    import nemoasr

    lib = nemoasr.lib()
    H, dh, D, Lmax = 8, 128, 1024, 72
    rng = np.random.default_rng(11)
    spec = [(7, 56), (7, 0), (14, 56), (16, 56), (9, 23), (1, 40)]
    cap = 96
    kv = rng.standard_normal((len(spec) * cap, 3 * D)).astype(np.float32)
    P = rng.standard_normal((2 * Lmax - 1, D)).astype(np.float32)
    bu, bv = [(0.1 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    chunks, m = [], 0
    for s, (c, cache) in enumerate(spec):
        chunks += [s * cap + cache + 3, m, c, cache]
        m += c
    dkv, dP, dbu, dbv = gpu.put(kv), gpu.put(P), gpu.put(bu), gpu.put(bv)
    dch = gpu.put(np.asarray(chunks, np.int32))
    dO, dOs = gpu.alloc(m * D * 4), gpu.alloc(m * D * 4)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dh)))
    gpu.begin()
    gpu.check(lib.nk_attention_rel_chunks(gpu.h, dkv.ptr, 3 * D, dch.ptr, len(spec), dP.ptr, dbu.ptr, dbv.ptr, dO.ptr,
                                          Lmax, H, dh, D, scale))
    gpu.check(lib.nk_attention_rel_chunks_split(gpu.h, dkv.ptr, 3 * D, dch.ptr, len(spec), dP.ptr, dbu.ptr, dbv.ptr,
                                                dOs.ptr, Lmax, H, dh, D, scale))
    gpu.end()
    assert np.array_equal(dOs.read((m, 2 * D), np.uint16), split_rows(dO.read((m, D))))


@pytest.mark.parametrize("M,D", [(40, 1024), (3585, 1024), (2050, 512)])
def test_dwconv_rows_split_bits(gpu, M, D):
    import nemoasr

    lib = nemoasr.lib()
    taps = 9
    rng = np.random.default_rng(12)
    din = rng.standard_normal((4000, D)).astype(np.float32)
    W = (rng.standard_normal((D, taps)) / 3).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b = (0.1 * rng.standard_normal(D)).astype(np.float32)
    pos = [10 + 4 * i for i in range(40)] + list(8 + rng.integers(0, 3990, M - 40))
    rows = []
    for p in pos:
        rows += [int(p), 0, 1, 0]
    ddin, dW, dg, db = gpu.put(din), gpu.put(W), gpu.put(g), gpu.put(b)
    drows = gpu.put(np.asarray(rows, np.int32))
    dY, dYs, dY40 = gpu.alloc(M * D * 4), gpu.alloc(M * D * 4), gpu.alloc(40 * D * 4)
    gpu.begin()
    gpu.check(lib.nk_dwconv_ln_silu_rows(gpu.h, ddin.ptr, drows.ptr, M, dW.ptr, dg.ptr, db.ptr, dY.ptr, D, taps, 1e-5))
    gpu.check(lib.nk_dwconv_ln_silu_rows_split(gpu.h, ddin.ptr, drows.ptr, M, dW.ptr, dg.ptr, db.ptr, None, dYs.ptr, D,
                                               taps, 1e-5))
    gpu.check(lib.nk_dwconv_ln_silu_rows(gpu.h, ddin.ptr, drows.ptr, 40, dW.ptr, dg.ptr, db.ptr, dY40.ptr, D, taps, 1e-5))
    gpu.end()
    y = dY.read((M, D))
    assert np.array_equal(dYs.read((M, 2 * D), np.uint16), split_rows(y))
    # the same row gives the same bits at any row count
    assert np.array_equal(bits(y[:40]), bits(dY40.read((40, D))))
    pick = list(range(40)) + list(range(40, M, max(1, M // 200))) + [M - 1]
    ref = np.concatenate([oracle.dwconv_ln_silu(din[pos[i] - 8:pos[i] + 1], W, g, b, 1) for i in pick])
    assert rel_err(y[pick], ref) < 1e-5


@pytest.mark.parametrize("M,K,split_in,paired,D", [(448, 4096, True, True, 1024), (448, 1024, True, False, 1024),
                                                   (3584, 4096, False, True, 1024), (301, 1024, False, False, 1024),
                                                   # 8 parts (past the four loaded ahead), and rows narrower than 1024
                                                   (301, 8192, False, True, 1024), (130, 4096, True, True, 512)])
def test_resid_pending_folded_by_layernorm(gpu, M, K, split_in, paired, D):
    """A residual update left pending (nk_gemm_resid: the K blocks' partial rows, K split or not) and
    applied by the LayerNorm that follows gives the residual and LayerNorm output of the update done
    by nk_gemm_split then the plain LayerNorm, bit for bit."""
    import ctypes as C

    import nemoasr

    L = nemoasr.lib()
    rng = np.random.default_rng([M, K, 4])
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = w_bf16(rng, D, K)
    X = rng.standard_normal((M, D)).astype(np.float32)
    g1, g2 = [(1 + 0.1 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    b1, b2 = [(0.1 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    dA = gpu.put(split_rows(A) if split_in else A)
    lda = 2 * K if split_in else K
    dW, dg1, db1, dg2, db2 = gpu.put(W), gpu.put(g1), gpu.put(b1), gpu.put(g2), gpu.put(b2)
    out = []
    for ks in (0, 1, None):
        dX, dY1, dYs = gpu.put(X), gpu.alloc(X.nbytes), gpu.alloc(X.nbytes)
        aa, a2 = (None, dA.ptr) if split_in else (dA.ptr, None)
        prev = L.nk_gemm_ksplit(-1 if ks is None else ks)
        try:
            gpu.begin()
            if ks is None:  # the update applied by the call, then the plain split LayerNorm
                gpu.check(L.nk_gemm_split(gpu.h, aa, a2, lda, dW.ptr, K, None, dX.ptr, None, D, None, M, D, K, 0, 1, 0.5))
                pend = None
            else:
                r = nemoasr.Resid()
                gpu.check(L.nk_gemm_resid(gpu.h, aa, a2, lda, dW.ptr, K, dX.ptr, D, M, D, K, 0.5, C.byref(r)))
                assert r.nparts == (1 if ks == 0 else K // 1024 if K > 1024 else 2)
                pend = C.byref(r)
            gpu.check(L.nk_layernorm2_split(gpu.h, dX.ptr, pend, dg1.ptr, db1.ptr, dg2.ptr if paired else None,
                                            db2.ptr if paired else None, dY1.ptr if paired else None, dYs.ptr, M, D,
                                            1e-5))
            gpu.end()
        finally:
            L.nk_gemm_ksplit(prev)
        out.append((dX.read((M, D)), dYs.read((M, 2 * D), np.uint16), dY1.read((M, D)) if paired else None))
    for x, ys, y1 in out[:2]:
        assert np.array_equal(bits(x), bits(out[2][0]))
        assert np.array_equal(ys, out[2][1])
        if paired:
            assert np.array_equal(bits(y1), bits(out[2][2]))
    ref = oracle.gemm(A, W, None, 0, True, 0.5, C0=X)
    assert rel_err(out[2][0], ref) < 2e-5


@pytest.mark.parametrize("M,nparts,N,act,mode,xf", [
    (1, 8, 2048, 3, 1, True), (2, 8, 2048, 3, 1, True), (4, 8, 2048, 3, 1, True), (3, 3, 4096, 1, 2, True),
    (1, 11, 3072, 0, 1, True), (7, 8, 2048, 3, 1, True), (1, 0, 2048, 3, 1, True), (2, 3, 4096, 1, 2, False),
    (7, 4, 3072, 0, 1, True), (7, 4, 2048, 3, 1, True), (14, 4, 4096, 1, 1, True), (14, 4, 4096, 1, 2, False),
    (16, 2, 2048, 3, 2, True), (5, 1, 1024, 0, 1, True), (7, 0, 3072, 0, 1, True)])
def test_gemm_ln_pending_fold_bits(gpu, M, nparts, N, act, mode, xf):
    """A pending residual update (partial rows: the fused attention's eight heads, the few-row
    kernel's four K shares) applied by the LayerNorm-fused GEMM that reads the residual next
    (nk_gemm_ln_pend: inside the prologue of the GEMV for M <= 4 and of the few-row kernel for
    M <= 16 with at most four parts; a copy and nk_resid_fold first otherwise) gives, bit for bit,
    the updated residual (when asked for) and the outputs of nk_resid_fold followed by nk_gemm_ln;
    the input rows are left as they were."""
    import ctypes as C

    import nemoasr

    L = nemoasr.lib()
    K = 1024
    rng = np.random.default_rng([M, nparts, N, 31])
    X = rng.standard_normal((M, K)).astype(np.float32)
    P = (0.3 * rng.standard_normal((max(nparts, 1), M, K))).astype(np.float32)
    W = w_bf16(rng, N, K)
    g1, g2 = [(1 + 0.1 * rng.standard_normal(K)).astype(np.float32) for _ in range(2)]
    b1, b2 = [(0.1 * rng.standard_normal(K)).astype(np.float32) for _ in range(2)]
    nout = N // 2 if act == 3 else N
    dW, dP, dg1, db1, dg2, db2 = (gpu.put(a) for a in (W, P, g1, b1, g2, b2))
    tmp = gpu.alloc(M * K * 4)
    pend = nemoasr.Resid(dP.ptr, nparts, 0.75)
    ln2 = (dg2.ptr, db2.ptr) if mode == 2 else (None, None)
    outs = []
    for fused in (False, True):
        dX, dXf, dC, dL1 = gpu.put(X), gpu.alloc(M * K * 4), gpu.alloc(M * nout * 4), gpu.alloc(M * K * 4)
        gpu.begin()
        if fused:
            gpu.check(L.nk_gemm_ln_pend(gpu.h, dX.ptr, K, dW.ptr, K, None, dC.ptr, nout, None, M, N, K, act, 0, 1.0,
                                        mode, dg1.ptr, db1.ptr, *ln2, dL1.ptr if mode == 2 else None, tmp.ptr, 1e-5,
                                        C.byref(pend), dXf.ptr if xf else None))
        else:
            gpu.check(L.nk_copy(gpu.h, dX.ptr, dXf.ptr, M * K))
            gpu.check(L.nk_resid_fold(gpu.h, dXf.ptr, K, M, K, C.byref(pend)))
            gpu.check(L.nk_gemm_ln(gpu.h, dXf.ptr, K, dW.ptr, K, None, dC.ptr, nout, None, M, N, K, act, 0, 1.0, mode,
                                   dg1.ptr, db1.ptr, *ln2, dL1.ptr if mode == 2 else None, tmp.ptr, 1e-5))
        gpu.end()
        outs.append((dX.read((M, K)), dXf.read((M, K)), dC.read((M, nout)), dL1.read((M, K)) if mode == 2 else None))
    (x0, xf0, c0, l0), (x1, xf1, c1, l1) = outs
    assert np.array_equal(bits(x1), bits(X))
    assert np.array_equal(bits(c1), bits(c0))
    if mode == 2:
        assert np.array_equal(bits(l1), bits(l0))
    ref = X + np.float32(0.75) * P[:nparts].sum(axis=0, dtype=np.float64).astype(np.float32)
    assert rel_err(xf0, ref) < 1e-6
    if xf:
        assert np.array_equal(bits(xf1), bits(xf0))
    else:
        assert not np.any(xf1)


@pytest.mark.parametrize("M,N,K", [(7, 1024, 4096), (14, 1024, 1024), (16, 1024, 4096), (1, 1024, 4096),
                                   (3, 1024, 4096)])
def test_gemm_pend_then_fold_bits(gpu, M, N, K):
    """A few-row residual update left pending (nk_gemm_pend: the few-row kernel's K shares, C
    untouched) and applied by the next LayerNorm-fused GEMM gives, bit for bit, what the update
    applied at once (nk_gemm with accumulate) followed by nk_gemm_ln gives; a kernel that does not
    split K updates C itself and leaves nothing pending."""
    import ctypes as C

    import nemoasr

    L = nemoasr.lib()
    D, NQ = 1024, 3072
    rng = np.random.default_rng([M, N, K, 5])
    A = rng.standard_normal((M, K)).astype(np.float32)
    X = rng.standard_normal((M, N)).astype(np.float32)
    W = w_bf16(rng, N, K)
    Wq = w_bf16(rng, NQ, D)
    g1 = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(D)).astype(np.float32)
    dA, dW, dWq, dg1, db1 = (gpu.put(a) for a in (A, W, Wq, g1, b1))
    tmp = gpu.alloc(M * D * 4)
    outs = []
    for pending in (False, True):
        dX, dXf, dQ = gpu.put(X), gpu.alloc(M * D * 4), gpu.alloc(M * NQ * 4)
        pend = nemoasr.Resid()
        gpu.begin()
        if pending:
            gpu.check(L.nk_gemm_pend(gpu.h, dA.ptr, K, dW.ptr, K, dX.ptr, N, M, N, K, 0.5, C.byref(pend)))
            xf = dXf.ptr if pend.nparts else None
            gpu.check(L.nk_gemm_ln_pend(gpu.h, dX.ptr, D, dWq.ptr, D, None, dQ.ptr, NQ, None, M, NQ, D, 0, 0, 1.0, 1,
                                        dg1.ptr, db1.ptr, None, None, None, tmp.ptr, 1e-5, C.byref(pend), xf))
        else:
            gpu.check(L.nk_gemm(gpu.h, dA.ptr, K, dW.ptr, K, None, dX.ptr, N, M, N, K, 0, 1, 0.5))
            gpu.check(L.nk_gemm_ln(gpu.h, dX.ptr, D, dWq.ptr, D, None, dQ.ptr, NQ, None, M, NQ, D, 0, 0, 1.0, 1,
                                   dg1.ptr, db1.ptr, None, None, None, tmp.ptr, 1e-5))
        gpu.end()
        res = (dXf if pending and pend.nparts else dX).read((M, D))
        outs.append((res, dQ.read((M, NQ)), pend.nparts, dX.read((M, D))))
    (r0, q0, _, _), (r1, q1, nparts, x1) = outs
    assert np.array_equal(bits(r1), bits(r0))
    assert np.array_equal(bits(q1), bits(q0))
    if nparts:
        assert nparts == 4
        assert np.array_equal(bits(x1), bits(X))
    ref = oracle.gemm(A, W, None, 0, True, 0.5, C0=X)
    assert rel_err(r1, ref) < 2e-5
