"""Committed golden fixtures (tests/golden/kernels.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture bit for bit (so the restatement cannot drift unnoticed).
GPU: the HIP kernels reproduce the fixtures through the kernel C ABI, to the same tolerances as the
per-kernel parity tests (index outputs exact).
"""
import os

import numpy as np
import pytest

import oracle
from conftest import rel_err

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kernels.npz")


@pytest.fixture(scope="module")
def gold():
    z = np.load(GOLD)
    return {k: z[k] for k in z.files}


def case(g, name):
    return {k.split("/", 1)[1]: v for k, v in g.items() if k.startswith(name + "/")}


# ---- CPU: the oracle reproduces the fixtures ---------------------------------------------------
def test_oracle_gemm(gold):
    for act in range(4):
        c = case(gold, f"gemm_act{act}")
        Y = oracle.gemm(c["A"], c["W"], c["bias"], int(c["act"]), bool(c["acc"]), float(c["alpha"]),
                        C0=c["C0"] if c["acc"] else None)
        np.testing.assert_array_equal(Y, c["Y"])
    c = case(gold, "gemm_ldw")
    np.testing.assert_array_equal(oracle.gemm(c["A"], c["W"], None, 2, False, 1.0, ldw=112, K=int(c["K"])), c["Y"])


def test_oracle_norms(gold):
    c = case(gold, "layernorm")
    np.testing.assert_array_equal(oracle.layernorm(c["X"], c["g"], c["b"]), c["Y"])
    c = case(gold, "layernorm2")
    y1, y2 = oracle.layernorm2(c["X"], c["g1"], c["b1"], c["g2"], c["b2"])
    np.testing.assert_array_equal(y1, c["Y1"])
    np.testing.assert_array_equal(y2, c["Y2"])


def test_oracle_attention(gold):
    c = case(gold, "attention")
    H, dh, n, L, Lmax = (int(c[k]) for k in ("H", "dh", "c", "L", "Lmax"))
    D = H * dh
    kv = c["kv"]
    O = oracle.attention_rel(kv[L - n:], kv[:, D:2 * D].copy(), kv[:, 2 * D:].copy(), c["P"], c["bu"], c["bv"], n, L, Lmax, H, dh)
    np.testing.assert_array_equal(O, c["O"])


def test_oracle_convs(gold):
    c = case(gold, "dwconv")
    np.testing.assert_array_equal(oracle.dwconv_ln_silu(c["din"], c["W"], c["g"], c["b"], int(c["c"])), c["Y"])
    c = case(gold, "subsampling")
    Y0 = oracle.conv2d_c1_s2_relu(c["X"], c["W0"], c["b0"])
    np.testing.assert_array_equal(Y0, c["Y0"])
    Yd = oracle.dwconv2d_s2(Y0, c["Wd"], c["bd"])
    np.testing.assert_array_equal(Yd, c["Yd"])
    np.testing.assert_array_equal(oracle.flatten_cf(Yd), c["flat"])


def test_oracle_decoder_kernels(gold):
    c = case(gold, "lstm")
    co, ho = oracle.lstm_cell(c["gates"], c["c_in"])
    np.testing.assert_array_equal(co, c["c_out"])
    np.testing.assert_array_equal(ho, c["h_out"])
    for name in ("joint", "joint_tie"):
        c = case(gold, name)
        i, v, _ = oracle.joint_argmax(c["enc"], c["pred"], c["W"], c["bias"])
        assert i == int(c["idx"]) and np.float32(v) == c["val"]
    assert int(case(gold, "joint_tie")["idx"]) == 5  # exact tie: lowest index
    c = case(gold, "ptab")
    np.testing.assert_array_equal(oracle.ptab(c["W"], int(c["D"]), int(c["Lmax"])), c["P"])


# ---- GPU: the HIP kernels reproduce the fixtures ------------------------------------------------
@pytest.mark.gpu
def test_gpu_golden_gemm(gpu, gold):
    from test_gpu_kernels import GEMM_TOL, run_gemm

    for act in range(4):
        c = case(gold, f"gemm_act{act}")
        for kind in (0, 1):
            Y = run_gemm(gpu, c["A"], c["W"], c["bias"], int(c["act"]), int(c["acc"]), float(c["alpha"]),
                         C0=c["C0"].copy() if c["acc"] else None, kind=kind)
            assert rel_err(Y, c["Y"]) < GEMM_TOL, (act, kind)
    c = case(gold, "gemm_ldw")
    Y = run_gemm(gpu, c["A"], c["W"], None, 2, 0, 1.0, ldw=112, K=int(c["K"]))
    assert rel_err(Y, c["Y"]) < GEMM_TOL


@pytest.mark.gpu
def test_gpu_golden_layernorm(gpu, gold):
    import nemoasr

    L = nemoasr.lib()
    c = case(gold, "layernorm2")
    X = c["X"]
    M, D = X.shape
    dX, dY1, dY2 = gpu.put(X), gpu.alloc(X.nbytes), gpu.alloc(X.nbytes)
    ps = [gpu.put(c[k]) for k in ("g1", "b1", "g2", "b2")]
    gpu.begin()
    gpu.check(L.nk_layernorm2(gpu.h, dX.ptr, *(p.ptr for p in ps), dY1.ptr, dY2.ptr, M, D, 1e-5))
    gpu.end()
    assert rel_err(dY1.read((M, D)), c["Y1"]) < 1e-5
    assert rel_err(dY2.read((M, D)), c["Y2"]) < 1e-5


@pytest.mark.gpu
def test_gpu_golden_dwconv(gpu, gold):
    import nemoasr

    L = nemoasr.lib()
    c = case(gold, "dwconv")
    n, D = int(c["c"]), c["din"].shape[1]
    dd, dW, dg, db, dY = gpu.put(c["din"]), gpu.put(c["W"]), gpu.put(c["g"]), gpu.put(c["b"]), gpu.alloc(n * D * 4)
    gpu.begin()
    gpu.check(L.nk_dwconv_ln_silu(gpu.h, dd.ptr, dW.ptr, dg.ptr, db.ptr, dY.ptr, n, D, 9, 1e-5))
    gpu.end()
    assert rel_err(dY.read((n, D)), c["Y"]) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("device_loop", [True, False])
def test_gpu_golden_decoder_kernels(gpu, gold, device_loop):
    """The LSTM cell and the joint argmax kernels the batched greedy loop launches (the device loop's
    argmax-key GEMM, or logits + argmax_rows in the host loop), on the golden cases, including the
    planted exact tie (lowest index wins)."""
    from conftest import joint_argmax_rows, lstm_cell_rows

    c = case(gold, "lstm")
    co, ho = lstm_cell_rows(gpu, c["gates"], c["c_in"])
    assert rel_err(co, c["c_out"]) < 1e-6
    assert rel_err(ho, c["h_out"]) < 1e-6
    for name in ("joint", "joint_tie"):
        c = case(gold, name)
        (idx, val), = joint_argmax_rows(gpu, c["enc"][None], c["pred"], c["W"], c["bias"], device_loop)
        assert idx == int(c["idx"]), name
        assert abs(val - float(c["val"])) <= 1e-5 * max(1.0, abs(float(c["val"]))), name
