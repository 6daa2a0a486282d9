"""Pins the oracle's kernel restatements (oracle/oracle_kernels.c) against independent references:
numpy float64 GEMMs, torch CPU conv2d / LSTMCell, closed forms and special cases chosen so that a
dropped term, a wrong sign or index, or a transposed operand fails.  CPU only."""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err


def bf16(x):
    return oracle.f32_to_bf16(np.asarray(x, np.float32))


def wide(u):
    return oracle.bf16_to_f32(u).astype(np.float64)


def np_act(v, act):
    if act == 1:
        return v / (1.0 + np.exp(-v))
    if act == 2:
        return np.maximum(v, 0.0)
    return v


@pytest.mark.parametrize("M,N,K", [(1, 8, 16), (3, 40, 64), (7, 96, 256), (16, 64, 1024), (33, 17, 40)])
@pytest.mark.parametrize("act", [0, 1, 2])
def test_gemm_matches_float64(M, N, K, act):
    rng = np.random.default_rng([M, N, K, act])
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = bf16(rng.standard_normal((N, K)) / np.sqrt(K))
    b = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    ref = C0.astype(np.float64) + 0.75 * np_act(A.astype(np.float64) @ wide(W).T + b, act)
    got = oracle.gemm(A, W, b, act, True, 0.75, C0=C0)
    assert rel_err(got, ref) < 1e-5


def test_gemm_glu_pairs_halves():
    rng = np.random.default_rng(1)
    M, N, K = 5, 64, 128
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = bf16(rng.standard_normal((N, K)) / np.sqrt(K))
    b = rng.standard_normal(N).astype(np.float32)
    z = A.astype(np.float64) @ wide(W).T + b
    ref = z[:, : N // 2] / (1.0 + np.exp(-z[:, N // 2:])) * 2.0
    got = oracle.gemm(A, W, b, 3, False, 2.0)
    assert got.shape == (M, N // 2)
    assert rel_err(got, ref) < 1e-5


def test_gemm_identity_weights_and_row_stride():
    """W = I (bf16 1.0 = 0x3F80): C = A + b exactly; a row stride larger than K reads the first K."""
    K = 32
    W = np.zeros((K, K + 8), np.uint16)
    W[np.arange(K), np.arange(K)] = 0x3F80
    A = np.arange(3 * K, dtype=np.float32).reshape(3, K) / 7
    b = np.linspace(-1, 1, K).astype(np.float32)
    got = oracle.gemm(A, W, b, 0, False, 1.0, ldw=K + 8, K=K)
    np.testing.assert_array_equal(got, A + b)


def test_layernorm_closed_forms():
    rng = np.random.default_rng(2)
    D = 256
    g = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    b = (0.3 * rng.standard_normal(D)).astype(np.float32)
    X = (3 * rng.standard_normal((4, D)) + 2).astype(np.float32)
    x = X.astype(np.float64)
    mu = x.mean(1, keepdims=True)
    ref = (x - mu) / np.sqrt(((x - mu) ** 2).mean(1, keepdims=True) + 1e-5) * g + b
    assert rel_err(oracle.layernorm(X, g, b), ref) < 1e-5
    const = np.full((2, D), 3.25, np.float32)  # zero variance: output is beta
    np.testing.assert_array_equal(oracle.layernorm(const, g, b), np.broadcast_to(b, (2, D)))
    g2 = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(D)).astype(np.float32)
    y1, y2 = oracle.layernorm2(X, g, b, g2, b2)
    np.testing.assert_array_equal(y1, oracle.layernorm(X, g, b))
    np.testing.assert_array_equal(y2, oracle.layernorm(y1, g2, b2))


def naive_attention(q, K, V, P, u, v, c, cache, Lmax, H, dh):
    """Float64 rel-pos attention built from absolute positions: query i sits at position cache+i,
    key j at position j; the table row for relative distance d is (Lmax-1) - d."""
    L = cache + c
    out = np.zeros((c, H * dh))
    for h in range(H):
        sl = slice(h * dh, (h + 1) * dh)
        for i in range(c):
            dist = (cache + i) - np.arange(L)
            rows = (Lmax - 1) - dist
            s = (K[:, sl] @ (q[i, sl] + u[sl]) + P[rows][:, sl] @ (q[i, sl] + v[sl])) / np.sqrt(dh)
            p = np.exp(s - s.max())
            out[i, sl] = (p / p.sum()) @ V[:, sl]
    return out


@pytest.mark.parametrize("c,cache", [(1, 0), (1, 56), (7, 56), (14, 10), (16, 56)])
def test_attention_rel_naive(c, cache):
    H, dh, Lmax = 2, 128, 72
    D = H * dh
    rng = np.random.default_rng([c, cache])
    L = cache + c
    q = rng.standard_normal((c, D)).astype(np.float32)
    K = rng.standard_normal((L, D)).astype(np.float32)
    V = rng.standard_normal((L, D)).astype(np.float32)
    P = rng.standard_normal((2 * Lmax - 1, D)).astype(np.float32)
    u = (0.2 * rng.standard_normal(D)).astype(np.float32)
    v = (0.2 * rng.standard_normal(D)).astype(np.float32)
    ref = naive_attention(q.astype(np.float64), K.astype(np.float64), V.astype(np.float64), P.astype(np.float64),
                          u.astype(np.float64), v.astype(np.float64), c, cache, Lmax, H, dh)
    got = oracle.attention_rel(q, K, V, P, u, v, c, L, Lmax, H, dh)
    assert rel_err(got, ref) < 1e-5


def test_attention_special_cases():
    H, dh, Lmax = 1, 128, 72
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, dh)).astype(np.float32)
    V = rng.standard_normal((1, dh)).astype(np.float32)
    K = rng.standard_normal((1, dh)).astype(np.float32)
    P = rng.standard_normal((2 * Lmax - 1, dh)).astype(np.float32)
    z = np.zeros(dh, np.float32)
    # one key: softmax is 1, the output is that value row
    np.testing.assert_allclose(oracle.attention_rel(q, K, V, P, z, z, 1, 1, Lmax, H, dh), V, rtol=0, atol=1e-6)
    # no position term and no biases: plain scaled-dot-product attention
    L = 9
    q = rng.standard_normal((3, dh)).astype(np.float32)
    K = rng.standard_normal((L, dh)).astype(np.float32)
    V = rng.standard_normal((L, dh)).astype(np.float32)
    ref = torch.softmax(torch.tensor(q, dtype=torch.float64) @ torch.tensor(K, dtype=torch.float64).T / np.sqrt(dh),
                        dim=1) @ torch.tensor(V, dtype=torch.float64)
    got = oracle.attention_rel(q, K, V, np.zeros_like(P), z, z, 3, L, Lmax, H, dh)
    assert rel_err(got, ref.numpy()) < 1e-5


def test_position_table_closed_form():
    D, Lmax = 64, 20
    rng = np.random.default_rng(6)
    W = bf16(rng.standard_normal((D, D)) / np.sqrt(D))
    pos = (Lmax - 1 - np.arange(2 * Lmax - 1))[:, None].astype(np.float64)
    div = np.exp(np.arange(0, D, 2) * -(np.log(10000.0) / D))
    pe = np.zeros((2 * Lmax - 1, D))
    pe[:, 0::2] = np.sin(pos * div)
    pe[:, 1::2] = np.cos(pos * div)
    ref = pe.astype(np.float32).astype(np.float64) @ wide(W).T
    got = oracle.ptab(W, D, Lmax)
    assert rel_err(got, ref) < 1e-5
    # the centre row is position 0: sin(0) = 0, cos(0) = 1
    eye = np.zeros((D, D), np.uint16)
    eye[np.arange(D), np.arange(D)] = 0x3F80  # bf16 1.0
    centre = oracle.ptab(eye, D, Lmax)[Lmax - 1]
    np.testing.assert_array_equal(centre, np.tile(np.float32([0.0, 1.0]), D // 2))


@pytest.mark.parametrize("c", [1, 4, 14])
def test_dwconv_ln_silu(c):
    D, taps = 64, 9
    rng = np.random.default_rng(c)
    din = rng.standard_normal((taps - 1 + c, D)).astype(np.float32)
    W = rng.standard_normal((D, taps)).astype(np.float32) / 3
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b = (0.1 * rng.standard_normal(D)).astype(np.float32)
    conv = np.stack([np.correlate(din[:, ch].astype(np.float64), W[ch].astype(np.float64), "valid") for ch in range(D)], 1)
    mu = conv.mean(1, keepdims=True)
    y = (conv - mu) / np.sqrt(((conv - mu) ** 2).mean(1, keepdims=True) + 1e-5) * g + b
    ref = y / (1 + np.exp(-y))
    assert rel_err(oracle.dwconv_ln_silu(din, W, g, b, c), ref) < 1e-5


def test_dwconv_impulse_recovers_taps():
    """A unit impulse in the history at row r gives conv output W[:, 8 - r + t] at output t:
    the causal taps are applied oldest-first (checked before the LayerNorm on one channel pair)."""
    D, taps = 4, 9
    W = np.arange(D * taps, dtype=np.float32).reshape(D, taps) / 10
    din = np.zeros((taps, D), np.float32)
    din[3] = 1.0  # impulse 5 rows before the output row
    g = np.ones(D, np.float32)
    b = np.zeros(D, np.float32)
    y = oracle.dwconv_ln_silu(din, W, g, b, 1)[0]
    conv = W[:, 3].astype(np.float64)  # output row 0 reads din rows 0..8 with taps 0..8
    mu = conv.mean()
    z = (conv - mu) / np.sqrt(((conv - mu) ** 2).mean() + 1e-5)
    np.testing.assert_allclose(y, z / (1 + np.exp(-z)), rtol=1e-5)


def torch_causal_conv(x, w, b, groups):
    """3x3 stride 2 with 2 rows/cols of padding before and 1 after (time and frequency)."""
    xp = torch.nn.functional.pad(x, (2, 1, 2, 1))
    return torch.nn.functional.conv2d(xp, w, b, stride=2, groups=groups)


@pytest.mark.parametrize("T", [8, 24, 33, 72])
def test_subsampling_convs_vs_torch(T):
    rng = np.random.default_rng(T)
    F, C = 128, 16
    X = rng.standard_normal((T, F)).astype(np.float32)
    W0 = rng.standard_normal((C, 9)).astype(np.float32) / 3
    b0 = rng.standard_normal(C).astype(np.float32)
    W2 = rng.standard_normal((C, 9)).astype(np.float32) / 3
    b2 = rng.standard_normal(C).astype(np.float32)
    y0 = oracle.conv2d_c1_s2_relu(X, W0, b0)
    t0 = torch.relu(torch_causal_conv(torch.tensor(X, dtype=torch.float64)[None, None],
                                      torch.tensor(W0, dtype=torch.float64).reshape(C, 1, 3, 3),
                                      torch.tensor(b0, dtype=torch.float64), 1))[0]  # [C][T1][F1]
    assert y0.shape == (t0.shape[1], t0.shape[2], C)
    assert rel_err(y0, t0.permute(1, 2, 0).numpy()) < 1e-5
    y1 = oracle.dwconv2d_s2(y0, W2, b2)
    t1 = torch_causal_conv(t0[None], torch.tensor(W2, dtype=torch.float64).reshape(C, 1, 3, 3),
                           torch.tensor(b2, dtype=torch.float64), C)[0]
    assert rel_err(y1, t1.permute(1, 2, 0).numpy()) < 1e-5
    # channel-major flatten, as torch's x.transpose(1, 2).reshape(b, t, c * f) of a [b][c][t][f] map
    flat = oracle.flatten_cf(y1)
    ref = torch.tensor(y1).permute(2, 0, 1)[None].transpose(1, 2).reshape(1, y1.shape[0], -1)[0].numpy()
    np.testing.assert_array_equal(flat, ref)


def test_lstm_matches_torch_lstmcell():
    """Wx x + b + Wh h, gate order i, f, g, o and the cell update equal torch.nn.LSTMCell with
    bias_ih = b and bias_hh = 0 (one fused bias)."""
    H = 48
    rng = np.random.default_rng(8)
    Wx = bf16(rng.standard_normal((4 * H, H)) / np.sqrt(H))
    Wh = bf16(rng.standard_normal((4 * H, H)) / np.sqrt(H))
    b = (0.3 * rng.standard_normal(4 * H)).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    h = rng.standard_normal(H).astype(np.float32)
    c = rng.standard_normal(H).astype(np.float32)
    gates = oracle.gemm(x[None], Wx, b, 0, False, 1.0)
    gates = oracle.gemm(h[None], Wh, None, 0, True, 1.0, C0=gates)[0]
    c1, h1 = oracle.lstm_cell(gates, c)
    cell = torch.nn.LSTMCell(H, H).double()
    with torch.no_grad():
        cell.weight_ih.copy_(torch.tensor(wide(Wx)))
        cell.weight_hh.copy_(torch.tensor(wide(Wh)))
        cell.bias_ih.copy_(torch.tensor(b, dtype=torch.float64))
        cell.bias_hh.zero_()
        th, tc = cell(torch.tensor(x, dtype=torch.float64)[None], (torch.tensor(h, dtype=torch.float64)[None],
                                                                    torch.tensor(c, dtype=torch.float64)[None]))
    assert rel_err(h1, th[0].numpy()) < 1e-5
    assert rel_err(c1, tc[0].numpy()) < 1e-5


def test_joint_argmax_and_ties():
    rng = np.random.default_rng(9)
    V, H = 97, 64
    W = bf16(rng.standard_normal((V, H)) / np.sqrt(H))
    b = rng.standard_normal(V).astype(np.float32)
    enc = rng.standard_normal(H).astype(np.float32)
    pred = rng.standard_normal(H).astype(np.float32)
    i, v, logits = oracle.joint_argmax(enc, pred, W, b)
    ref = wide(W) @ np.maximum(enc.astype(np.float64) + pred, 0) + b
    assert rel_err(logits, ref) < 1e-5
    assert i == int(np.argmax(logits)) and v == logits[i]
    b2 = np.zeros(V, np.float32)
    b2[[5, 40, 90]] = 2.0
    i2, _, _ = oracle.joint_argmax(enc, pred, np.zeros((V, H), np.uint16), b2)
    assert i2 == 5  # equal scores: lowest index wins
