"""The reference's GPU runtime interface (include/nemo_gpu.h: src/gpu.h:7-41) and parameter blocks
(include/nemo_kernel_params.h: src/kernel_params.h:22-32), driven the way the reference's host
drives them: buffers filled and read through gpu_buf_ptr, arguments bound by index with GPU_BUF /
GPU_BYTES, kernels named as in src/kernels.metal, dispatched by total threads, by groups and by
groups with function constants.  Each sequence below replays the reference's own dispatch sites
with their parameters (src/model.c:70-122 launchers, src/encoder.c:120-188 for one conformer block
and the subsampling, src/decoder.c:57-90 for one prediction update and joint round) and is checked
against the oracle."""
import ctypes as C

import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu

_u = C.c_uint32


def _params(name, fields):
    return type(name, (C.Structure,), {"_fields_": [(f, C.c_float if f in ("alpha", "eps", "scale", "value") else _u)
                                                    for f in fields]})


GemmParams = _params("GemmParams", "M N K lda ldw ldc has_bias act accumulate alpha".split())
LnParams = _params("LnParams", "M D eps".split())
AttnParams = _params("AttnParams", "c L Lmax H dh D ldq ldk scale".split())
GluParams = _params("GluParams", "M D".split())
DwParams = _params("DwParams", "c D taps eps".split())
Conv2dParams = _params("Conv2dParams", "T F T1 F1 C".split())
FlatParams = _params("FlatParams", "T F C".split())
CountParams = _params("CountParams", "n".split())
FillParams = _params("FillParams", "n value".split())
LstmParams = _params("LstmParams", "H".split())
JointParams = _params("JointParams", "V H enc_row enc_ld".split())
JOINT_GROUPS, GEMM_SIMDS, LN_THREADS, ATT_DH, GEMM_ROWS = 64, 8, 256, 128, 16


class RefHost:
    """The reference host's view of the GPU: gpu_t, buffers with host pointers, dispatch by name."""

    def __init__(self, gpu):
        import nemoasr

        self.L = nemoasr.lib()
        self.nemoasr = nemoasr
        self.g = gpu.h
        self.bufs = []

    def alloc(self, nbytes):
        b = self.L.gpu_buf_alloc(self.g, nbytes)
        assert b
        self.bufs.append(b)
        return b

    def ptr(self, b, dtype, count):
        p = self.L.gpu_buf_ptr(b)
        assert p, self.L.gpu_last_error(self.g).decode()
        return np.ctypeslib.as_array((C.c_char * (count * np.dtype(dtype).itemsize)).from_address(p)).view(dtype)

    def put(self, a):
        a = np.ascontiguousarray(a)
        b = self.alloc(max(a.nbytes, 16))
        self.ptr(b, a.dtype, a.size)[:] = a.reshape(-1)
        return b

    def get(self, b, dtype, shape, byte_off=0):
        n = int(np.prod(shape))
        return self.ptr(b, dtype, (byte_off // np.dtype(dtype).itemsize) + n)[byte_off // np.dtype(dtype).itemsize:].reshape(shape).copy()

    def begin(self):
        assert self.L.gpu_begin(self.g) == 0

    def end(self):
        err = C.create_string_buffer(512)
        rc = self.L.gpu_end(self.g, err, 512)
        assert rc == 0, err.value.decode()

    def dispatch(self, kernel, items, grid, block, groups=False, fc=None):
        arr, keep = self.nemoasr.gpu_args(*items)
        if fc is not None:
            fca = (_u * len(fc))(*fc)
            rc = self.L.gpu_dispatch_groups_fc(self.g, kernel.encode(), fca, len(fc), arr, len(items), *grid, *block)
        elif groups:
            rc = self.L.gpu_dispatch_groups(self.g, kernel.encode(), arr, len(items), *grid, *block)
        else:
            rc = self.L.gpu_dispatch(self.g, kernel.encode(), arr, len(items), *grid, *block)
        assert rc == 0, self.L.gpu_last_error(self.g).decode()
        del keep

    # src/model.c:70-99: the reference's k_gemm, with its kernel choice, function constants and grid
    def k_gemm(self, A, a_off, lda, W, w_off, ldw, bias, Cb, c_off, ldc, M, N, K, act, acc, alpha):
        p = GemmParams(M, N, K, lda, ldw, ldc, int(bias is not None), act, int(acc), alpha)
        items = [(A, a_off), (W, w_off), (bias if bias is not None else A, 0), (Cb, c_off), p]
        nout = N // 2 if act == 3 else N
        if M <= 4 or (M <= GEMM_ROWS and K % 256):
            cpt = GEMM_SIMDS if act == 3 else GEMM_SIMDS * 2
            self.dispatch("gemm_spec", items, ((nout + cpt - 1) // cpt, 1, 1), (GEMM_SIMDS * 32, 1, 1), fc=[M, 2, 2])
        elif K % 256 == 0:
            tm = 2 if M > 8 else 1
            cpt = 8 if act == 3 else 16
            self.dispatch("gemm_mma", items, ((nout + cpt - 1) // cpt, (M + 8 * tm - 1) // (8 * tm), 1), (32 * 8, 1, 1),
                          fc=[M, 0, 0, tm, 2, 8, 32])
        else:
            self.dispatch("gemm_bf16", items, ((N + GEMM_SIMDS - 1) // GEMM_SIMDS, 1, 1), (GEMM_SIMDS * 32, 1, 1),
                          groups=True)

    def k_layernorm(self, X, x_off, g, b, Y, y_off, M, D, eps=1e-5):  # src/model.c:106-111
        self.dispatch("layernorm", [(X, x_off), (g, 0), (b, 0), (Y, y_off), LnParams(M, D, eps)], (M, 1, 1),
                      (LN_THREADS, 1, 1), groups=True)

    def k_layernorm2(self, X, g1, b1, g2, b2, Y1, Y2, M, D, eps=1e-5):  # src/model.c:100-105
        self.dispatch("layernorm2", [(X, 0), (g1, 0), (b1, 0), (g2, 0), (b2, 0), (Y1, 0), (Y2, 0), LnParams(M, D, eps)],
                      (M, 1, 1), (LN_THREADS, 1, 1), groups=True)

    def close(self):
        for b in self.bufs:
            self.L.gpu_buf_free(b)
        self.bufs = []


@pytest.fixture
def host(gpu):
    h = RefHost(gpu)
    yield h
    h.close()


def _w(rng, n, k):
    return oracle.f32_to_bf16((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))


def test_buffer_host_pointer_and_copy_fill(host):
    """gpu_buf_ptr: host writes before a batch reach the kernels, kernel results are read through
    the pointer after gpu_end, twice in a row (src/model.c:112-122 launchers, dispatch by threads)."""
    n = 1000
    src = host.alloc(4 * n)
    dst, fil = host.alloc(4 * n), host.alloc(4 * n)
    for rnd in range(2):
        x = np.arange(n, dtype=np.float32) * (rnd + 1)
        host.ptr(src, np.float32, n)[:] = x
        host.begin()
        host.dispatch("copy_f32", [(src, 0), (dst, 0), CountParams(n)], (n, 1, 1), (256, 1, 1))
        host.dispatch("fill_f32", [(fil, 40), FillParams(n - 10, 2.5 + rnd)], (n - 10, 1, 1), (256, 1, 1))
        host.end()
        assert np.array_equal(host.get(dst, np.float32, (n,)), x)
        f = host.get(fil, np.float32, (n,))
        assert np.all(f[10:] == 2.5 + rnd) and (rnd or np.all(f[:10] == 0))


def test_conformer_block_reference_sequence(host):
    """One conformer block at 560 ms (c = 7 rows) with 20 cached frames, dispatched exactly as
    src/encoder.c:150-188 does (LayerNorm dispatches, k_gemm's kernel choice, attention_rel with its
    K/V offsets into the cache, the GLU written into the conv history, dwconv_ln_silu reading 8 rows
    of history, the paired LayerNorm with the next block's FF1 norm), weights at byte offsets in one
    arena; the block's outputs, the cache rows and the conv history rows against the oracle."""
    rng = np.random.default_rng(152)
    D, FF, H, dh, Lmax, taps, c, cache = 1024, 4096, 8, 128, 72, 9, 7, 20
    conv_left = taps - 1
    pos = conv_left + cache                       # rows [0, 8) the empty conv history, then the cache
    L = cache + c
    cap = pos + c + 4
    mats = {"ff1_w1": _w(rng, FF, D), "ff1_w2": _w(rng, D, FF), "wqkv": _w(rng, 3 * D, D), "wo": _w(rng, D, D),
            "pw1": _w(rng, 2 * D, D), "pw2": _w(rng, D, D), "ff2_w1": _w(rng, FF, D), "ff2_w2": _w(rng, D, FF)}
    arena, offs, off = [], {}, 0
    for k, m in mats.items():
        offs[k] = off
        arena.append(m.reshape(-1))
        off += m.size * 2
        pad = (-off) % 4096
        arena.append(np.zeros(pad // 2, np.uint16))
        off += pad
    Wb = host.put(np.concatenate(arena))
    vec = lambda s=0.1, m=0.0: (m + s * rng.standard_normal(D)).astype(np.float32)
    ln = {k: (vec(0.1, 1.0), vec(0.05)) for k in ("ff1", "att", "conv", "ff2", "out", "ff1_next")}
    lnb = {k: (host.put(g), host.put(b)) for k, (g, b) in ln.items()}
    P = (0.5 * rng.standard_normal((2 * Lmax - 1, D))).astype(np.float32)
    bu, bv = vec(0.1), vec(0.1)
    dw = (rng.standard_normal((D, taps)) / 3).astype(np.float32)
    bn_g, bn_b = vec(0.1, 1.0), vec(0.05)
    h0 = rng.standard_normal((c, D)).astype(np.float32)
    kv0 = np.zeros((cap, 3 * D), np.float32)
    kv0[conv_left:pos] = rng.standard_normal((cache, 3 * D)).astype(np.float32)
    din0 = np.zeros((cap, D), np.float32)
    din0[conv_left:pos] = rng.standard_normal((cache, D)).astype(np.float32)

    h, t, t2 = host.put(h0), host.alloc(c * D * 4), host.alloc(c * D * 4)
    ff, att, y = host.alloc(c * FF * 4), host.alloc(c * D * 4), host.alloc(c * D * 4)
    kvb, dinb = host.put(kv0), host.put(din0)
    Pb, bub, bvb, dwb, bngb, bnbb = (host.put(a) for a in (P, bu, bv, dw, bn_g, bn_b))
    rowb, kvrowb = D * 4, 3 * D * 4
    host.begin()
    host.k_layernorm(h, 0, *lnb["ff1"], t2, 0, c, D)
    host.k_gemm(t2, 0, D, Wb, offs["ff1_w1"], D, None, ff, 0, FF, c, FF, D, 1, 0, 1.0)
    host.k_gemm(ff, 0, FF, Wb, offs["ff1_w2"], FF, None, h, 0, D, c, D, FF, 0, 1, 0.5)
    host.k_layernorm(h, 0, *lnb["att"], t, 0, c, D)
    host.k_gemm(t, 0, D, Wb, offs["wqkv"], D, None, kvb, pos * kvrowb, 3 * D, c, 3 * D, D, 0, 0, 1.0)
    kv_start = (pos - cache) * kvrowb
    ap = AttnParams(c, L, Lmax, H, dh, D, 3 * D, 3 * D, float(np.float32(1.0) / np.sqrt(np.float32(dh))))
    host.dispatch("attention_rel", [(kvb, pos * kvrowb), (kvb, kv_start + rowb), (kvb, kv_start + 2 * rowb), (Pb, 0),
                                    (bub, 0), (bvb, 0), (att, 0), ap], (H, c, 1), (ATT_DH, 1, 1), groups=True)
    host.k_gemm(att, 0, D, Wb, offs["wo"], D, None, h, 0, D, c, D, D, 0, 1, 1.0)
    host.k_layernorm(h, 0, *lnb["conv"], t, 0, c, D)
    host.k_gemm(t, 0, D, Wb, offs["pw1"], D, None, dinb, pos * rowb, D, c, 2 * D, D, 3, 0, 1.0)
    host.dispatch("dwconv_ln_silu", [(dinb, (pos - conv_left) * rowb), (dwb, 0), (bngb, 0), (bnbb, 0), (y, 0),
                                     DwParams(c, D, taps, 1e-5)], (c, 1, 1), (LN_THREADS, 1, 1), groups=True)
    host.k_gemm(y, 0, D, Wb, offs["pw2"], D, None, h, 0, D, c, D, D, 0, 1, 1.0)
    host.k_layernorm(h, 0, *lnb["ff2"], t, 0, c, D)
    host.k_gemm(t, 0, D, Wb, offs["ff2_w1"], D, None, ff, 0, FF, c, FF, D, 1, 0, 1.0)
    host.k_gemm(ff, 0, FF, Wb, offs["ff2_w2"], FF, None, h, 0, D, c, D, FF, 0, 1, 0.5)
    host.k_layernorm2(h, *lnb["out"], *lnb["ff1_next"], t, t2, c, D)
    host.end()

    # the oracle, same sequence
    o = oracle
    x = h0.copy()
    a = o.layernorm(x, *ln["ff1"])
    f = o.gemm(a, mats["ff1_w1"], None, 1)
    x = o.gemm(f, mats["ff1_w2"], None, 0, True, 0.5, C0=x)
    a = o.layernorm(x, *ln["att"])
    kv = kv0.copy()
    kv[pos:pos + c] = o.gemm(a, mats["wqkv"])
    at = o.attention_rel(kv[pos:pos + c], kv[pos - cache:pos + c, D:2 * D], kv[pos - cache:pos + c, 2 * D:], P, bu, bv,
                         c, L, Lmax, H, dh)
    x = o.gemm(at, mats["wo"], None, 0, True, 1.0, C0=x)
    a = o.layernorm(x, *ln["conv"])
    din = din0.copy()
    din[pos:pos + c] = o.gemm(a, mats["pw1"], None, 3)
    yy = o.dwconv_ln_silu(din[pos - conv_left:pos + c], dw, bn_g, bn_b, c)
    x = o.gemm(yy, mats["pw2"], None, 0, True, 1.0, C0=x)
    a = o.layernorm(x, *ln["ff2"])
    f = o.gemm(a, mats["ff2_w1"], None, 1)
    x = o.gemm(f, mats["ff2_w2"], None, 0, True, 0.5, C0=x)
    y1, y2 = o.layernorm2(x, *ln["out"], *ln["ff1_next"])

    assert rel_err(host.get(h, np.float32, (c, D)), x) < 2e-4
    assert rel_err(host.get(t, np.float32, (c, D)), y1) < 2e-4
    assert rel_err(host.get(t2, np.float32, (c, D)), y2) < 2e-4
    kvg = host.get(kvb, np.float32, (cap, 3 * D))
    assert rel_err(kvg[pos:pos + c], kv[pos:pos + c]) < 2e-4
    assert np.array_equal(kvg[:pos], kv0[:pos]) and np.array_equal(kvg[pos + c:], kv0[pos + c:])
    dg = host.get(dinb, np.float32, (cap, D))
    assert rel_err(dg[pos:pos + c], din[pos:pos + c]) < 2e-4
    assert np.array_equal(dg[:pos], din0[:pos])


def test_subsampling_reference_sequence(host):
    """The dw-striding subsampling of one 560 ms window (72 mel rows), dispatched as
    src/encoder.c:118-142 does (conv2d_c1_s2_relu and dwconv2d_s2 by total threads, the 1x1 convs
    and the output projection through k_gemm, flatten_cf), against the oracle."""
    rng = np.random.default_rng(118)
    nwin, F, CH, D = 72, 128, 256, 1024
    sub = oracle.sub_len
    T1, F1 = sub(nwin), F // 2 + 1
    T2, F2 = T1 // 2 + 1, F1 // 2 + 1
    T3, F3 = T2 // 2 + 1, F2 // 2 + 1
    X = rng.standard_normal((nwin, F)).astype(np.float32)
    w0, b0 = (rng.standard_normal((CH, 9)) / 3).astype(np.float32), (0.1 * rng.standard_normal(CH)).astype(np.float32)
    w2, b2 = (rng.standard_normal((CH, 9)) / 3).astype(np.float32), (0.1 * rng.standard_normal(CH)).astype(np.float32)
    w5, b5 = (rng.standard_normal((CH, 9)) / 3).astype(np.float32), (0.1 * rng.standard_normal(CH)).astype(np.float32)
    w3, w6, wo = _w(rng, CH, CH), _w(rng, CH, CH), _w(rng, D, CH * F3)
    b3, b6, bo = ((0.1 * rng.standard_normal(n)).astype(np.float32) for n in (CH, CH, D))
    win = host.put(X)
    bw = [host.put(a) for a in (w0, b0, w2, b2, w5, b5, b3, b6, bo)]
    W3, W6, WO = host.put(w3), host.put(w6), host.put(wo)
    c0, c1, c2 = host.alloc(T1 * F1 * CH * 4), host.alloc(T2 * F2 * CH * 4), host.alloc(T2 * F2 * CH * 4)
    c3, c4, flat = host.alloc(T3 * F3 * CH * 4), host.alloc(T3 * F3 * CH * 4), host.alloc(T3 * F3 * CH * 4)
    pre = host.alloc(T3 * D * 4)
    host.begin()
    host.dispatch("conv2d_c1_s2_relu", [(win, 0), (bw[0], 0), (bw[1], 0), (c0, 0), Conv2dParams(nwin, F, T1, F1, CH)],
                  (CH, F1, T1), (CH, 1, 1))
    host.dispatch("dwconv2d_s2", [(c0, 0), (bw[2], 0), (bw[3], 0), (c1, 0), Conv2dParams(T1, F1, T2, F2, CH)],
                  (CH, F2, T2), (CH, 1, 1))
    host.k_gemm(c1, 0, CH, W3, 0, CH, bw[6], c2, 0, CH, T2 * F2, CH, CH, 2, 0, 1.0)
    host.dispatch("dwconv2d_s2", [(c2, 0), (bw[4], 0), (bw[5], 0), (c3, 0), Conv2dParams(T2, F2, T3, F3, CH)],
                  (CH, F3, T3), (CH, 1, 1))
    host.k_gemm(c3, 0, CH, W6, 0, CH, bw[7], c4, 0, CH, T3 * F3, CH, CH, 2, 0, 1.0)
    host.dispatch("flatten_cf", [(c4, 0), (flat, 0), FlatParams(T3, F3, CH)], (CH, F3, T3), (CH, 1, 1))
    host.k_gemm(flat, 0, CH * F3, WO, 0, CH * F3, bw[8], pre, 0, D, T3, D, CH * F3, 0, 0, 1.0)
    host.end()
    o = oracle
    r0 = o.conv2d_c1_s2_relu(X, w0, b0)
    r1 = o.dwconv2d_s2(r0, w2, b2)
    r2 = o.gemm(r1.reshape(-1, CH), w3, b3, 2).reshape(T2, F2, CH)
    r3 = o.dwconv2d_s2(r2, w5, b5)
    r4 = o.gemm(r3.reshape(-1, CH), w6, b6, 2).reshape(T3, F3, CH)
    fl = o.flatten_cf(r4)
    ref = o.gemm(fl, wo, bo)
    assert rel_err(host.get(c1, np.float32, (T2, F2, CH)), r1) < 1e-5
    assert rel_err(host.get(flat, np.float32, (T3, CH * F3)), fl) < 2e-5
    assert rel_err(host.get(pre, np.float32, (T3, D)), ref) < 2e-5


def test_decoder_round_reference_sequence(host):
    """One prediction update and one joint round of 5 frames, dispatched as src/decoder.c:57-90 does
    (embedding row written through gpu_buf_ptr, the two LSTM layers as k_gemm + k_gemm (+=) +
    lstm_cell, joint.pred, joint_partial over JOINT_GROUPS x rows, argmax_reduce), against the
    oracle: LSTM states, the per-slot partial bests (the reference's layout), argmax indices."""
    rng = np.random.default_rng(57)
    P, J, V, rows, enc_row = 640, 640, 1025, 5, 3
    wx = [_w(rng, 4 * P, P) for _ in range(2)]
    wh = [_w(rng, 4 * P, P) for _ in range(2)]
    lb = [(0.1 * rng.standard_normal(4 * P)).astype(np.float32) for _ in range(2)]
    wjp, bjp = _w(rng, J, P), (0.1 * rng.standard_normal(J)).astype(np.float32)
    wout, bout = _w(rng, V, J), (0.1 * rng.standard_normal(V)).astype(np.float32)
    x0 = rng.standard_normal(P).astype(np.float32)
    hs = [rng.standard_normal(P).astype(np.float32) * 0.5 for _ in range(2)]
    cs = [rng.standard_normal(P).astype(np.float32) * 0.5 for _ in range(2)]
    enc = rng.standard_normal((enc_row + rows + 2, J)).astype(np.float32)
    xb = host.alloc(P * 4)
    gates, pred = host.alloc(4 * P * 4), host.alloc(J * 4)
    WX, WH, LB = [host.put(a) for a in wx], [host.put(a) for a in wh], [host.put(a) for a in lb]
    HB, CB = [host.put(a) for a in hs], [host.put(a) for a in cs]
    HP, CP = [host.alloc(P * 4) for _ in range(2)], [host.alloc(P * 4) for _ in range(2)]
    WJP, BJP, WOUT, BOUT, ENC = host.put(wjp), host.put(bjp), host.put(wout), host.put(bout), host.put(enc)
    nslot = JOINT_GROUPS * GEMM_SIMDS
    pv, pi, am = host.alloc(rows * nslot * 4), host.alloc(rows * nslot * 4), host.alloc(2 * rows * 4)
    host.ptr(xb, np.float32, P)[:] = x0          # src/decoder.c:60-64: the host writes x
    host.begin()
    inp = xb
    for l in range(2):
        host.k_gemm(inp, 0, P, WX[l], 0, P, LB[l], gates, 0, 4 * P, 1, 4 * P, P, 0, 0, 1.0)
        host.k_gemm(HB[l], 0, P, WH[l], 0, P, None, gates, 0, 4 * P, 1, 4 * P, P, 0, 1, 1.0)
        host.dispatch("lstm_cell", [(gates, 0), (CB[l], 0), (CP[l], 0), (HP[l], 0), LstmParams(P)], (P, 1, 1),
                      (64, 1, 1))
        inp = HP[l]
    host.k_gemm(HP[1], 0, P, WJP, 0, P, BJP, pred, 0, J, 1, J, P, 0, 0, 1.0)
    host.dispatch("joint_partial", [(ENC, 0), (pred, 0), (WOUT, 0), (BOUT, 0), (pv, 0), (pi, 0),
                                    JointParams(V, J, enc_row, J)], (JOINT_GROUPS, rows, 1), (GEMM_SIMDS * 32, 1, 1),
                  groups=True)
    host.dispatch("argmax_reduce", [(pv, 0), (pi, 0), (am, 0), CountParams(nslot)], (rows, 1, 1), (256, 1, 1),
                  groups=True)
    host.end()
    o = oracle
    inp_r = x0
    hp_r = []
    for l in range(2):
        g = o.gemm(inp_r[None], wx[l], lb[l])
        g = o.gemm(hs[l][None], wh[l], None, 0, True, 1.0, C0=g)[0]
        c_r, h_r = o.lstm_cell(g, cs[l])
        assert rel_err(host.get(CP[l], np.float32, (P,)), c_r) < 2e-5
        assert rel_err(host.get(HP[l], np.float32, (P,)), h_r) < 2e-5
        hp_r.append(h_r)
        inp_r = h_r
    pred_r = o.gemm(hp_r[1][None], wjp, bjp)[0]
    assert rel_err(host.get(pred, np.float32, (J,)), pred_r) < 2e-5
    got_am = host.get(am, np.int32, (rows, 2))
    got_pv = host.get(pv, np.float32, (rows, nslot))
    got_pi = host.get(pi, np.int32, (rows, nslot))
    predg = host.get(pred, np.float32, (J,))
    for r in range(rows):
        idx, val, logits = o.joint_argmax(enc[enc_row + r], predg, wout, bout)
        # partial layout: slot s keeps the best of n = s, s + 512, ... (lowest index on ties)
        for s in (0, 1, 511):
            ns = np.arange(s, V, nslot)
            assert got_pi[r, s] == ns[np.argmax(logits[ns])]
            assert abs(got_pv[r, s] - logits[ns].max()) <= 1e-4 * max(1.0, abs(logits[ns].max()))
        top2 = np.sort(logits)[-2:]
        if top2[1] - top2[0] > 1e-4:
            assert got_am[r, 0] == idx, r
        assert abs(got_am[r, 1:].view(np.float32)[0] - val) <= 1e-4 * max(1.0, abs(val))


def test_glu_and_refusals(host):
    """The standalone glu kernel (src/kernels.metal:349-356); unknown kernels, wrong argument counts
    and wrong parameter blocks fail the batch with a message and launch nothing."""
    rng = np.random.default_rng(349)
    M, D = 3, 700
    X = rng.standard_normal((M, 2 * D)).astype(np.float32)
    Xb, Yb = host.put(X), host.alloc(M * D * 4)
    host.begin()
    host.dispatch("glu", [(Xb, 0), (Yb, 0), GluParams(M, D)], (D, M, 1), (256, 1, 1))
    host.end()
    ref = X[:, :D] / (1.0 + np.exp(-X[:, D:].astype(np.float64)))
    assert rel_err(host.get(Yb, np.float32, (M, D)), ref) < 1e-6
    L, g = host.L, host.g
    launches = L.gpu_launch_count(g)
    import nemoasr
    for kernel, items in (("gemm_cuda", [(Xb, 0), (Yb, 0), GluParams(M, D)]),
                          ("glu", [(Xb, 0), GluParams(M, D)]),
                          ("glu", [(Xb, 0), (Yb, 0), CountParams(3)]),
                          ("glu", [(Xb, 0), (Yb, 10 ** 9), GluParams(M, D)])):
        arr, keep = nemoasr.gpu_args(*items)
        assert L.gpu_begin(g) == 0
        assert L.gpu_dispatch(g, kernel.encode(), arr, len(items), 1, 1, 1, 1, 1, 1) != 0
        err = C.create_string_buffer(512)
        assert L.gpu_end(g, err, 512) != 0 and err.value
    assert L.gpu_launch_count(g) == launches
