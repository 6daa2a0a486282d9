#!/usr/bin/env python3
"""Writes the committed golden fixtures from the oracle (the CPU restatement in oracle/).

kernels.npz     seeded inputs and oracle outputs for every kernel at small shapes
                (keys '<case>/<name>'), read by tests/test_golden.py on the CPU (the oracle must
                reproduce them bit for bit) and by the GPU tests (the HIP kernels must match them
                to the stated tolerances).
tiny_tokens.json token ids of short synthetic clips through the tiny seeded model.

Run from the repository root:  python tests/golden/make_golden.py
The fixtures change only when the oracle's arithmetic changes; regenerate and review the diff then.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(REPO, "oracle"), os.path.join(REPO, "nemo-c_amd"), os.path.join(REPO, "tests")]

import oracle  # noqa: E402

TOKEN_CASES = [
    # name, right context, blank bias, language, seconds, audio seed
    ("r0_en", 0, 0.0, "en-US", 1.0, 11),
    ("r6_en", 6, 0.0, "en-US", 2.0, 12),
    ("r13_auto", 13, 0.0, "auto", 2.5, 13),
    ("r6_blank07", 6, 0.7, "en-US", 2.0, 14),
    ("r1_blank06", 1, 0.6, "auto", 1.5, 15),
]


def w_bf16(rng, n, k):
    return oracle.f32_to_bf16(rng.standard_normal((n, k)).astype(np.float32) / np.sqrt(k))


def kernel_cases():
    rng = np.random.default_rng(20261201)
    out = {}

    def put(case, **kv):
        for k, v in kv.items():
            out[f"{case}/{k}"] = np.asarray(v)

    # GEMM: every epilogue, accumulate + alpha, ldw > K (prompt W0 layout)
    for act in range(4):
        M, N, K = 3, 48, 80
        A = rng.standard_normal((M, K)).astype(np.float32)
        W = w_bf16(rng, N, K)
        b = (0.1 * rng.standard_normal(N)).astype(np.float32)
        C0 = rng.standard_normal((M, N // 2 if act == 3 else N)).astype(np.float32)
        acc, alpha = (1, 0.5) if act == 0 else (0, 1.0)
        Y = oracle.gemm(A, W, b, act, bool(acc), alpha, C0=C0 if acc else None)
        put(f"gemm_act{act}", A=A, W=W, bias=b, C0=C0, act=act, acc=acc, alpha=alpha, Y=Y)
    A = rng.standard_normal((2, 96)).astype(np.float32)
    W = w_bf16(rng, 32, 112)
    put("gemm_ldw", A=A, W=W, K=96, Y=oracle.gemm(A, W, None, 2, False, 1.0, ldw=112, K=96))

    # LayerNorm and the paired form
    X = (3.0 + 2.0 * rng.standard_normal((3, 256))).astype(np.float32)
    g1, b1, g2, b2 = (1 + 0.1 * rng.standard_normal((4, 256))).astype(np.float32)
    put("layernorm", X=X, g=g1, b=b1, Y=oracle.layernorm(X, g1, b1))
    Y1, Y2 = oracle.layernorm2(X, g1, b1, g2, b2)
    put("layernorm2", X=X, g1=g1, b1=b1, g2=g2, b2=b2, Y1=Y1, Y2=Y2)

    # rel-pos attention: 2 heads of 16, c=3 queries over L=9 keys, Lmax 12
    H, dh, c, L, Lmax = 2, 16, 3, 9, 12
    D = H * dh
    kv = rng.standard_normal((L, 3 * D)).astype(np.float32)
    P = rng.standard_normal((2 * Lmax - 1, D)).astype(np.float32)
    bu, bv = (0.1 * rng.standard_normal((2, D))).astype(np.float32)
    Q = kv[L - c:]
    O = oracle.attention_rel(Q, kv[:, D:2 * D].copy(), kv[:, 2 * D:].copy(), P, bu, bv, c, L, Lmax, H, dh)
    put("attention", kv=kv, P=P, bu=bu, bv=bv, c=c, L=L, Lmax=Lmax, H=H, dh=dh, O=O)

    # causal depthwise conv + LN + SiLU: 8 history rows + c=3
    din = rng.standard_normal((8 + 3, 64)).astype(np.float32)
    Wd = (rng.standard_normal((64, 9)) / 3).astype(np.float32)
    g, b = (1 + 0.1 * rng.standard_normal((2, 64))).astype(np.float32)
    put("dwconv", din=din, W=Wd, g=g, b=b, c=3, Y=oracle.dwconv_ln_silu(din, Wd, g, b, 3))

    # subsampling convolutions on a 7 x 12 window with 4 channels
    Xm = rng.standard_normal((7, 12)).astype(np.float32)
    W0, b0 = (rng.standard_normal((4, 9)) / 3).astype(np.float32), (0.1 * rng.standard_normal(4)).astype(np.float32)
    Y0 = oracle.conv2d_c1_s2_relu(Xm, W0, b0)
    Wd2, bd2 = (rng.standard_normal((4, 9)) / 3).astype(np.float32), (0.1 * rng.standard_normal(4)).astype(np.float32)
    Yd = oracle.dwconv2d_s2(Y0, Wd2, bd2)
    put("subsampling", X=Xm, W0=W0, b0=b0, Y0=Y0, Wd=Wd2, bd=bd2, Yd=Yd, flat=oracle.flatten_cf(Yd))

    # LSTM cell and joint argmax (with a planted exact tie at indices 5 and 9)
    gates = (2 * rng.standard_normal(4 * 40)).astype(np.float32)
    cin = rng.standard_normal(40).astype(np.float32)
    co, ho = oracle.lstm_cell(gates, cin)
    put("lstm", gates=gates, c_in=cin, c_out=co, h_out=ho)
    enc, pred = rng.standard_normal((2, 48)).astype(np.float32)
    Wj = w_bf16(rng, 33, 48)
    bj = (0.1 * rng.standard_normal(33)).astype(np.float32)
    i, v, logits = oracle.joint_argmax(enc, pred, Wj, bj)
    put("joint", enc=enc, pred=pred, W=Wj, bias=bj, idx=i, val=np.float32(v), logits=logits)
    Wt = np.zeros((12, 48), np.uint16)
    Wt[5] = Wt[9] = Wj[0]
    bt = np.zeros(12, np.float32)
    i, v, logits = oracle.joint_argmax(enc, pred, Wt, bt)
    put("joint_tie", enc=enc, pred=pred, W=Wt, bias=bt, idx=i, val=np.float32(v))

    # sinusoidal relative-position table projected by a linear_pos weight
    Wp = w_bf16(rng, 32, 32)
    put("ptab", W=Wp, D=32, Lmax=6, P=oracle.ptab(Wp, 32, 6))
    return out


def token_cases():
    import mel_ref
    import synth
    from conftest import model_dir

    cases = []
    for name, right, bb, lang, secs, aseed in TOKEN_CASES:
        om = oracle.Model(model_dir("tiny", 0, bb), lang)
        s = oracle.Session(om, right)
        s.feed_mel(mel_ref.logmel(synth.make_audio(secs, seed=aseed)), final=True)
        cases.append({"name": name, "model_seed": 0, "blank_bias": bb, "language": lang, "right": right,
                      "seconds": secs, "audio_seed": aseed, "chunks": s.chunks, "frames": s.frames,
                      "tokens": s.tokens})
    return cases


def main():
    k = kernel_cases()
    np.savez_compressed(os.path.join(HERE, "kernels.npz"), **k)
    with open(os.path.join(HERE, "tiny_tokens.json"), "w") as f:
        json.dump({"model": "tiny seeded random-init (synth.TINY_DIMS, seed 0)", "cases": token_cases()}, f, indent=1)
    print("wrote", len(k), "arrays and", len(TOKEN_CASES), "token cases")


if __name__ == "__main__":
    main()
