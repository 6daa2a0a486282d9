"""Pins the oracle's streaming bookkeeping and decoder (oracle/oracle_stream.c) on the CPU.

- The window / lo / hi rule (reference src/encoder.c:213-251) emits, over a whole stream, exactly
  the frames of an offline subsampling of all mel frames, contiguously and in order; and the
  subsampled rows a chunk emits equal the offline rows (the 16-row mel cache covers the causal
  receptive field).  Offline reference: torch conv2d with the same causal padding.
- Feeding granularity does not change any output (tokens and every per-layer activation).
- The decoder equals a one-frame-at-a-time greedy RNN-T loop (the semantics of the reference's
  MLX parity script, tools/mlx_reference.py:100-122) run from the oracle's per-kernel functions.
- reset followed by a replay equals a fresh stream.
"""
import json
import os

import numpy as np
import pytest
import torch

import mel_ref
import oracle
import synth
from conftest import model_dir

HERE = os.path.dirname(os.path.abspath(__file__))


def sub(n):
    return n // 2 + 1


@pytest.mark.parametrize("chunk_mel", [8, 16, 56, 112])
@pytest.mark.parametrize("batch", [1, 10, 1000])
def test_plan_emits_offline_frames(chunk_mel, batch):
    for n in list(range(1, 120)) + [333, 1001]:
        b = oracle.EncBook(0, 0, 0, 0, 0)
        fed, total, emitted = 0, 0, 0
        while True:
            if fed < n:
                k = min(batch, n - fed)
                fed += k
                b.pending_n += k
            final = fed >= n
            while True:
                before = b.emitted
                p = oracle.enc_plan(b, final, chunk_mel)
                if not p.ran:
                    break
                assert p.take <= chunk_mel and p.nwin <= 16 + chunk_mel
                if p.c:
                    assert before == emitted  # contiguous, in order
                    emitted += p.c
                    assert b.emitted == emitted
                total += p.c
            if final and b.closed:
                break
        assert total == sub(sub(sub(n))), (n, chunk_mel, batch)


def offline_pre_encode(mel, om):
    """Whole-clip subsampling with torch (f64), channel-major flatten, output projection."""
    t = om.t
    pe = "encoder.pre_encode."
    w = lambda n: torch.tensor(oracle.bf16_to_f32(t[pe + n]).astype(np.float64))
    x = torch.tensor(mel.astype(np.float64))[None, None]
    pad = lambda z: torch.nn.functional.pad(z, (2, 1, 2, 1))
    C = w("conv.0.bias").numel()
    x = torch.relu(torch.nn.functional.conv2d(pad(x), w("conv.0.weight").reshape(C, 1, 3, 3), w("conv.0.bias"), stride=2))
    x = torch.nn.functional.conv2d(pad(x), w("conv.2.weight").reshape(C, 1, 3, 3), w("conv.2.bias"), stride=2, groups=C)
    x = torch.relu(torch.nn.functional.conv2d(x, w("conv.3.weight").reshape(C, C, 1, 1), w("conv.3.bias")))
    x = torch.nn.functional.conv2d(pad(x), w("conv.5.weight").reshape(C, 1, 3, 3), w("conv.5.bias"), stride=2, groups=C)
    x = torch.relu(torch.nn.functional.conv2d(x, w("conv.6.weight").reshape(C, C, 1, 1), w("conv.6.bias")))
    T3 = x.shape[2]
    flat = x[0].permute(1, 0, 2).reshape(T3, -1)  # [T][C*F]
    return (flat @ w("out.weight").T + w("out.bias")).numpy()


@pytest.mark.parametrize("right", [0, 6, 13])
def test_streamed_rows_equal_offline_subsampling(right):
    """Row k of the streamed pre-encode output equals row k of the offline one (layer-0 input):
    compare through the oracle's per-chunk windows at every chunk."""
    om = oracle.Model(model_dir("tiny"))
    mel = mel_ref.logmel(synth.make_audio(2.0, seed=3))
    full = offline_pre_encode(mel, om)
    chunk_mel = (right + 1) * 8
    b = oracle.EncBook(mel.shape[0], 0, 0, 0, 0)
    cache = np.zeros((0, 128), np.float32)
    pend = mel.copy()
    frames = []
    while True:
        p = oracle.enc_plan(b, True, chunk_mel)
        if not p.ran:
            break
        win = np.concatenate([cache, pend[:p.take]])
        pend = pend[p.take:]
        cache = win[-16:]
        if p.c:
            frames.append(offline_pre_encode(win, om)[p.lo:p.hi])
    got = np.concatenate(frames)
    assert got.shape == full.shape
    np.testing.assert_allclose(got, full, rtol=1e-9, atol=1e-9)


def _session_outputs(om, right, mel, step):
    s = oracle.Session(om, right, dump=True)
    for i in range(0, mel.shape[0], step):
        s.feed_mel(mel[i:i + step], final=i + step >= mel.shape[0])
    return s


@pytest.mark.parametrize("right", [0, 6, 13])
def test_feed_granularity_invariant(right):
    om = oracle.Model(model_dir("tiny"))
    mel = mel_ref.logmel(synth.make_audio(3.0, seed=4))
    ref = _session_outputs(om, right, mel, mel.shape[0])
    rl, rp, rj, rrows = ref.dumps()
    for step in (1, 7, 10):
        s = _session_outputs(om, right, mel, step)
        assert s.tokens == ref.tokens
        l, p, j, rows = s.dumps()
        np.testing.assert_array_equal(l, rl)
        np.testing.assert_array_equal(j, rj)


def greedy_one_frame(om, joint_enc):
    """tools/mlx_reference.py:100-122 semantics from the oracle's kernels: per frame, loop
    {prediction net from the committed state and last token; joint argmax; non-blank: emit and
    commit; blank or max_symbols: next frame}."""
    d, t = om.dims, om.t
    P, blank = d.pred_hidden, d.blank_id
    pfx = "decoder.prediction.dec_rnn.lstm."
    Wx = [t[f"{pfx}{l}.Wx"] for l in range(2)]
    Wh = [t[f"{pfx}{l}.Wh"] for l in range(2)]
    bl = [oracle.bf16_to_f32(t[f"{pfx}{l}.bias"]) for l in range(2)]
    emb = t["decoder.prediction.embed.weight"]
    Wp, bp = t["joint.pred.weight"], oracle.bf16_to_f32(t["joint.pred.bias"])
    Wo, bo = t["joint.joint_net.2.weight"], oracle.bf16_to_f32(t["joint.joint_net.2.bias"])
    h = [np.zeros(P, np.float32) for _ in range(2)]
    c = [np.zeros(P, np.float32) for _ in range(2)]
    last, out = blank, []
    for enc in joint_enc:
        symbols = 0
        while True:
            x = np.zeros(P, np.float32) if last == blank else oracle.bf16_to_f32(emb[last])
            hn, cn = [], []
            inp = x
            for l in range(2):
                g = oracle.gemm(inp[None], Wx[l], bl[l], 0, False, 1.0)
                g = oracle.gemm(h[l][None], Wh[l], None, 0, True, 1.0, C0=g)[0]
                c1, h1 = oracle.lstm_cell(g, c[l])
                hn.append(h1)
                cn.append(c1)
                inp = h1
            pred = oracle.gemm(hn[1][None], Wp, bp, 0, False, 1.0)[0]
            k, _, _ = oracle.joint_argmax(enc, pred, Wo, bo)
            if k != blank:
                out.append(k)
                last, h, c = k, hn, cn
                symbols += 1
            if k == blank or symbols >= d.max_symbols:
                break
    return out


@pytest.mark.parametrize("right", [0, 6])
def test_decoder_equals_one_frame_greedy(right):
    """Chunking does not enter the greedy loop: the state carries across chunks and the symbol
    count restarts at every frame (src/decoder.c:97-123), so one pass over all frames must agree."""
    om = oracle.Model(model_dir("tiny"))
    mel = mel_ref.logmel(synth.make_audio(1.5, seed=5))
    s = _session_outputs(om, right, mel, mel.shape[0])
    _, _, je, rows = s.dumps()
    assert sum(rows) == je.shape[0] > 0
    assert s.tokens == greedy_one_frame(om, je)


def test_decoder_with_blanks_equals_one_frame_greedy():
    """Same check on a model whose blank bias is raised (about half the frames decode to blank),
    so the speculative 16-frame batches and the redo-after-token path are both exercised."""
    om = oracle.Model(model_dir("tiny", blank_bias=0.7))
    mel = mel_ref.logmel(synth.make_audio(2.0, seed=6))
    s = _session_outputs(om, 6, mel, mel.shape[0])
    _, _, je, rows = s.dumps()
    best, _ = s.joint_log()
    assert 0.05 < np.mean(best == om.dims.blank_id) < 0.95
    assert s.tokens == greedy_one_frame(om, je)


def test_reset_equals_fresh():
    om = oracle.Model(model_dir("tiny"))
    mel = mel_ref.logmel(synth.make_audio(1.5, seed=7))
    s = oracle.Session(om, 6)
    s.feed_mel(mel, final=True)
    first = list(s.tokens)
    s.reset()
    s.feed_mel(mel, final=True)
    assert s.tokens == first


def test_golden_tokens():
    """Regression pin: committed token ids of the tiny model (tests/golden/make_golden.py)."""
    gold = json.load(open(os.path.join(HERE, "golden", "tiny_tokens.json")))
    for case in gold["cases"]:
        om = oracle.Model(model_dir("tiny", seed=case["model_seed"], blank_bias=case["blank_bias"]), case["language"])
        mel = mel_ref.logmel(synth.make_audio(case["seconds"], seed=case["audio_seed"]))
        s = oracle.Session(om, case["right"])
        s.feed_mel(mel, final=True)
        assert s.tokens == case["tokens"], case["name"]


@pytest.mark.parametrize("language", ["en-US", "auto"])
def test_prompt_fold_equals_one_hot_concat(language):
    """Pins the oracle's prompt fold (b_eff = b0 + W0[:, D + idx] in f32, src/model.c:312-322)
    against the unfolded layer it stands for: prompted = ReLU([h | one-hot(idx)] W0^T + b0) W2^T + b2
    in float64 over the full D + num_prompts columns of W0, with idx the language's entry in
    config.json's prompt_dictionary and h the last block's output rows of the same stream.  A wrong
    prompt index, a dropped one-hot term or a one-hot placed at column idx instead of D + idx all fail."""
    mdir = model_dir("tiny")
    cfg = json.load(open(os.path.join(mdir, "config.json")))
    dic = cfg["prompt"]["prompt_dictionary"]
    idx = dic[language]
    om = oracle.Model(mdir, language)
    d = om.dims
    o = oracle.Session(om, 6, dump=True)
    o.feed_mel(mel_ref.logmel(synth.make_audio(1.5, seed=41)), final=True)
    lay, prompted, _, _ = o.dumps()
    h = lay[:, -1].astype(np.float64)
    t = synth.load_safetensors(os.path.join(mdir, "model.safetensors"))

    def w(name):
        raw, shape = t[name]
        return oracle.bf16_to_f32(np.asarray(raw)).reshape(shape).astype(np.float64)

    W0, b0, W2, b2 = (w(n) for n in ("prompt_kernel.0.weight", "prompt_kernel.0.bias", "prompt_kernel.2.weight",
                                      "prompt_kernel.2.bias"))
    D, NP = d.d_model, d.num_prompts
    assert W0.shape == (d.prompt_hidden, D + NP)

    def unfolded(col):
        x = np.zeros((h.shape[0], D + NP))
        x[:, :D] = h
        if col is not None:
            x[:, col] = 1.0
        return np.maximum(x @ W0.T + b0, 0.0) @ W2.T + b2

    ref = unfolded(D + idx)
    err = float(np.max(np.abs(prompted - ref)) / np.max(np.abs(ref)))
    assert err < 1e-5, err
    other = next(v for k, v in dic.items() if v != idx)
    for wrong in (unfolded(D + other), unfolded(None), unfolded(idx)):
        assert float(np.max(np.abs(prompted - wrong)) / np.max(np.abs(ref))) > 1e-2


def test_token_check_follows_a_forced_tie(tiny_model_dir, monkeypatch):
    """The tie rule of conftest.check_tokens, on the CPU: a decode that took the runner-up at one
    committed decision (what a GPU does at a float tie) passes when that decision counts as a tie
    and the replay forced to it matches to the end; with the tie bound at 0 it fails; and a decode
    with a token changed at no decision of the replay's (a planted error) fails either way."""
    import conftest

    om = oracle.Model(tiny_model_dir, "en-US")
    mel = mel_ref.logmel(synth.make_audio(1.2, seed=31))
    o = oracle.Session(om, 6)
    o.feed_mel(mel, final=True)
    best, second, margin = o.decisions()
    assert len(best) > 10 and len(o.tokens) > 3
    assert np.all(second != best) and np.all(margin >= 0)
    j = 2 + int(np.argmin(margin[2:60]))  # the closest of the first decisions: no earlier one is as close
    forced = oracle.Session(om, 6)
    forced.force({j: int(second[j])})
    forced.feed_mel(mel, final=True)
    assert forced.tokens != o.tokens
    fb, _, _ = forced.decisions()
    assert fb[j] == second[j] and np.array_equal(fb[:j], best[:j])
    monkeypatch.setattr(conftest, "TOKEN_TIE", float(np.nextafter(margin[j], np.float32(np.inf))))
    assert np.all(margin[:j] >= conftest.TOKEN_TIE)  # so the check picks j
    assert conftest.check_tokens(forced.tokens, o.tokens, o.token_margins(), rerun=o.replayer()) == 1
    monkeypatch.setattr(conftest, "TOKEN_TIE", 0.0)
    with pytest.raises(AssertionError):
        conftest.check_tokens(forced.tokens, o.tokens, o.token_margins(), rerun=o.replayer())
    bad = list(o.tokens)
    bad[-1] = (bad[-1] + 1) % om.dims.vocab_size
    monkeypatch.setattr(conftest, "TOKEN_TIE", 1e-4)
    with pytest.raises(AssertionError):
        conftest.check_tokens(bad, o.tokens, o.token_margins(), rerun=o.replayer())
