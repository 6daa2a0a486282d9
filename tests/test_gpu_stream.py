"""End-to-end parity of the HIP streaming path against the oracle.

The product runs through the public C API (nemoasr_open / nemoasr_debug_feed_mel / nemoasr_feed)
on seeded random-init checkpoints and seeded synthetic audio; the oracle runs the same mel frames
through its CPU restatement.  Gates (from the scope of this path):
  - per-layer encoder activations: max|gpu - oracle| / max|oracle| <= 2e-3 for every layer;
  - joint.enc rows (the joint's encoder input): <= 1e-3; joint logits are checked per kernel;
  - emitted token ids: identical.
"""
import os
import wave

import numpy as np
import pytest

import mel_ref
import oracle
import synth
from conftest import model_dir, rel_err

pytestmark = pytest.mark.gpu

LAT_RIGHT = {80: 0, 160: 1, 320: 3, 560: 6, 1120: 13}


def run_pair(mdir, latency, seconds, seed, feed_frames=None, graphs=True):
    import nemoasr

    om = oracle.Model(mdir, "en-US")
    d = om.dims
    audio = synth.make_audio(seconds, seed=seed)
    mel = mel_ref.logmel(audio)
    step = feed_frames or mel.shape[0]
    o = oracle.Session(om, LAT_RIGHT[latency], dump=True)
    s = nemoasr.Session(mdir, "en-US", latency)
    s.set_dump(not graphs)
    if graphs:
        s.use_graphs(True)
    for i in range(0, mel.shape[0], step):
        fin = i + step >= mel.shape[0]
        o.feed_mel(mel[i:i + step], final=fin)
        s.feed_mel(mel[i:i + step], final=fin)
    return om, o, s, d


def check_parity(om, o, s, d, check_dumps=True):
    ol, op, oj, rows = o.dumps()
    toks_g = s.tokens()
    if check_dumps:
        gl, gp, gj = s.dumps(d.n_layers, d.d_model, d.joint_hidden)
        assert gl.shape == ol.shape, (gl.shape, ol.shape)
        errs = [rel_err(gl[:, l], ol[:, l]) for l in range(d.n_layers)]
        print("per-layer max rel err:", " ".join(f"{e:.1e}" for e in errs))
        assert max(errs) <= 2e-3, errs
        assert rel_err(gp, op) <= 2e-3
        assert rel_err(gj, oj) <= 1e-3
    if toks_g != o.tokens:
        first = next(i for i, (a, b) in enumerate(zip(toks_g + [-1], o.tokens + [-2])) if a != b)
        _, margin = o.joint_log()
        pytest.fail(f"tokens differ at {first} of {len(o.tokens)}; oracle min top-2 margin {margin.min():.3g}")


@pytest.mark.parametrize("latency", [80, 560, 1120])
def test_tiny_stream_parity(latency):
    mdir = model_dir("tiny")
    om, o, s, d = run_pair(mdir, latency, 3.0, seed=11, feed_frames=10, graphs=False)
    check_parity(om, o, s, d)
    s.close()


@pytest.mark.parametrize("latency,seconds", [(80, 2.0), (560, 3.0), (1120, 4.0)])
def test_full_stream_parity(latency, seconds):
    mdir = model_dir("full")
    om, o, s, d = run_pair(mdir, latency, seconds, seed=3, graphs=False)
    check_parity(om, o, s, d)
    s.close()


@pytest.mark.parametrize("latency", [80, 560])
def test_graph_replay_matches(latency):
    """Chunks replayed from captured hipGraphs give the oracle's tokens (and so the direct path's)."""
    mdir = model_dir("full")
    om, o, s, d = run_pair(mdir, latency, 3.0, seed=5, graphs=True)
    check_parity(om, o, s, d, check_dumps=False)
    s.close()


@pytest.mark.parametrize("latency", [80, 160])
def test_fused_launches_match_separate(latency):
    """The one- and two-row chunks' fused launches (attention + out_proj, dwconv + pw2) against the
    separate launches: every layer's activations within float rounding, identical tokens."""
    import nemoasr

    mdir = model_dir("full")
    d = oracle.Model(mdir, "en-US").dims
    mel = mel_ref.logmel(synth.make_audio(1.5, seed=21))
    out = []
    for fuse in (True, False):
        s = nemoasr.Session(mdir, "en-US", latency)
        s.fuse(fuse)
        s.set_dump(True)
        s.feed_mel(mel, final=True)
        out.append((s.tokens(), s.dumps(d.n_layers, d.d_model, d.joint_hidden)))
        s.close()
    (tf, (lf, pf, jf)), (ts, (ls, ps, js)) = out
    assert tf == ts
    assert rel_err(lf, ls) < 1e-5 and rel_err(jf, js) < 1e-5


def test_audio_api_tiny():
    """nemoasr_feed from audio in 100 ms blocks (the library's intended use, tools/libtest.c:20-26)
    gives the oracle's tokens from its own mel restatement."""
    import nemoasr

    mdir = model_dir("tiny")
    audio = synth.make_audio(2.5, seed=4)
    om = oracle.Model(mdir, "en-US")
    o = oracle.Session(om, LAT_RIGHT[560])
    o.feed_mel(mel_ref.logmel(audio), final=True)
    s = nemoasr.Session(mdir, "en-US", 560)
    text = ""
    for i in range(0, audio.size, 1600):
        text += s.feed(audio[i:i + 1600], final=i + 1600 >= audio.size)
    assert s.tokens() == o.tokens
    st = s.stats()
    assert st["tokens"] == len(o.tokens) and st["chunks"] == o.chunks
    s.close()


def test_reset_replays_identically():
    import nemoasr

    mdir = model_dir("tiny")
    mel = mel_ref.logmel(synth.make_audio(2.0, seed=9))
    s = nemoasr.Session(mdir, "en-US", 560)
    s.feed_mel(mel, final=True)
    first = s.tokens()
    s.reset("en-US", 560)
    s.feed_mel(mel, final=True)
    assert s.tokens() == first
    s.reset("en-US", 80)
    om = oracle.Model(mdir, "en-US")
    o = oracle.Session(om, 0)
    o.feed_mel(mel, final=True)
    s.feed_mel(mel, final=True)
    assert s.tokens() == o.tokens
    s.close()


@pytest.mark.parametrize("latency", [80, 560])
def test_parity_harness_end_to_end(tmp_path, latency):
    """The real-checkpoint harness (parity.py: WAV in, CLI-format dumps out, compare.py gates) on a
    synthetic checkpoint, against a reference directory in the MLX dump format that the oracle
    writes from the same WAV samples."""
    import parity

    mdir = model_dir("tiny")
    pcm = np.clip(np.round(synth.make_audio(2.5, seed=21) * 32768), -32768, 32767).astype(np.int16)
    wav = str(tmp_path / "in.wav")
    with wave.open(wav, "wb") as w:
        w.setnchannels(1)
        w.setsampwidth(2)
        w.setframerate(16000)
        w.writeframes(pcm.tobytes())
    x = pcm.astype(np.float32) / np.float32(32768)
    om = oracle.Model(mdir, "en-US")
    o = oracle.Session(om, LAT_RIGHT[latency], dump=True)
    mel = mel_ref.logmel(x)
    o.feed_mel(mel, final=True)
    _, prompted, _, _ = o.dumps()
    ref = str(tmp_path / "ref")
    os.makedirs(ref)
    mel.astype(np.float32).tofile(os.path.join(ref, "mel.f32"))
    prompted.astype(np.float32).tofile(os.path.join(ref, "enc_all.f32"))
    with open(os.path.join(ref, "tokens.txt"), "w") as f:
        f.write(" ".join(map(str, o.tokens)) + "\n\n")

    res = parity.run(mdir, wav, latency)
    out = str(tmp_path / "out")
    parity.write_dumps(out, res["mel"], res["enc"], res["tokens"])
    ok, rep = parity.compare(ref, out, om.dims.d_model)
    print("\n".join(rep))
    assert ok, rep
    assert res["mel"].shape == mel.shape and len(o.tokens) > 0
