"""End-to-end parity of the HIP streaming path against the oracle.

The product runs through the public C API (nemoasr_open / nemoasr_debug_feed_mel / nemoasr_feed)
on seeded random-init checkpoints and seeded synthetic audio; the oracle runs the same mel frames
through its CPU restatement.  Gates (from the scope of this path):
  - per-layer encoder activations: max|gpu - oracle| / max|oracle| <= 2e-3 for every layer;
  - joint.enc rows (the joint's encoder input): <= 1e-3; joint logits are checked per kernel;
  - emitted token ids: identical, except at a float tie of the oracle's greedy decision
    (conftest.check_tokens: top-2 joint margin below TOKEN_TIE); there the oracle is replayed with
    that decision taken the GPU's way and the comparison goes on to the end of the stream.
"""
import os
import wave

import numpy as np
import pytest

import mel_ref
import oracle
import synth
from conftest import check_oracle, check_tokens, model_dir, rel_err

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
    check_oracle(toks_g, o)


@pytest.mark.parametrize("latency", [80, 560, 1120])
def test_tiny_stream_parity(latency):
    mdir = model_dir("tiny")
    om, o, s, d = run_pair(mdir, latency, 3.0, seed=11, feed_frames=10, graphs=False)
    check_parity(om, o, s, d)
    s.close()


@pytest.mark.parametrize("latency,seconds", [(80, 2.0), (320, 2.0), (560, 3.0), (1120, 4.0)])
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
    separate launches: every layer's activations within float rounding, the oracle's tokens."""
    import nemoasr

    mdir = model_dir("full")
    om = oracle.Model(mdir, "en-US")
    d = om.dims
    mel = mel_ref.logmel(synth.make_audio(1.5, seed=21))
    o = oracle.Session(om, LAT_RIGHT[latency])
    o.feed_mel(mel, final=True)
    out = []
    for fuse in (True, False):
        s = nemoasr.Session(mdir, "en-US", latency)
        s.chain(False)  # one-row chunks would otherwise run the persistent chain, fused or not
        s.fuse(fuse)
        s.set_dump(True)
        s.feed_mel(mel, final=True)
        out.append((s.tokens(), s.dumps(d.n_layers, d.d_model, d.joint_hidden)))
        s.close()
    (tf, (lf, pf, jf)), (ts, (ls, ps, js)) = out
    check_oracle(tf, o, "fused: ")
    check_oracle(ts, o, "separate: ")
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
    if check_oracle(s.tokens(), o) is None:
        assert s.stats()["tokens"] == len(o.tokens)
    assert s.stats()["chunks"] == o.chunks
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
    check_oracle(s.tokens(), o)
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


def _golden_cases():
    import json

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_tokens.json")
    with open(path) as f:
        return json.load(f)["cases"]


RIGHT_LAT = {v: k for k, v in LAT_RIGHT.items()}


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c["name"])
def test_golden_token_cases(case):
    """The committed token fixtures (tests/golden/tiny_tokens.json: right contexts 0/6/13, en-US
    and auto prompts, blank-biased models) through the public API.  The blank-biased cases must
    actually take the blank branches of the greedy rule (symbol reset on a blank frame, first
    non-blank frame wins, later frames redone): fewer tokens than frames x max_symbols."""
    import nemoasr

    mdir = model_dir("tiny", case["model_seed"], case["blank_bias"])
    lat = RIGHT_LAT[case["right"]]
    mel = mel_ref.logmel(synth.make_audio(case["seconds"], seed=case["audio_seed"]))
    om = oracle.Model(mdir, case["language"])
    o = oracle.Session(om, case["right"])
    o.feed_mel(mel, final=True)
    assert o.tokens == case["tokens"]
    for graphs in (False, True):
        s = nemoasr.Session(mdir, case["language"], lat)
        s.use_graphs(graphs)
        s.feed_mel(mel, final=True)
        check_tokens(s.tokens(), case["tokens"], o.token_margins(), f"graphs {graphs}: ", rerun=o.replayer())
        assert s.stats()["chunks"] == case["chunks"]
        s.close()
    if case["blank_bias"] > 0:
        assert len(case["tokens"]) < case["frames"] * om.dims.max_symbols


@pytest.mark.parametrize("latency,seconds", [(80, 20.0), (560, 24.0)])
def test_stream_cache_compaction(latency, seconds):
    """A single stream long enough that its append-only K/V and conv caches (56 + 8 x 16 rows) are
    compacted at least once (past 184 encoder rows: ~15 s of audio), against the oracle, whose
    histories are plain sliding windows: compaction must be invisible in every layer's rows and in
    the tokens (the reference's epoch rule, src/encoder.c:199-211, :256)."""
    mdir = model_dir("tiny")
    om, o, s, d = run_pair(mdir, latency, seconds, seed=17, graphs=False)
    assert o.frames > 56 + 8 * 16
    check_parity(om, o, s, d)
    s.close()


@pytest.mark.parametrize("latency,seconds", [(80, 20.0), (560, 24.0)])
def test_stream_cache_compaction_graphs(latency, seconds):
    """The same through captured chunk graphs (compaction is a launch outside the chunk graph)."""
    mdir = model_dir("tiny")
    om, o, s, d = run_pair(mdir, latency, seconds, seed=17, graphs=True)
    check_parity(om, o, s, d, check_dumps=False)
    s.close()


@pytest.mark.parametrize("graphs", [False, True])
def test_full_skewed_stream_1120(graphs):
    """The full model with the joint bias skewed as in the 1120 ms benchmark workload
    (P(blank) ~ 0.5 over the benchmark's 30 s clip), on a 4 s clip whose frames mix blank frames,
    emits and redone frames (the oracle: 170 tokens over 51 frames; with random weights a stretch
    of audio tends to decode either to blanks only or to max_symbols per frame), against the oracle."""
    from conftest import SKEW_S1120

    mdir = model_dir("full", 0, *SKEW_S1120)
    om, o, s, d = run_pair(mdir, 1120, 4.0, seed=6, graphs=graphs)
    check_parity(om, o, s, d, check_dumps=not graphs)
    frames, toks = o.frames, len(o.tokens)
    assert 0 < toks < frames * om.dims.max_symbols, (frames, toks)
    s.close()


def _oracle_audio_tokens(mdir, audio16, latency):
    om = oracle.Model(mdir, "en-US")
    o = oracle.Session(om, LAT_RIGHT[latency])
    o.feed_mel(mel_ref.logmel(audio16), final=True)
    return o


@pytest.mark.parametrize("latency", [80, 560])
def test_api_ragged_and_empty_feeds(latency):
    """nemoasr_feed with empty calls (before, between, and as the final flush) and ragged piece sizes
    (1 sample up to several chunks) decodes exactly what one whole-clip call decodes, and the
    oracle's tokens (src/nemoasr.c:134-160: audio is queued and every ready chunk runs)."""
    import nemoasr

    mdir = model_dir("tiny")
    audio = synth.make_audio(2.3, seed=41)
    o = _oracle_audio_tokens(mdir, audio, latency)
    whole = nemoasr.Session(mdir, "en-US", latency)
    whole.feed(audio, final=True)
    rng = np.random.default_rng(latency)
    s = nemoasr.Session(mdir, "en-US", latency)
    assert s.feed(np.zeros(0, np.float32)) in ("", None)
    assert s.stats()["chunks"] == 0 and s.tokens() == []
    pos = 0
    while pos < audio.size:
        n = int(rng.choice([1, 7, 160, 1279, 1280, 1281, 4000, 17000]))
        s.feed(audio[pos:pos + n])
        if rng.random() < 0.2:
            s.feed(np.zeros(0, np.float32))
        pos += n
    s.feed(np.zeros(0, np.float32), final=True)  # the final flush carries no samples
    assert s.tokens() == whole.tokens()
    assert s.stats()["chunks"] == whole.stats()["chunks"] == o.chunks
    check_oracle(s.tokens(), o)
    s.close()
    whole.close()


@pytest.mark.parametrize("seconds", [0.05, 0.2, 0.6])
def test_api_clip_shorter_than_a_chunk(seconds):
    """Clips shorter than one 560 ms chunk: the final flush runs the partial window (the
    boundary rule of src/encoder.c) and decodes what the oracle decodes, including nothing."""
    import nemoasr

    mdir = model_dir("tiny")
    audio = synth.make_audio(seconds, seed=43)
    o = _oracle_audio_tokens(mdir, audio, 560)
    s = nemoasr.Session(mdir, "en-US", 560)
    s.feed(audio, final=True)
    check_oracle(s.tokens(), o)
    assert s.stats()["chunks"] == o.chunks
    s.close()


def _product_resample(x, rate):
    """The library's streaming resampler (pinned against the reference's src/resample.c on the CPU)."""
    import ctypes as C

    import nemoasr

    L = nemoasr.lib()
    r = L.rsmp_create(rate, 16000)
    buf = np.zeros(x.size * 16000 // rate + 4096, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    fp = C.POINTER(C.c_float)
    k = L.rsmp_process(r, x.ctypes.data_as(fp), x.size, buf.ctypes.data_as(fp), buf.size)
    k2 = L.rsmp_flush(r, buf[k:].ctypes.data_as(fp), buf.size - k)
    L.rsmp_destroy(r)
    return buf[:k + k2].copy()


@pytest.mark.parametrize("rate", [8000, 48000])
def test_api_input_rate(rate):
    """A session opened at another input rate resamples to 16 kHz on the host (src/nemoasr.c:66-87
    and :134-160) and decodes what the oracle decodes from the resampled samples."""
    import nemoasr

    mdir = model_dir("tiny")
    t = np.arange(int(2.0 * rate)) / rate
    audio = (0.05 * np.sin(2 * np.pi * 440 * t) + 0.02 * np.random.default_rng(rate).standard_normal(t.size))
    audio = audio.astype(np.float32)
    o = _oracle_audio_tokens(mdir, _product_resample(audio, rate), 560)
    s = nemoasr.Session(mdir, "en-US", 560, input_rate=rate)
    for i in range(0, audio.size, rate // 10):
        s.feed(audio[i:i + rate // 10], final=i + rate // 10 >= audio.size)
    check_oracle(s.tokens(), o)
    assert s.stats()["chunks"] == o.chunks
    s.close()


@pytest.mark.parametrize("latency", [80, 560, 1120])
def test_first_chunks_replay_prepared_graphs(latency):
    """The warm-up at open runs silence through the session's own encoder, capturing each chunk
    shape's graph on first sight, and captures the decoder's graphs of every run size (the
    reference warms its pipelines the same way, src/warmup.c:7-42): the stream's first three chunks
    then issue no direct kernel launch.  The same holds after nemoasr_prepare_latency of another
    latency and a reset to it (the prepared encoder is kept), and the decode is the oracle's."""
    import ctypes as C

    import nemoasr

    mdir = model_dir("tiny")
    L = nemoasr.lib()
    other = 560 if latency != 560 else 1120
    s = nemoasr.Session(mdir, "en-US", latency)
    err = C.create_string_buffer(256)
    for lat in (latency, other):
        chunk = 8 * (LAT_RIGHT[lat] + 1)
        mel = mel_ref.logmel(synth.make_audio(4.0 * chunk * 0.01 + 0.3, seed=50 + lat))
        if lat != latency:
            assert L.nemoasr_prepare_latency(s.h, lat, err, 256) == 0, err.value
            s.reset("en-US", lat)
        n0 = L.nemoasr_debug_launches(s.h)
        s.feed_mel(mel[:3 * chunk], final=False)
        assert s.stats()["chunks"] == 3
        assert L.nemoasr_debug_launches(s.h) == n0, f"{lat} ms: direct launches in the first chunks"
        s.feed_mel(mel[3 * chunk:], final=True)
        om = oracle.Model(mdir, "en-US")
        o = oracle.Session(om, LAT_RIGHT[lat])
        o.feed_mel(mel, final=True)
        check_oracle(s.tokens(), o, f"{lat} ms: ")
    s.close()
