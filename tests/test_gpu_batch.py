"""Multi-stream batching (include/nemoasr_batch.h) against the oracle.

Every stream of a batch must emit exactly the tokens that the oracle's single-stream session emits
for that stream's audio, whatever the other streams do: different lengths, staggered starts,
streams ending while others continue, a slot reused after reset (conftest.check_tokens: at a float
tie of the oracle's greedy decision the oracle is replayed with that decision taken the GPU's way,
and the comparison goes on to the end of the stream).  The
joint.enc rows of each stream (the joint's encoder input) are held to the encoder gate of the
single-stream tests (1e-3 relative).
"""
import numpy as np
import pytest

import mel_ref
import oracle
import synth
from conftest import check_tokens, model_dir, rel_err

pytestmark = pytest.mark.gpu

LAT_RIGHT = {80: 0, 160: 1, 320: 3, 560: 6, 1120: 13}


_ORACLE = {}


def oracle_run(om, latency, mel, key=None):
    """Oracle tokens, joint.enc rows, per-token decision margins and the replay for ties
    (oracle.Session.replayer) of one stream (cached by key across parametrizations)."""
    if key is not None and key in _ORACLE:
        return _ORACLE[key]
    o = oracle.Session(om, LAT_RIGHT[latency], dump=True)
    o.feed_mel(mel, final=True)
    _, _, oj, _ = o.dumps()
    res = (list(o.tokens), oj, o.token_margins(), o.replayer())
    if key is not None:
        _ORACLE[key] = res
    print(f"  oracle {key or ''}: {mel.shape[0]} mel rows, {len(o.tokens)} tokens", flush=True)
    return res


def drive(b, mels, starts, piece):
    """Feed each stream `piece` mel rows per tick from tick starts[s] on, one batch step per tick."""
    pos = [0] * len(mels)
    tick = 0
    while any(p < m.shape[0] for p, m in zip(pos, mels)):
        for s, m in enumerate(mels):
            if tick < starts[s] or pos[s] >= m.shape[0]:
                continue
            end = min(pos[s] + piece, m.shape[0])
            b.push_mel(s, m[pos[s]:end], final=end >= m.shape[0])
            pos[s] = end
        b.step()
        tick += 1
    b.run()


def check_streams(b, om, latency, mels, J, tag=None):
    for s, m in enumerate(mels):
        toks, oj, margins, rerun = oracle_run(om, latency, m, None if tag is None else (tag, s))
        gj = b.joint_enc(s, J)
        assert gj.shape == oj.shape, (s, gj.shape, oj.shape)
        err = rel_err(gj, oj)
        assert err <= 1e-3, (s, err)
        check_tokens(b.tokens(s), toks, margins, f"stream {s}: ", rerun=rerun)


@pytest.mark.parametrize("device_loop", [True, False])
@pytest.mark.parametrize("latency", [80, 560, 1120])
def test_tiny_batch_matches_oracle(latency, device_loop):
    """Both greedy loops: device-resident (graph runs of steps) and one host round trip per step."""
    import nemoasr

    mdir = model_dir("tiny")
    om = oracle.Model(mdir, "en-US")
    secs = [2.0, 1.3, 2.6, 0.4, 1.9, 2.2]
    mels = [mel_ref.logmel(synth.make_audio(t, seed=40 + i)) for i, t in enumerate(secs)]
    starts = [0, 0, 3, 5, 1, 9]
    b = nemoasr.Batch(mdir, "en-US", latency, streams=len(mels))
    b.device_decoder(device_loop)
    b.set_dump(True)
    drive(b, mels, starts, piece=8 * (LAT_RIGHT[latency] + 1))
    check_streams(b, om, latency, mels, om.dims.joint_hidden, tag=("tiny", latency))
    st = b.stats()
    assert st["chunks"] > 0 and st["tokens"] == sum(len(b.tokens(s)) for s in range(len(mels)))
    b.close()


def test_batch_loop_choice_only_before_input():
    """The greedy loop (device-resident or host-driven) is chosen before any input: the two keep
    their greedy state apart, so a later switch is refused and the batch decodes on as it was."""
    import nemoasr

    mdir = model_dir("tiny")
    om = oracle.Model(mdir, "en-US")
    mels = [mel_ref.logmel(synth.make_audio(t, seed=70 + i)) for i, t in enumerate([1.5, 0.9])]
    b = nemoasr.Batch(mdir, "en-US", 80, streams=len(mels))
    b.device_decoder(False)
    b.device_decoder(True)
    b.set_dump(True)
    b.push_mel(0, mels[0][:16])
    with pytest.raises(RuntimeError):
        b.device_decoder(False)
    b.push_mel(0, mels[0][16:], final=True)
    b.push_mel(1, mels[1], final=True)
    b.run()
    check_streams(b, om, 80, mels, om.dims.joint_hidden, tag=("tiny-choice", 80))
    b.close()


@pytest.mark.parametrize("graphs", [False, True])
def test_full_batch_matches_oracle(graphs):
    """Full-size model, 560 ms, four streams in lockstep (graph replay of the steady step) and
    one that starts late and ends early."""
    import nemoasr

    mdir = model_dir("full")
    om = oracle.Model(mdir, "en-US")
    secs = [2.5, 2.5, 2.0, 2.5, 1.2]
    mels = [mel_ref.logmel(synth.make_audio(t, seed=60 + i)) for i, t in enumerate(secs)]
    b = nemoasr.Batch(mdir, "en-US", 560, streams=len(mels))
    b.use_graphs(graphs)
    b.set_dump(True)
    drive(b, mels, [0, 0, 0, 0, 4], piece=56)
    check_streams(b, om, 560, mels, om.dims.joint_hidden, tag=("full", 560))
    b.close()


def test_batch_matches_sessions_full():
    """Sixteen streams at 560 ms and sixteen single-stream sessions (different kernels: many-row
    MFMA tiles against weight-streaming GEMVs), both against the oracle."""
    import nemoasr

    mdir = model_dir("full")
    om = oracle.Model(mdir, "en-US")
    mels = [mel_ref.logmel(synth.make_audio(1.5 + 0.1 * (i % 5), seed=80 + i)) for i in range(16)]
    b = nemoasr.Batch(mdir, "en-US", 560, streams=16)
    for s, m in enumerate(mels):
        b.push_mel(s, m, final=True)
    b.run()
    sess = nemoasr.Session(mdir, "en-US", 560)
    for s, m in enumerate(mels):
        toks, _, margins, rerun = oracle_run(om, 560, m)
        sess.reset("en-US", 560)
        sess.feed_mel(m, final=True)
        check_tokens(b.tokens(s), toks, margins, f"batch stream {s}: ", rerun=rerun)
        check_tokens(sess.tokens(), toks, margins, f"session {s}: ", rerun=rerun)
    sess.close()
    b.close()


@pytest.mark.parametrize("latency", [560, 1120])
def test_batch_many_streams_compacted(latency):
    """130 streams, three row blocks of the greedy loop's GEMMs: the compacted step rows, the row
    blocks past the live count that return at once and the joint GEMM's device-side row count,
    with streams of different lengths and starts (so the live count changes from step to step),
    against the oracle (and single-stream sessions, also against the oracle).  Streams 93 and 121
    carried float ties of the oracle (top-2 margins 3.9e-6 and 2.8e-6 at tokens 59 and 52) when the
    GPU still summed with atomics; any tie is followed to the end of its stream."""
    import nemoasr

    mdir = model_dir("tiny")
    om = oracle.Model(mdir, "en-US")
    S = 130
    mels = [mel_ref.logmel(synth.make_audio(0.4 + 0.07 * (i % 23), seed=300 + i)) for i in range(S)]
    b = nemoasr.Batch(mdir, "en-US", latency, streams=S)
    drive(b, mels, [i % 5 for i in range(S)], piece=8 * (LAT_RIGHT[latency] + 1))
    sess = nemoasr.Session(mdir, "en-US", latency)
    ties = 0
    for s, m in enumerate(mels):
        toks, _, margins, rerun = oracle_run(om, latency, m, ("many", latency, s))
        sess.reset("en-US", latency)
        sess.feed_mel(m, final=True)
        ties += check_tokens(b.tokens(s), toks, margins, f"batch stream {s}: ", rerun=rerun) or 0
        ties += check_tokens(sess.tokens(), toks, margins, f"session {s}: ", rerun=rerun) or 0
    print(f"  {ties} float ties among {2 * S} decodes, each followed to the end of its stream", flush=True)
    sess.close()
    b.close()


@pytest.mark.parametrize("latency", [80, 560])
def test_batch_cache_compaction(latency):
    """Streams long enough that their K/V and conv cache regions (56 + 8 x cmax rows) fill and
    are compacted at least once, next to a short stream, with staggered starts, against the
    oracle (whose histories are plain sliding windows: compaction must be invisible)."""
    import nemoasr

    mdir = model_dir("tiny")
    om = oracle.Model(mdir, "en-US")
    secs = [9.5, 8.8, 10.2, 2.0] if latency == 80 else [24.0, 22.5, 25.0, 6.0]
    mels = [mel_ref.logmel(synth.make_audio(t, seed=500 + i)) for i, t in enumerate(secs)]
    b = nemoasr.Batch(mdir, "en-US", latency, streams=len(mels))
    b.set_dump(True)
    drive(b, mels, [0, 3, 1, 7], piece=8 * (LAT_RIGHT[latency] + 1))
    check_streams(b, om, latency, mels, om.dims.joint_hidden)
    b.close()


@pytest.mark.parametrize("gpu_fe", [True, False])
def test_batch_audio_and_reset(gpu_fe):
    """Audio pushed in 100 ms blocks, text per stream, and a slot reused after reset_stream; log-mel
    on the GPU (default) and on the host."""
    import nemoasr

    mdir = model_dir("tiny")
    om = oracle.Model(mdir, "en-US")
    audios = [synth.make_audio(t, seed=90 + i) for i, t in enumerate([1.8, 2.3, 1.1])]
    b = nemoasr.Batch(mdir, "en-US", 560, streams=3)
    b.gpu_frontend(gpu_fe)
    for i in range(0, max(a.size for a in audios), 1600):
        for s, a in enumerate(audios):
            if i < a.size:
                b.push(s, a[i:i + 1600], final=i + 1600 >= a.size)
        b.step()
    b.run()
    for s, a in enumerate(audios):
        toks, _, margins, rerun = oracle_run(om, 560, mel_ref.logmel(a))
        check_tokens(b.tokens(s), toks, margins, f"stream {s}: ", rerun=rerun)
        b.text(s)
    first = b.tokens(1)
    b.reset_stream(1)
    assert b.tokens(1) == []
    b.push(1, audios[1], final=True)
    b.run()
    assert b.tokens(1) == first
    b.close()


@pytest.mark.parametrize("latency", [80, 1120])
def test_batch_gpu_frontend_matches_host(latency):
    """The GPU log-mel front end against the host's, full model, audio fed in uneven pieces: the
    same tokens and joint.enc rows within float rounding (the spectra are computed identically;
    only the log may round differently), and the oracle's tokens."""
    import nemoasr

    mdir = model_dir("full")
    om = oracle.Model(mdir, "en-US")
    audios = [synth.make_audio(t, seed=200 + i) for i, t in enumerate([2.2, 1.6, 2.9, 0.7])]
    out = []
    for gpu_fe in (True, False):
        b = nemoasr.Batch(mdir, "en-US", latency, streams=len(audios))
        b.gpu_frontend(gpu_fe)
        b.set_dump(True)
        pieces = [2100, 900, 4700, 1600]
        pos = [0] * len(audios)
        while any(p < a.size for p, a in zip(pos, audios)):
            for s, a in enumerate(audios):
                if pos[s] < a.size:
                    n = pieces[s % len(pieces)]
                    b.push(s, a[pos[s]:pos[s] + n], final=pos[s] + n >= a.size)
                    pos[s] += n
            b.step()
        b.run()
        out.append([(b.tokens(s), b.joint_enc(s, om.dims.joint_hidden)) for s in range(len(audios))])
        b.close()
    for s, a in enumerate(audios):
        (tg, jg), (th, jh) = out[0][s], out[1][s]
        assert rel_err(jg, jh) < 1e-4, s
        toks, _, margins, rerun = oracle_run(om, latency, mel_ref.logmel(a))
        check_tokens(tg, toks, margins, f"gpu front end, stream {s}: ", rerun=rerun)
        check_tokens(th, toks, margins, f"host front end, stream {s}: ", rerun=rerun)


def test_batch_mixed_input_rejected():
    """With the GPU front end a stream takes either audio or mel rows until it is reset."""
    import nemoasr

    mdir = model_dir("tiny")
    b = nemoasr.Batch(mdir, "en-US", 560, streams=2)
    b.push(0, np.zeros(1600, np.float32))
    with pytest.raises(RuntimeError):
        b.push_mel(0, np.zeros((8, 128), np.float32))
    b.push_mel(1, np.zeros((8, 128), np.float32))
    with pytest.raises(RuntimeError):
        b.push(1, np.zeros(1600, np.float32))
    with pytest.raises(RuntimeError):
        b.gpu_frontend(False)
    b.reset_stream(1)
    b.push(1, np.zeros(1600, np.float32))
    b.close()


@pytest.mark.parametrize("device_loop", [True, False])
@pytest.mark.parametrize("bias,lang,latency", [(0.7, "en-US", 560), (0.6, "auto", 160), (0.7, "auto", 1120)])
def test_batch_blank_biased(bias, lang, latency, device_loop):
    """Blank-biased tiny models (the settings of the r6_blank07 / r1_blank06 fixtures): both batched
    greedy loops must take the blank branches (symbol reset, first non-blank frame wins, later
    frames redone, a prediction carried into the next chunk) and give the oracle's tokens."""
    import nemoasr

    mdir = model_dir("tiny", 0, bias)
    om = oracle.Model(mdir, lang)
    secs = [2.0, 1.5, 2.6, 0.9, 1.8]
    mels = [mel_ref.logmel(synth.make_audio(t, seed=14 + 7 * i)) for i, t in enumerate(secs)]
    b = nemoasr.Batch(mdir, lang, latency, streams=len(mels))
    b.device_decoder(device_loop)
    b.set_dump(True)
    drive(b, mels, [0, 1, 0, 2, 1], piece=8 * (LAT_RIGHT[latency] + 1))
    check_streams(b, om, latency, mels, om.dims.joint_hidden, tag=("blank", bias, lang, latency))
    st = b.stats()
    assert 0 < st["tokens"] < st["rows"] * om.dims.max_symbols, st
    b.close()


@pytest.mark.parametrize("latency", [1120, 560])
def test_batch_auto_prompt_full(latency):
    """Full model with the language auto-detect prompt (the one-hot folded into the first prompt
    layer's bias, src/model.c:312-322), staggered streams, against the oracle."""
    import nemoasr

    mdir = model_dir("full")
    om = oracle.Model(mdir, "auto")
    secs = [2.5, 1.6, 2.9]
    mels = [mel_ref.logmel(synth.make_audio(t, seed=900 + i)) for i, t in enumerate(secs)]
    b = nemoasr.Batch(mdir, "auto", latency, streams=len(mels))
    b.set_dump(True)
    drive(b, mels, [0, 2, 1], piece=8 * (LAT_RIGHT[latency] + 1))
    check_streams(b, om, latency, mels, om.dims.joint_hidden, tag=("auto", latency))
    b.close()


def test_batch_skewed_auto_full():
    """The full model skewed as in the 256-stream benchmark workload (auto prompt, P(blank) ~ 0.7),
    five staggered streams at 1120 ms through the device-resident batched loop, against the oracle."""
    import nemoasr
    from conftest import SKEW_B256

    mdir = model_dir("full", 0, *SKEW_B256)
    om = oracle.Model(mdir, "auto")
    secs = [3.0, 2.2, 3.4, 1.5, 2.8]
    mels = [mel_ref.logmel(synth.make_audio(t, seed=1000 + i)) for i, t in enumerate(secs)]
    b = nemoasr.Batch(mdir, "auto", 1120, streams=len(mels))
    b.set_dump(True)
    drive(b, mels, [0, 1, 2, 0, 3], piece=8 * 14)
    check_streams(b, om, 1120, mels, om.dims.joint_hidden, tag=("skew256",))
    st = b.stats()
    assert 0 < st["tokens"] < st["rows"] * om.dims.max_symbols, st
    b.close()


def test_batch_single_stream_and_empty_steps():
    """A batch of one stream equals the oracle; steps with nothing ready (before any push, after
    the end) run nothing and return 0."""
    import nemoasr

    mdir = model_dir("tiny")
    b = nemoasr.Batch(mdir, "en-US", 560, 1)
    assert b.step() == 0 and b.run() == 0
    audio = synth.make_audio(2.0, seed=47)
    om = oracle.Model(mdir, "en-US")
    o = oracle.Session(om, 6)
    o.feed_mel(mel_ref.logmel(audio), final=True)
    b.push(0, audio, final=True)
    b.run()
    check_tokens(b.tokens(0), o.tokens, o.token_margins(), rerun=o.replayer())
    assert b.step() == 0 and b.stats()["chunks"] == o.chunks
    b.close()


def test_batch64_full_model_rows448():
    """The 64-stream, 560 ms workload at its real row count, end to end with the full model: stream
    s starts at step s % 8 and takes 8 - s % 8 chunks (tests/golden/make_batch64.py), so at step 7
    all 64 streams run a chunk in one batched step (448 encoder rows per GEMM) with 0 to 7 chunks
    of cache history each.  Every stream's tokens against the oracle's (committed fixture, the tie
    rule replaying the oracle only if a tie occurs) and two joint.enc rows per stream (1e-3)."""
    import os

    import nemoasr

    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "batch64_560.npz"))
    mdir = model_dir("full")
    S, piece = 64, 56
    mels = [mel_ref.logmel(synth.make_audio((8 - s % 8) * 0.56, seed=6400 + s)) for s in range(S)]
    b = nemoasr.Batch(mdir, "en-US", 560, streams=S)
    b.set_dump(True)
    pos, tick, step_rows = [0] * S, 0, []
    while any(p < m.shape[0] for p, m in zip(pos, mels)):
        for s, m in enumerate(mels):
            if tick < s % 8 or pos[s] >= m.shape[0]:
                continue
            end = min(pos[s] + piece, m.shape[0])
            if m.shape[0] - end < 8:  # the frame left over by the mel framing goes with the last chunk
                end = m.shape[0]
            b.push_mel(s, m[pos[s]:end], final=end >= m.shape[0])
            pos[s] = end
        rows0 = b.stats()["rows"]
        n = b.step()
        step_rows.append((n, b.stats()["rows"] - rows0))
        tick += 1
    b.run()
    print(f"  (streams, rows) per step: {step_rows}", flush=True)
    assert (64, 448) in step_rows
    om = None
    J = 640
    for s in range(S):
        toks = g["tokens"][g["offsets"][s]:g["offsets"][s + 1]].astype(int).tolist()
        margins = g["margins"][g["margin_offsets"][s]:g["margin_offsets"][s + 1]]
        je = b.joint_enc(s, J)
        fr = g["joint_enc_frames"][s]
        assert je.shape[0] == fr[1] + 1, (s, je.shape)
        assert rel_err(je[fr], g["joint_enc"][s]) <= 1e-3, s

        def rerun(forced, s=s):
            nonlocal om
            om = om or oracle.Model(mdir, "en-US")
            o = oracle.Session(om, LAT_RIGHT[560])
            o.feed_mel(mels[s], final=True)
            return o.replayer()(forced)

        check_tokens(b.tokens(s), toks, margins, f"stream {s}: ", rerun=rerun)
    b.close()
