"""The persistent encoder chain of one-row chunks (80 ms latency, kernels/nk_chain.hip) against
the oracle and against the per-kernel sequence it replaces.

The chain runs all 24 conformer blocks of a chunk in one launch of 256 resident workgroups that
hand each block's intermediate rows to one another; its arithmetic is the per-kernel path's with
other summation orders, so it is held to the same gates as every other path (per-layer 2e-3,
joint.enc 1e-3, tokens identical up to float ties, conftest.check_oracle) and, against the
per-kernel sequence on the same input, to float rounding.
"""
import numpy as np
import pytest

import mel_ref
import oracle
import synth
from conftest import check_oracle, model_dir, rel_err

pytestmark = pytest.mark.gpu

RIGHT_80MS = 0


def run_session(mdir, mel, chain, dump=True, graphs=False, step=None):
    import nemoasr

    s = nemoasr.Session(mdir, "en-US", 80)
    s.chain(chain)
    s.set_dump(dump)
    s.use_graphs(graphs)
    n0 = s.launches()
    step = step or mel.shape[0]
    for i in range(0, mel.shape[0], step):
        s.feed_mel(mel[i:i + step], final=i + step >= mel.shape[0])
    return s, s.launches() - n0


def test_chain_usable_on_full_model():
    import nemoasr

    s = nemoasr.Session(model_dir("full"), "en-US", 80)
    assert s.chain_usable()
    s.close()
    t = nemoasr.Session(model_dir("tiny"), "en-US", 80)
    assert not t.chain_usable()  # d_model 256: the per-kernel sequence
    t.close()


def test_chain_per_layer_parity():
    """Every block output, the prompted rows and joint.enc of 2 s at 80 ms against the oracle; the
    chain replaces ~190 launches per one-row chunk by one."""
    mdir = model_dir("full")
    om = oracle.Model(mdir, "en-US")
    d = om.dims
    mel = mel_ref.logmel(synth.make_audio(2.0, seed=3))
    o = oracle.Session(om, RIGHT_80MS, dump=True)
    o.feed_mel(mel, final=True)
    s, n_on = run_session(mdir, mel, chain=True)
    gl, gp, gj = s.dumps(d.n_layers, d.d_model, d.joint_hidden)
    ol, op, oj, rows = o.dumps()
    assert gl.shape == ol.shape, (gl.shape, ol.shape)
    errs = [rel_err(gl[:, l], ol[:, l]) for l in range(d.n_layers)]
    print("per-layer max rel err:", " ".join(f"{e:.1e}" for e in errs))
    assert max(errs) <= 2e-3, errs
    assert rel_err(gp, op) <= 2e-3
    assert rel_err(gj, oj) <= 1e-3
    check_oracle(s.tokens(), o)
    frames = gl.shape[0]
    s.close()
    s2, n_off = run_session(mdir, mel, chain=False)
    s2.close()
    print(f"launches: chain {n_on}, per-kernel {n_off}, {frames} frames")
    assert n_off - n_on >= 150 * (frames - 4), (n_on, n_off, frames)


def test_chain_matches_per_kernel():
    """Chain and per-kernel sequence on the same mel frames: every layer within float rounding of
    each other, the same tokens as the oracle."""
    mdir = model_dir("full")
    om = oracle.Model(mdir, "en-US")
    d = om.dims
    mel = mel_ref.logmel(synth.make_audio(1.5, seed=21))
    o = oracle.Session(om, RIGHT_80MS)
    o.feed_mel(mel, final=True)
    out = []
    for chain in (True, False):
        s, _ = run_session(mdir, mel, chain=chain)
        out.append((s.tokens(), s.dumps(d.n_layers, d.d_model, d.joint_hidden)))
        s.close()
    (tc, (lc, pc, jc)), (tk, (lk, pk, jk)) = out
    check_oracle(tc, o, "chain: ")
    check_oracle(tk, o, "per-kernel: ")
    errs = [rel_err(lc[:, l], lk[:, l]) for l in range(d.n_layers)]
    print("chain vs per-kernel, per layer:", " ".join(f"{e:.1e}" for e in errs))
    assert max(errs) < 1e-4 and rel_err(jc, jk) < 1e-4


def test_chain_graph_replay_fed_in_pieces():
    """The chain inside the replayed chunk graph, audio fed 7 mel frames at a time: every chunk's
    descriptor (position, cache length, epoch) is read on the device, so one graph serves them all;
    tokens against the oracle."""
    mdir = model_dir("full")
    om = oracle.Model(mdir, "en-US")
    mel = mel_ref.logmel(synth.make_audio(3.0, seed=5))
    o = oracle.Session(om, RIGHT_80MS)
    o.feed_mel(mel, final=True)
    s, _ = run_session(mdir, mel, chain=True, dump=False, graphs=True, step=7)
    check_oracle(s.tokens(), o)
    s.close()


def test_chain_repeatable():
    """Two sessions on the same input: identical block outputs (the chain's sums have a fixed
    order; which workgroup finishes first changes nothing)."""
    mdir = model_dir("full")
    om = oracle.Model(mdir, "en-US")
    d = om.dims
    mel = mel_ref.logmel(synth.make_audio(1.0, seed=8))
    res = []
    for _ in range(2):
        s, _ = run_session(mdir, mel, chain=True)
        res.append(s.dumps(d.n_layers, d.d_model, d.joint_hidden)[0].copy())
        s.close()
    assert np.array_equal(res[0], res[1])


def test_chain_timeout_is_an_error():
    """The failure path of the chain's bounded waits, forced from the host: with a hand-off bound
    of one poll the first launch gives up (every workgroup leaves at its next barrier or wait, no
    wait is unbounded) and the session reports the time-out as an error; a session opened after
    it computes the same block outputs as one that never timed out."""
    import nemoasr

    mdir = model_dir("full")
    om = oracle.Model(mdir, "en-US")
    d = om.dims
    mel = mel_ref.logmel(synth.make_audio(1.0, seed=13))
    s = nemoasr.Session(mdir, "en-US", 80)
    s.chain(True)
    s.use_graphs(False)
    s.chain_spin(1)
    with pytest.raises(RuntimeError, match="encoder chain: hand-off [0-9]+ timed out"):
        s.feed_mel(mel, final=True)
    s.close()
    outs = []
    for _ in range(2):
        t, _ = run_session(mdir, mel, chain=True)
        outs.append(t.dumps(d.n_layers, d.d_model, d.joint_hidden)[0].copy())
        t.close()
    assert np.array_equal(outs[0], outs[1])
