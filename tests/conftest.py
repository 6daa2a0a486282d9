import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "nemo-c_amd"), os.path.join(REPO, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

MODEL_CACHE = os.environ.get("NEMO_MODEL_CACHE", "/tmp/nemo_models")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: full-size model on the CPU oracle")


# GPU files in the order their evidence builds on each other: per-kernel parity first, then the
# single stream end to end, then the multi-stream batch (built from the same kernels), then the
# allocation-free entry point; so that under -x a failure in a later layer cannot hide the
# foundational results.  Files not listed keep their place ahead of these.
_FILE_ORDER = {"test_golden.py": 0, "test_gpu_kernels.py": 1, "test_gpu_split.py": 1, "test_gpu_refabi.py": 1,
               "test_gpu_stream.py": 2, "test_gpu_determinism.py": 3,
               "test_gpu_batch.py": 4, "test_zz_no_alloc.py": 5}


def pytest_collection_modifyitems(session, config, items):
    items.sort(key=lambda it: _FILE_ORDER.get(os.path.basename(str(it.fspath)), -1))


# Greedy decisions whose top-2 joint margin in the oracle is below TOKEN_TIE (absolute logit units)
# are float ties: the GPU sums in another order (MFMA blocks, wavefront reductions), so the winner of
# such a decision may differ.  Measured oracle margins: median 0.1 (tiny model) / 0.5 (full), 1% below
# 2e-3; the two flips seen on the GPU were at 3.9e-6 and 2.8e-6.
TOKEN_TIE = 1e-4
MAX_TIES = 8

# decodes compared, ties followed to the end of the stream, ties where a comparison had to stop
TIE_STATS = {"decodes": 0, "ties_followed": 0, "ties_stopped": 0}


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    if TIE_STATS["decodes"]:
        terminalreporter.write_line(
            f"token parity: {TIE_STATS['decodes']} decodes compared with the oracle; float ties taken on the GPU's side "
            f"and compared to the end: {TIE_STATS['ties_followed']}; comparisons stopped at a tie: "
            f"{TIE_STATS['ties_stopped']}")


def check_oracle(got, o, what=""):
    """check_tokens against an oracle.Session, with its replay for ties (followed to the end)."""
    return check_tokens(got, o.tokens, o.token_margins(), what, rerun=o.replayer())


def _first_diff(got, ref):
    return next(i for i, (a, b) in enumerate(zip(got + [-1], ref + [-2])) if a != b)


def check_tokens(got, ref, margins, what="", rerun=None):
    """Token ids must equal the oracle's.  The only exception is a float tie: at the first differing
    position k the oracle's decisions that produced its token k (the blank frames since token k-1 and
    the emitting frame; past the last token, the trailing decisions) must include one with a top-2
    margin below TOKEN_TIE.
    With `rerun` (oracle.Session.replayer), the comparison goes on to the end of the stream: the oracle is
    replayed with that decision forced to its runner-up (the GPU's side of the tie), and the GPU's
    tokens must equal the replay's, up to MAX_TIES such ties.  Without it the comparison stops at the
    tie (counted as stopped).  Returns the number of ties taken, or None when the first comparison
    is already identical."""
    TIE_STATS["decodes"] += 1
    got, ref = list(got), list(ref)
    if got == ref:
        return None
    if rerun is None:
        k = _first_diff(got, ref)
        m = float(margins[min(k, len(margins) - 1)])
        msg = (f"{what}tokens differ at {k} of {len(ref)} (gpu {got[k] if k < len(got) else 'end'}, "
               f"oracle {ref[k] if k < len(ref) else 'end'}); oracle decision margin {m:.3g}, tie bound {TOKEN_TIE:g}")
        print(msg, flush=True)
        assert m < TOKEN_TIE, msg
        TIE_STATS["ties_stopped"] += 1
        return 1
    forced = {}
    while True:
        toks, best, second, margin, blank = rerun(forced)
        if got == toks:
            print(f"{what}{len(forced)} float tie(s) taken on the GPU's side; tokens equal to the end", flush=True)
            TIE_STATS["ties_followed"] += len(forced)
            return len(forced)
        k = _first_diff(got, toks)
        emit = [j for j, b in enumerate(best) if b != blank]
        lo = emit[k - 1] + 1 if k > 0 else 0
        hi = emit[k] + 1 if k < len(emit) else len(best)
        ties = [j for j in range(lo, hi) if margin[j] < TOKEN_TIE and j not in forced]
        msg = (f"{what}tokens differ at {k} of {len(toks)} (gpu {got[k] if k < len(got) else 'end'}, "
               f"oracle {toks[k] if k < len(toks) else 'end'}) after {len(forced)} tie(s); smallest margin of the "
               f"decisions {lo}..{hi - 1}: {float(min(margin[lo:hi], default=np.inf)):.3g}, tie bound {TOKEN_TIE:g}")
        print(msg, flush=True)
        assert ties and len(forced) < MAX_TIES, msg
        forced[ties[0]] = int(second[ties[0]])


def model_dir(kind: str, seed: int = 0, blank_bias: float = 0.0, label_shift: float = 0.0) -> str:
    import synth

    dims = synth.TINY_DIMS if kind == "tiny" else synth.FULL_DIMS
    d = os.path.join(MODEL_CACHE, f"{kind}_s{seed}_b{blank_bias:g}" + (f"_l{label_shift:g}" if label_shift else ""))
    synth.write_model(d, dims, seed, blank_bias, label_shift)
    return d


# joint-bias skews of the skewed benchmark workloads (bench.py): one stream at 1120 ms with
# P(blank) ~ 0.5, and 256 streams with the auto prompt at P(blank) ~ 0.7
SKEW_S1120 = (2.0, 0.0188)
SKEW_B256 = (2.0, 0.0619)


@pytest.fixture(scope="session")
def tiny_model_dir():
    return model_dir("tiny")


@pytest.fixture(scope="session")
def full_model_dir():
    return model_dir("full")


@pytest.fixture(scope="session")
def tiny_oracle(tiny_model_dir):
    import oracle

    return oracle.Model(tiny_model_dir, "en-US")


@pytest.fixture(scope="session")
def gpu():
    import nemoasr

    g = nemoasr.Gpu()
    yield g
    g.close()


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    """max |a - b| / max |b| (the reference's encoder gate, tools/compare.py:30-32)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = max(float(np.max(np.abs(b))) if b.size else 0.0, 1e-30)
    return float(np.max(np.abs(a - b))) / den if b.size else 0.0


# ---- the product's decoder pieces, driven one kernel at a time ---------------------------------
def lstm_cell_rows(gpu, gates: np.ndarray, c_in: np.ndarray):
    """The LSTM cell of the batched greedy loop (nk_lstm_cell_rows, kernel lstm_cell_rows) on one
    row: gates [4H] (i, f, g, o), c_in [H] -> (c_out, h_out)."""
    import nemoasr

    L = nemoasr.lib()
    H = c_in.size
    hc = np.zeros((3, H), np.float32)
    hc[0] = c_in
    dg, dhc, dout = gpu.put(np.ascontiguousarray(gates, np.float32)), gpu.put(hc), gpu.alloc(H * 4)
    rows = [gpu.put(np.array([i], np.int32)) for i in (0, 1, 2)]
    gpu.begin()
    gpu.check(L.nk_lstm_cell_rows(gpu.h, dg.ptr, dhc.ptr, rows[0].ptr, rows[1].ptr, rows[2].ptr, dout.ptr, 1, H))
    gpu.end()
    out = dhc.read((3, H))
    np.testing.assert_array_equal(dout.read(H), out[2])
    return out[1], out[2]


def joint_argmax_rows(gpu, enc: np.ndarray, pred: np.ndarray, W: np.ndarray, bias: np.ndarray, device_loop: bool):
    """argmax_n W[n] . relu(enc[r] + pred) + bias[n] for every row r of enc, through the batched
    loop's kernels: joint_in_rows, then either the joint GEMM with the argmax-key epilogue
    (gemm_mx64x64_argmax, the device loop; the keys of each row reduced here) or the joint GEMM into
    logits and argmax_rows (the host loop).  Operands are zero-padded to the kernels' multiples,
    which changes no score.  Returns [(index, value)] per row."""
    import nemoasr

    L = nemoasr.lib()
    R, J = enc.shape
    V = W.shape[0]
    Jp, N = -(-J // 32) * 32, -(-V // 64) * 64
    Wp = np.zeros((N, Jp), np.uint16)
    Wp[:V, :J] = W
    bp = np.zeros(N, np.float32)
    bp[:V] = bias
    ep = np.zeros((R, Jp), np.float32)
    ep[:, :J] = enc
    pp = np.zeros((1, Jp), np.float32)
    pp[0, :J] = pred
    de, dp, dW, db = gpu.put(ep), gpu.put(pp), gpu.put(Wp), gpu.put(bp)
    erow, prow = gpu.put(np.arange(R, dtype=np.int32)), gpu.put(np.zeros(R, np.int32))
    jin = gpu.alloc(R * Jp * 4)
    gpu.begin()
    gpu.check(L.nk_joint_in_rows(gpu.h, de.ptr, dp.ptr, erow.ptr, prow.ptr, jin.ptr, R, Jp))
    if device_loop:
        parts = N // 32
        keys = gpu.alloc(R * parts * 8)
        gpu.check(L.nk_gemm_argmax(gpu.h, jin.ptr, Jp, dW.ptr, Jp, db.ptr, keys.ptr, parts, R, N, Jp, V))
    else:
        logits, out = gpu.alloc(R * N * 4), gpu.alloc(2 * R * 4)
        gpu.check(L.nk_gemm(gpu.h, jin.ptr, Jp, dW.ptr, Jp, db.ptr, logits.ptr, N, R, N, Jp, 0, 0, 1.0))
        gpu.check(L.nk_argmax_rows(gpu.h, logits.ptr, N, R, V, out.ptr))
    gpu.end()
    res = []
    if device_loop:
        k = keys.read((R, parts), np.uint64).max(axis=1)
        for best in k:
            best = int(best)
            idx = 0xFFFFFFFF - (best & 0xFFFFFFFF)
            ordv = best >> 32
            bits = ordv & 0x7FFFFFFF if ordv & 0x80000000 else (~ordv) & 0xFFFFFFFF
            res.append((idx, float(np.array([bits], np.uint32).view(np.float32)[0])))
    else:
        o = out.read(2 * R, np.int32)
        for r in range(R):
            res.append((int(o[2 * r]), float(o[2 * r + 1:2 * r + 2].view(np.float32)[0])))
    return res
