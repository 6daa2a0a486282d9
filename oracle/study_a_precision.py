#!/usr/bin/env python3
"""Numerics study on the oracle: what rounding the GEMMs' f32 activations (the A operand) to a
single bf16 does to the gates of this path, against the bf16 hi + lo pair the batched GPU GEMMs
feed their MFMAs, on clips of the five benchmark workloads (full random-init model).

For each clip the oracle decodes three times: A in f32 (the reference's arithmetic), A as bf16
hi + lo, and A as one bf16.  Reported per variant against f32: the largest per-layer encoder error
(max |d| / max |ref| of each layer's output rows, the 2e-3 gate), the joint.enc error (the 1e-3
gate), and whether the token ids are identical (first differing token and the f32 decode's decision
margin there).

Run from the repository root:  python oracle/study_a_precision.py   (about five minutes, 8 cores)
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
sys.path[:0] = [HERE, os.path.join(REPO, "nemo-c_amd")]

import mel_ref  # noqa: E402
import oracle  # noqa: E402
import synth  # noqa: E402

CACHE = os.environ.get("NEMO_MODEL_CACHE", "/tmp/nemo_models")
LAT_RIGHT = {80: 0, 560: 6, 1120: 13}
MODES = {0: "f32", 2: "bf16 hi+lo", 1: "bf16"}


def model(blank_bias=0.0, label_shift=0.0):
    d = os.path.join(CACHE, f"full_s0_b{blank_bias:g}" + (f"_l{label_shift:g}" if label_shift else ""))
    synth.write_model(d, synth.FULL_DIMS, 0, blank_bias, label_shift)
    return d


# (workload, latency, language, skew, seconds, audio seed)
CLIPS = [
    ("S80", 80, "en-US", (0.0, 0.0), 4.0, 0),
    ("S560", 560, "en-US", (0.0, 0.0), 10.0, 0),
    ("S1120 P(blank) 0.5", 1120, "en-US", (2.0, 0.0188), 12.0, 0),
    ("B64 stream", 560, "en-US", (0.0, 0.0), 6.0, 1000),
    ("B64 stream", 560, "en-US", (0.0, 0.0), 6.0, 1001),
    ("B256 stream, auto, P(blank) 0.7", 1120, "auto", (2.0, 0.0619), 8.0, 1000),
    ("B256 stream, auto, P(blank) 0.7", 1120, "auto", (2.0, 0.0619), 8.0, 1001),
]


def decode(om, right, mel, mode):
    oracle.lib().or_set_gemm_a_mode(mode)
    try:
        o = oracle.Session(om, right, dump=True)
        o.feed_mel(mel, final=True)
        lay, _, je, _ = o.dumps()
        return list(o.tokens), lay, je, o.token_margins()
    finally:
        oracle.lib().or_set_gemm_a_mode(0)


def rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b))) / max(float(np.max(np.abs(b))), 1e-30)


def main():
    models = {}
    rows = []
    t0 = time.time()
    for name, lat, lang, skew, secs, seed in CLIPS:
        key = (skew, lang)
        if key not in models:
            models[key] = oracle.Model(model(*skew), lang)
        om = models[key]
        mel = mel_ref.logmel(synth.make_audio(secs, seed=seed))
        ref_t, ref_l, ref_j, ref_m = decode(om, LAT_RIGHT[lat], mel, 0)
        for mode in (2, 1):
            t, lay, je, _ = decode(om, LAT_RIGHT[lat], mel, mode)
            layer_err = max(rel(lay[:, l], ref_l[:, l]) for l in range(lay.shape[1]))
            joint_err = rel(je, ref_j)
            if t == ref_t:
                tok = "identical"
            else:
                k = next(i for i, (a, b) in enumerate(zip(t + [-1], ref_t + [-2])) if a != b)
                tok = f"differ at token {k} of {len(ref_t)} (f32 decision margin {float(ref_m[min(k, len(ref_m) - 1)]):.3g})"
            rows.append((name, lat, secs, seed, MODES[mode], layer_err, joint_err, tok))
            print(f"{name:34s} {lat:5d} ms {secs:4.0f} s seed {seed:4d}  A {MODES[mode]:10s}  per-layer {layer_err:.2e}  "
                  f"joint.enc {joint_err:.2e}  tokens {tok}   [{time.time() - t0:.0f} s]", flush=True)
    print("\n| workload | clip | A operand | max per-layer error | joint.enc error | tokens |")
    print("|---|---|---|---|---|---|")
    for name, lat, secs, seed, mode, le, je, tok in rows:
        print(f"| {name} | {lat} ms, {secs:g} s, seed {seed} | {mode} | {le:.2e} | {je:.2e} | {tok} |")


if __name__ == "__main__":
    main()
