#!/usr/bin/env python3
"""Writes tests/golden/batch64_560.npz: the oracle's decode of the 64-stream, 560 ms workload at
its full row count, for tests/test_gpu_batch.py::test_batch64_full_model_rows448.

Stream s (of 64) starts at batch step s % 8 and is fed 8 - s % 8 chunks of 560 ms (its own seeded
synthetic audio, seed 6400 + s), so at step 7 every stream takes a chunk: 448 encoder rows in one
batched step, with streams holding 0 to 7 chunks of cache history (the cache fill levels of the
64-stream benchmark workload).  Model: the full random-init model (seed 0), prompt en-US.
Stored per stream: the token ids, the oracle's per-token decision margins (the tie rule of the
token check), and two joint.enc rows (frames 0 and the last frame) with their indices.

Run from the repository root (about two minutes on eight cores):  python tests/golden/make_batch64.py
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(REPO, "oracle"), os.path.join(REPO, "nemo-c_amd"), os.path.join(REPO, "tests")]

import mel_ref  # noqa: E402
import oracle  # noqa: E402
import synth  # noqa: E402
from conftest import model_dir  # noqa: E402

S, CHUNK_S, RIGHT = 64, 0.56, 6


def stream_audio(s: int) -> np.ndarray:
    return synth.make_audio((8 - s % 8) * CHUNK_S, seed=6400 + s)


def main():
    om = oracle.Model(model_dir("full"), "en-US")
    toks, offs, margins, je, je_idx = [], [0], [], [], []
    t0 = time.time()
    for s in range(S):
        mel = mel_ref.logmel(stream_audio(s))
        o = oracle.Session(om, RIGHT, dump=True)
        o.feed_mel(mel, final=True)
        _, _, oj, _ = o.dumps()
        toks += o.tokens
        offs.append(len(toks))
        margins.append(o.token_margins())
        idx = [0, oj.shape[0] - 1]
        je.append(oj[idx])
        je_idx.append(idx)
        print(f"stream {s}: {mel.shape[0]} mel rows, {oj.shape[0]} frames, {len(o.tokens)} tokens, "
              f"{time.time() - t0:.0f} s", flush=True)
    np.savez_compressed(os.path.join(HERE, "batch64_560.npz"), tokens=np.array(toks, np.int16),
                        offsets=np.array(offs, np.int32), margins=np.concatenate(margins).astype(np.float32),
                        margin_offsets=np.cumsum([0] + [m.size for m in margins]).astype(np.int32),
                        joint_enc=np.stack(je).astype(np.float32), joint_enc_frames=np.array(je_idx, np.int32))


if __name__ == "__main__":
    main()
