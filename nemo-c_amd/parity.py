"""Real-checkpoint parity harness: one WAV file through the library, checked against a directory
of MLX reference dumps.

It joins two pieces of the reference's parity tooling:
  - the dumps its CLI writes with --dump-mel / --dump-enc / --dump-tokens (src/main.c:99, :112,
    :128, :209-211): the front end's log-mel frames, the post-prompt encoder rows of every chunk,
    the emitted token ids.  `run` produces the same three artefacts through the public C API of
    this library (nemoasr_open / nemoasr_feed) and its dump hooks, feeding the file the way the
    CLI does (src/main.c:230-252): pieces of one chunk of audio, the last one final;
  - the comparison of those dumps with the MLX reference directory (tools/compare.py:1-45),
    with the same gates: log-mel max |diff| < 1e-3 with equal shapes, encoder rows
    max |diff| / max |ref| < 1e-2 with equal shapes, token ids identical.

Reference directory (written by the reference's tools/mlx_reference.py:94-126):
    mel.f32      (T, 128) float32        enc_all.f32  (rows, d_model) float32
    tokens.txt   line 1: ids separated by spaces, line 2: the text      meta.json
Dump directory (the CLI's format, written by `write_dumps`):
    mel.f32      (T, 128) float32        enc.f32      (rows, d_model) float32
    tokens.txt   one id per line

One difference from tools/compare.py: a dump directory with none of the three files fails
(compare.py reports success when it finds nothing to compare).

Usage:
    python parity.py compare REF_DIR OUT_DIR [--d-model 1024]
    python parity.py run --model-dir DIR --wav FILE --out OUT_DIR [--ref REF_DIR]
                         [--latency 560] [--language en-US]
"""
from __future__ import annotations

import argparse
import json
import os
import struct
import sys

import numpy as np

N_MEL = 128
LATENCIES = (80, 160, 320, 560, 1120)
MEL_GATE = 1e-3   # tools/compare.py:21
ENC_GATE = 1e-2   # tools/compare.py:31


# ---- WAV input (src/wav.c:10-62) --------------------------------------------------------------

def read_wav_mono(path: str) -> tuple[int, np.ndarray]:
    """(sample rate, float32 mono samples) of a RIFF/WAVE file: PCM 16, 24 or 32 bit, or IEEE
    float 32 bit, WAVE_FORMAT_EXTENSIBLE resolved to its sub-format; channels averaged in double
    precision; a data chunk running past the end of the file is cut at the end (src/wav.c)."""
    with open(path, "rb") as f:
        buf = f.read()
    if len(buf) < 12:
        raise ValueError("not a WAV file")
    if buf[0:4] != b"RIFF" or buf[8:12] != b"WAVE":
        raise ValueError("not a RIFF/WAVE file")
    fmt = channels = bits = rate = 0
    data = None
    pos = 12
    while pos + 8 <= len(buf):
        cid = buf[pos:pos + 4]
        clen = struct.unpack_from("<I", buf, pos + 4)[0]
        body = pos + 8
        if cid == b"fmt ":
            fmt, channels, rate = struct.unpack_from("<HHI", buf, body)
            bits = struct.unpack_from("<H", buf, body + 14)[0]
            if fmt == 0xFFFE and clen >= 26:
                fmt = struct.unpack_from("<H", buf, body + 24)[0]
        elif cid == b"data":
            data = buf[body:min(body + clen, len(buf))]
        pos += 8 + clen + (clen & 1)
    if data is None or channels <= 0 or bits <= 0:
        raise ValueError("missing fmt/data chunk")
    if not ((fmt == 1 and bits in (16, 24, 32)) or (fmt == 3 and bits == 32)):
        raise ValueError(f"unsupported WAV format {fmt} / {bits} bits")
    bps = bits // 8
    frames = len(data) // (bps * channels)
    raw = np.frombuffer(data, dtype=np.uint8, count=frames * channels * bps)
    if fmt == 3:
        v = raw.view("<f4").astype(np.float64)
    elif bits == 16:
        v = raw.view("<i2").astype(np.float64) / 32768.0
    elif bits == 24:
        b = raw.reshape(-1, 3).astype(np.int32)
        x = (b[:, 0] << 8) | (b[:, 1] << 16) | (b[:, 2] << 24)   # sign lands in bit 31
        v = (x >> 8).astype(np.float64) / 8388608.0
    else:
        v = raw.view("<i4").astype(np.float64) / 2147483648.0
    v = v.reshape(frames, channels)
    acc = v[:, 0].copy()
    for ch in range(1, channels):   # channel order, like the C loop
        acc += v[:, ch]
    return int(rate), (acc / channels).astype(np.float32)


# ---- running the library ----------------------------------------------------------------------

def _dims(model_dir: str) -> tuple[int, int, int]:
    with open(os.path.join(model_dir, "config.json")) as f:
        cfg = json.load(f)
    e, j = cfg.get("encoder", {}), cfg.get("joint", {})
    return int(e.get("n_layers", 24)), int(e.get("d_model", 1024)), int(j.get("joint_hidden", 640))


def run(model_dir: str, wav: str, latency_ms: int = 560, language: str = "en-US") -> dict:
    """Transcribe `wav` with dumps on.  Returns mel (T, 128), enc (rows, d_model), tokens, text."""
    import nemoasr

    if latency_ms not in LATENCIES:
        raise ValueError(f"latency must be one of {LATENCIES}")
    rate, audio = read_wav_mono(wav)
    n_layers, d_model, joint_hidden = _dims(model_dir)
    s = nemoasr.Session(model_dir, language, latency_ms, rate)
    try:
        s.set_dump(True)
        piece = max(1, latency_ms * rate // 1000)   # one chunk of audio (src/main.c:230)
        text = ""
        if audio.size == 0:
            text += s.feed(audio, final=True)
        for pos in range(0, audio.size, piece):
            text += s.feed(audio[pos:pos + piece], final=pos + piece >= audio.size)
        _, prompted, _ = s.dumps(n_layers, d_model, joint_hidden)
        return {"mel": s.mel_dump(), "enc": prompted, "tokens": s.tokens(), "text": text,
                "d_model": d_model}
    finally:
        s.close()


def write_dumps(out_dir: str, mel: np.ndarray, enc: np.ndarray, tokens: list[int]) -> None:
    """The CLI's dump files (src/main.c:99, :112, :128)."""
    os.makedirs(out_dir, exist_ok=True)
    np.ascontiguousarray(mel, dtype=np.float32).tofile(os.path.join(out_dir, "mel.f32"))
    np.ascontiguousarray(enc, dtype=np.float32).tofile(os.path.join(out_dir, "enc.f32"))
    with open(os.path.join(out_dir, "tokens.txt"), "w") as f:
        for t in tokens:
            f.write(f"{int(t)}\n")


# ---- comparison (tools/compare.py:1-45) -------------------------------------------------------

def _load(path: str, cols: int) -> np.ndarray:
    a = np.fromfile(path, dtype=np.float32)
    if a.size % cols:
        raise ValueError(f"{path}: {a.size} floats is not a whole number of {cols}-wide rows")
    return a.reshape(-1, cols)


def compare(ref_dir: str, out_dir: str, d_model: int = 1024) -> tuple[bool, list[str]]:
    """Check the dumps in `out_dir` against the reference directory.  Returns (ok, report)."""
    ok, seen, rep = True, 0, []
    p = os.path.join(out_dir, "mel.f32")
    if os.path.exists(p):
        seen += 1
        rm, cm = _load(os.path.join(ref_dir, "mel.f32"), N_MEL), _load(p, N_MEL)
        if rm.shape == cm.shape:
            d = np.abs(rm - cm)
            mx = float(d.max()) if d.size else 0.0
            rep.append(f"mel: ref {rm.shape} ours {cm.shape} max abs diff {mx:.3e} mean "
                       f"{float(d.mean()) if d.size else 0.0:.3e}")
            ok &= mx < MEL_GATE
        else:
            rep.append(f"mel: ref {rm.shape} ours {cm.shape} SHAPE MISMATCH")
            ok = False
    p = os.path.join(out_dir, "enc.f32")
    if os.path.exists(p):
        seen += 1
        re_, ce = _load(os.path.join(ref_dir, "enc_all.f32"), d_model), _load(p, d_model)
        n = min(len(re_), len(ce))
        if n:
            d = np.abs(re_[:n] - ce[:n])
            rel = float(d.max()) / (float(np.abs(re_[:n]).max()) + 1e-9)
            rep.append(f"enc: ref {re_.shape} ours {ce.shape} max abs diff {float(d.max()):.3e} "
                       f"(rel {rel:.2e}) mean {float(d.mean()):.3e}")
            ok &= rel < ENC_GATE and re_.shape == ce.shape
        else:
            rep.append(f"enc: ref {re_.shape} ours {ce.shape} no rows")
            ok = False
    p = os.path.join(out_dir, "tokens.txt")
    if os.path.exists(p):
        seen += 1
        with open(os.path.join(ref_dir, "tokens.txt")) as f:
            rt = [int(x) for x in f.readline().split()]
        with open(p) as f:
            ct = [int(line) for line in f if line.strip()]
        same = rt == ct
        rep.append(f"tokens: ref {len(rt)} ours {len(ct)} identical={same}")
        if not same:
            first = next(i for i, (a, b) in enumerate(zip(rt + [None], ct + [None])) if a != b)
            a = rt[first] if first < len(rt) else "end"
            b = ct[first] if first < len(ct) else "end"
            rep.append(f"  first difference at {first}: ref {a} ours {b}")
        ok &= same
    if not seen:
        rep.append(f"{out_dir}: no mel.f32, enc.f32 or tokens.txt to compare")
        ok = False
    rep.append("PARITY OK" if ok else "PARITY FAILED")
    return ok, rep


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("compare", help="compare a dump directory with a reference directory")
    c.add_argument("ref_dir")
    c.add_argument("out_dir")
    c.add_argument("--d-model", type=int, default=1024)
    r = sub.add_parser("run", help="transcribe a WAV file with dumps, optionally compare")
    r.add_argument("--model-dir", required=True)
    r.add_argument("--wav", required=True)
    r.add_argument("--out", required=True)
    r.add_argument("--ref")
    r.add_argument("--latency", type=int, default=560, choices=LATENCIES)
    r.add_argument("--language", default="en-US")
    a = ap.parse_args(argv)
    if a.cmd == "compare":
        ok, rep = compare(a.ref_dir, a.out_dir, a.d_model)
    else:
        res = run(a.model_dir, a.wav, a.latency, a.language)
        write_dumps(a.out, res["mel"], res["enc"], res["tokens"])
        print(res["text"].strip())
        if not a.ref:
            return 0
        ok, rep = compare(a.ref, a.out, res["d_model"])
    print("\n".join(rep))
    return 0 if ok else 1


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    sys.exit(main())
