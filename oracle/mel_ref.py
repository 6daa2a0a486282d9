"""ORACLE — test infrastructure only.

numpy restatement of the log-mel front end of nemoasr-c (reference src/mel.c, constants in
src/mel.h:8-13):
  pre-emphasis 0.97 (mel.c:148-153), symmetric Hann(400) centred in a 512-point FFT (mel.c:86-88),
  10 ms hop, centred frames with reflect padding and no edge repeat (mel.c:129-138, :169-176),
  power spectrum from a double-precision FFT cast to f32 (mel.c:175-176), 128 Slaney mel bins with
  Slaney area normalisation (mel.c:50-80), log(x + 2^-24) (mel.c:32, :182).

The streaming front end emits frame t only once every sample it reads is present (mel.c:156-158),
so its frames equal the whole-clip computation below; the final flush adds the frames that read
past the end with reflection (mel.c:157).
"""
from __future__ import annotations

import numpy as np

SR, NFFT, WIN, HOP, NMEL = 16000, 512, 400, 160, 128
NFREQ = NFFT // 2 + 1
LOG_GUARD = np.float32(2.0 ** -24)


def hz_to_mel(f):
    f = np.asarray(f, dtype=np.float64)
    f_sp, min_log_hz = 200.0 / 3.0, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0
    m = f / f_sp
    return np.where(f >= min_log_hz, min_log_mel + np.log(np.maximum(f, 1e-30) / min_log_hz) / logstep, m)


def mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    f_sp, min_log_hz = 200.0 / 3.0, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0
    return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), f_sp * m)


def filterbank() -> np.ndarray:
    """[NMEL][NFREQ] f32 triangular Slaney filters with 2/(f_{m+2}-f_m) normalisation."""
    freqs = (SR / 2) * np.arange(NFREQ, dtype=np.float64) / (NFREQ - 1)
    lo, hi = hz_to_mel(0.0), hz_to_mel(SR / 2.0)
    f_pts = mel_to_hz(lo + (hi - lo) * np.arange(NMEL + 2, dtype=np.float64) / (NMEL + 1))
    fb = np.zeros((NMEL, NFREQ), dtype=np.float32)
    for m in range(NMEL):
        enorm = 2.0 / (f_pts[m + 2] - f_pts[m])
        down = (freqs - f_pts[m]) / (f_pts[m + 1] - f_pts[m])
        up = (f_pts[m + 2] - freqs) / (f_pts[m + 2] - f_pts[m + 1])
        fb[m] = (np.maximum(np.minimum(down, up), 0.0) * enorm).astype(np.float32)
    return fb


def window() -> np.ndarray:
    w = np.zeros(NFFT, dtype=np.float32)
    n = np.arange(WIN, dtype=np.float64)
    left = (NFFT - WIN) // 2
    w[left:left + WIN] = (0.5 * (1.0 - np.cos(2.0 * np.pi * n / (WIN - 1)))).astype(np.float32)
    return w


def preemphasis(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    y = np.empty_like(x)
    if x.size:
        y[0] = x[0]
        y[1:] = x[1:] - np.float32(0.97) * x[:-1]
    return y


def logmel(x: np.ndarray, final: bool = True) -> np.ndarray:
    """All frames the streaming front end emits for the whole clip x (final=True), or the frames
    available before the final flush (final=False)."""
    y = preemphasis(x)
    N = y.size
    if N == 0:
        return np.zeros((0, NMEL), dtype=np.float32)
    nfr = N // HOP + 1 if final else (max(N - NFFT // 2, -1) // HOP + 1 if N >= NFFT // 2 else 0)
    if nfr <= 0:
        return np.zeros((0, NMEL), dtype=np.float32)
    g = (np.arange(nfr)[:, None] * HOP - NFFT // 2) + np.arange(NFFT)[None, :]
    g = np.where(g < 0, -g, g)
    g = np.where(g >= N, 2 * N - 2 - g, g)
    valid = (g >= 0) & (g < N)
    frames = np.where(valid, y[np.clip(g, 0, N - 1)], np.float32(0))
    frames = (frames * window()[None, :]).astype(np.float32).astype(np.float64)
    spec = np.fft.rfft(frames, axis=1)
    power = (spec.real ** 2 + spec.imag ** 2).astype(np.float32)
    acc = (power.astype(np.float64) @ filterbank().astype(np.float64).T).astype(np.float32)
    return np.log(acc + LOG_GUARD).astype(np.float32)
