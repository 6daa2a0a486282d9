"""Host side of the real-checkpoint parity harness (nemo-c_amd/parity.py): the WAV reader against
closed-form sample values, and the comparison gates of the reference's tools/compare.py against
planted differences.  No GPU."""
import os
import struct
import wave

import numpy as np
import pytest

import parity


def _riff(fmt_body: bytes, data: bytes, extra_chunks: bytes = b"") -> bytes:
    chunks = b"fmt " + struct.pack("<I", len(fmt_body)) + fmt_body + extra_chunks
    chunks += b"data" + struct.pack("<I", len(data)) + data
    return b"RIFF" + struct.pack("<I", 4 + len(chunks)) + b"WAVE" + chunks


def _fmt(tag, channels, rate, bits):
    bps = bits // 8
    return struct.pack("<HHIIHH", tag, channels, rate, rate * channels * bps, channels * bps, bits)


def test_wav_pcm16_stereo_written_by_wave_module(tmp_path):
    p = str(tmp_path / "s16.wav")
    left = np.array([0, 32767, -32768, 1000, -1], np.int16)
    right = np.array([0, 32767, 0, -3000, -1], np.int16)
    with wave.open(p, "wb") as w:
        w.setnchannels(2)
        w.setsampwidth(2)
        w.setframerate(44100)
        w.writeframes(np.stack([left, right], 1).tobytes())
    rate, x = parity.read_wav_mono(p)
    assert rate == 44100
    want = ((left.astype(np.float64) / 32768 + right.astype(np.float64) / 32768) / 2).astype(np.float32)
    np.testing.assert_array_equal(x, want)
    assert x[1] == np.float32(32767 / 32768) and x[2] == np.float32(-0.5)


def test_wav_pcm24_and_pcm32_extremes(tmp_path):
    # 24-bit: 0x7fffff, 0x800000, 0x000001, 0xffffff -> +max, -1, 1 lsb, -1 lsb
    d24 = bytes([0xFF, 0xFF, 0x7F, 0x00, 0x00, 0x80, 0x01, 0x00, 0x00, 0xFF, 0xFF, 0xFF])
    p = tmp_path / "s24.wav"
    p.write_bytes(_riff(_fmt(1, 1, 16000, 24), d24))
    rate, x = parity.read_wav_mono(str(p))
    assert rate == 16000
    np.testing.assert_array_equal(x, np.float32([8388607 / 8388608, -1.0, 1 / 8388608, -1 / 8388608]))
    d32 = struct.pack("<4i", 2**31 - 1, -2**31, 1 << 16, -(1 << 30))
    p.write_bytes(_riff(_fmt(1, 1, 8000, 32), d32))
    _, x = parity.read_wav_mono(str(p))
    np.testing.assert_array_equal(x, np.float32([(2**31 - 1) / 2**31, -1.0, 2.0**-15, -0.5]))


def test_wav_float_extensible_odd_chunk_and_truncated_data(tmp_path):
    vals = np.float32([0.25, -0.75, 0.5, 0.125, 1.5, -2.0])
    # WAVE_FORMAT_EXTENSIBLE (0xFFFE) with IEEE-float sub-format 3 at byte 24 of the fmt body
    body = _fmt(0xFFFE, 2, 22050, 32) + struct.pack("<HHIH", 22, 32, 0x3, 3) + bytes(14)
    odd = b"LIST" + struct.pack("<I", 3) + b"abc" + b"\x00"   # odd-sized chunk, padded
    raw = _riff(body, vals.tobytes(), odd)
    p = tmp_path / "f32.wav"
    p.write_bytes(raw)
    rate, x = parity.read_wav_mono(str(p))
    assert rate == 22050
    np.testing.assert_array_equal(x, np.float32([(0.25 - 0.75) / 2, (0.5 + 0.125) / 2, (1.5 - 2.0) / 2]))
    p.write_bytes(raw[:-5])   # data chunk cut mid-frame: whole frames only
    _, x = parity.read_wav_mono(str(p))
    np.testing.assert_array_equal(x, np.float32([-0.25, 0.3125]))


def test_wav_rejects(tmp_path):
    p = tmp_path / "bad.wav"
    p.write_bytes(b"RIFX\x00\x00\x00\x00WAVE")
    with pytest.raises(ValueError, match="RIFF"):
        parity.read_wav_mono(str(p))
    p.write_bytes(_riff(_fmt(1, 1, 16000, 8), b"\x80\x80"))
    with pytest.raises(ValueError, match="unsupported"):
        parity.read_wav_mono(str(p))
    p.write_bytes(b"RIFF" + struct.pack("<I", 4) + b"WAVE")
    with pytest.raises(ValueError, match="missing"):
        parity.read_wav_mono(str(p))


def _ref_dir(root, mel, enc, toks, text="hello"):
    os.makedirs(root, exist_ok=True)
    mel.astype(np.float32).tofile(os.path.join(root, "mel.f32"))
    enc.astype(np.float32).tofile(os.path.join(root, "enc_all.f32"))
    with open(os.path.join(root, "tokens.txt"), "w") as f:
        f.write(" ".join(map(str, toks)) + "\n" + text + "\n")
    return root


@pytest.fixture
def dumps(tmp_path):
    g = np.random.default_rng(1)
    mel = g.standard_normal((40, 128)).astype(np.float32) * 3
    enc = g.standard_normal((5, 64)).astype(np.float32)
    toks = [5, 17, 3, 3, 90]
    ref = _ref_dir(str(tmp_path / "ref"), mel, enc, toks)
    return ref, str(tmp_path / "out"), mel, enc, toks


def test_compare_identical_passes(dumps):
    ref, out, mel, enc, toks = dumps
    parity.write_dumps(out, mel, enc, toks)
    ok, rep = parity.compare(ref, out, d_model=64)
    assert ok and rep[-1] == "PARITY OK", rep
    with open(os.path.join(out, "tokens.txt")) as f:   # CLI format: one id per line
        assert f.read() == "5\n17\n3\n3\n90\n"


@pytest.mark.parametrize("delta,ok", [(5e-4, True), (2e-3, False)])
def test_compare_mel_gate(dumps, delta, ok):
    ref, out, mel, enc, toks = dumps
    m = mel.copy()
    m[7, 100] += delta
    parity.write_dumps(out, m, enc, toks)
    assert parity.compare(ref, out, d_model=64)[0] is ok


def test_compare_mel_shape(dumps):
    ref, out, mel, enc, toks = dumps
    parity.write_dumps(out, mel[:-1], enc, toks)
    ok, rep = parity.compare(ref, out, d_model=64)
    assert not ok and "SHAPE MISMATCH" in rep[0]


@pytest.mark.parametrize("rel,ok", [(5e-3, True), (2e-2, False)])
def test_compare_encoder_gate_is_relative_to_max(dumps, rel, ok):
    ref, out, mel, enc, toks = dumps
    e = enc.copy()
    e[2, 3] += rel * np.abs(enc).max()
    parity.write_dumps(out, mel, e, toks)
    assert parity.compare(ref, out, d_model=64)[0] is ok


def test_compare_encoder_row_count(dumps):
    ref, out, mel, enc, toks = dumps
    parity.write_dumps(out, mel, np.concatenate([enc, enc[:1]]), toks)   # rows agree, one extra
    assert not parity.compare(ref, out, d_model=64)[0]
    parity.write_dumps(out, mel, enc[:0], toks)
    ok, rep = parity.compare(ref, out, d_model=64)
    assert not ok and "no rows" in rep[1]


def test_compare_tokens(dumps):
    ref, out, mel, enc, toks = dumps
    parity.write_dumps(out, mel, enc, toks[:2] + [4] + toks[3:])
    ok, rep = parity.compare(ref, out, d_model=64)
    assert not ok and any("first difference at 2: ref 3 ours 4" in r for r in rep)
    parity.write_dumps(out, mel, enc, toks[:-1])
    ok, rep = parity.compare(ref, out, d_model=64)
    assert not ok and any("first difference at 4: ref 90 ours end" in r for r in rep)


def test_compare_only_present_artefacts_and_empty_dir(dumps):
    ref, out, mel, enc, toks = dumps
    parity.write_dumps(out, mel, enc, toks)
    os.remove(os.path.join(out, "enc.f32"))
    assert parity.compare(ref, out, d_model=64)[0]
    for f in ("mel.f32", "tokens.txt"):
        os.remove(os.path.join(out, f))
    ok, rep = parity.compare(ref, out, d_model=64)
    assert not ok and "no mel.f32" in rep[0]


def test_cli_compare_exit_codes(dumps, capsys):
    ref, out, mel, enc, toks = dumps
    parity.write_dumps(out, mel, enc, toks)
    assert parity.main(["compare", ref, out, "--d-model", "64"]) == 0
    parity.write_dumps(out, mel, enc, [1])
    assert parity.main(["compare", ref, out, "--d-model", "64"]) == 1
    assert "PARITY FAILED" in capsys.readouterr().out
