"""Seeded synthetic checkpoint and audio for the streaming FastConformer-RNNT path.

The checkpoint follows the tensor names, shapes and dtype (BF16) that the loader enforces
(reference: src/model.c:41-47 `need`, src/model.c:215-282 tensor list) and the
config.json keys it reads (src/model.c:125-172).  Weights are random: matrices
N(0, 1/fan_in), LayerNorm gamma ~1 / beta ~0, small biases.  The joint output bias can be
skewed toward the blank class to give a chosen blank probability: blank_bias is added to the blank
class's bias and label_shift subtracted from every other class's bias.  The biases are stored as
bf16, whose spacing near a skew of 2 is 2^-6; splitting the skew between a bf16-exact blank_bias
and a small label_shift (spacing ~2^-11 near 0.1) sets it about 30 times more finely.

Audio is 16 kHz float32: pink noise at -20 dBFS RMS plus random linear sine chirps.
Every array is a pure function of (seed, tensor name), so a model or clip is bit-identical on
every machine.
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
import zlib

import numpy as np

# Shapes of the model the streaming benchmarks are quoted on (FastConformer 0.6B, RNNT).
FULL_DIMS = dict(
    feat_in=128, n_layers=24, d_model=1024, n_heads=8, ff_expansion_factor=4,
    subsampling_factor=8, subsampling_conv_channels=256, conv_kernel_size=9,
    num_prompts=128, prompt_hidden=2048, pred_hidden=640, vocab_size=1024, joint_hidden=640,
    max_symbols=10,
)

# A small model with the same structural constants (head_dim 128, conv kernel 9, x8
# subsampling, 128 mel bins, 2 LSTM layers) for fast CPU checks.
TINY_DIMS = dict(
    feat_in=128, n_layers=2, d_model=256, n_heads=2, ff_expansion_factor=4,
    subsampling_factor=8, subsampling_conv_channels=32, conv_kernel_size=9,
    num_prompts=16, prompt_hidden=128, pred_hidden=64, vocab_size=96, joint_hidden=64,
    max_symbols=10,
)

LANGS = ["auto", "en-US", "de-DE", "es-ES", "fr-FR", "it-IT", "ja-JP", "ko-KR", "zh-CN", "ru-RU"]
ATT_CONTEXT = [[56, 0], [56, 1], [56, 3], [56, 6], [56, 13]]


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_to_f32(u: np.ndarray) -> np.ndarray:
    return (u.astype(np.uint32) << np.uint32(16)).view(np.float32)


def _vocab(n: int) -> list[str]:
    out = ["<unk>", "<pad>", "<s>", "</s>"] + [f"<{l}>" for l in LANGS if l != "auto"]
    letters = "abcdefghijklmnopqrstuvwxyz"
    i = 0
    while len(out) < n:
        a, b, c = letters[i % 26], letters[(i // 26) % 26], letters[(i // 676) % 26]
        piece = (a + b + c)[: 1 + (i % 3)]
        out.append(("▁" + piece) if i % 2 == 0 else piece)
        i += 1
    return out[:n]


def tensor_specs(d: dict) -> list[tuple[str, tuple, str, float]]:
    """(name, shape, kind, scale) for every tensor of the checkpoint."""
    D, FF, CH = d["d_model"], d["d_model"] * d["ff_expansion_factor"], d["subsampling_conv_channels"]
    f3 = d["feat_in"]
    for _ in range(3):
        f3 = f3 // 2 + 1
    PH, NP, H = d["prompt_hidden"], d["num_prompts"], d["n_heads"]
    P, J, V = d["pred_hidden"], d["joint_hidden"], d["vocab_size"]
    s = []
    pre = "encoder.pre_encode."
    for i in (0, 2, 5):
        s.append((f"{pre}conv.{i}.weight", (CH, 1, 3, 3), "mat", 1 / 9))
        s.append((f"{pre}conv.{i}.bias", (CH,), "bias", 0.05))
    for i in (3, 6):
        s.append((f"{pre}conv.{i}.weight", (CH, CH, 1, 1), "mat", 1 / CH))
        s.append((f"{pre}conv.{i}.bias", (CH,), "bias", 0.05))
    s.append((f"{pre}out.weight", (D, CH * f3), "mat", 1 / (CH * f3)))
    s.append((f"{pre}out.bias", (D,), "bias", 0.05))
    for l in range(d["n_layers"]):
        p = f"encoder.layers.{l}."
        for ff in ("feed_forward1", "feed_forward2"):
            s.append((f"{p}{ff}.linear1.weight", (FF, D), "mat", 1 / D))
            s.append((f"{p}{ff}.linear2.weight", (D, FF), "mat", 1 / FF))
        for w in ("q", "k", "v", "out", "pos"):
            s.append((f"{p}self_attn.linear_{w}.weight", (D, D), "mat", 1 / D))
        s.append((f"{p}self_attn.pos_bias_u", (H, D // H), "bias", 0.1))
        s.append((f"{p}self_attn.pos_bias_v", (H, D // H), "bias", 0.1))
        s.append((f"{p}conv.pointwise_conv1.weight", (2 * D, D, 1), "mat", 1 / D))
        s.append((f"{p}conv.pointwise_conv2.weight", (D, D, 1), "mat", 1 / D))
        s.append((f"{p}conv.depthwise_conv.weight", (D, 1, d["conv_kernel_size"]), "mat", 1 / d["conv_kernel_size"]))
        s.append((f"{p}conv.batch_norm.weight", (D,), "gamma", 0.1))
        s.append((f"{p}conv.batch_norm.bias", (D,), "bias", 0.05))
        for n in ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out"):
            s.append((f"{p}{n}.weight", (D,), "gamma", 0.1))
            s.append((f"{p}{n}.bias", (D,), "bias", 0.05))
    s.append(("prompt_kernel.0.weight", (PH, D + NP), "mat", 1 / (D + NP)))
    s.append(("prompt_kernel.0.bias", (PH,), "bias", 0.05))
    s.append(("prompt_kernel.2.weight", (D, PH), "mat", 1 / PH))
    s.append(("prompt_kernel.2.bias", (D,), "bias", 0.05))
    for l in range(2):
        q = f"decoder.prediction.dec_rnn.lstm.{l}."
        s.append((q + "Wx", (4 * P, P), "mat", 1 / P))
        s.append((q + "Wh", (4 * P, P), "mat", 1 / P))
        s.append((q + "bias", (4 * P,), "bias", 0.1))
    s.append(("decoder.prediction.embed.weight", (V + 1, P), "mat", 1.0))
    s.append(("joint.enc.weight", (J, D), "mat", 1 / D))
    s.append(("joint.enc.bias", (J,), "bias", 0.05))
    s.append(("joint.pred.weight", (J, P), "mat", 1 / P))
    s.append(("joint.pred.bias", (J,), "bias", 0.05))
    s.append(("joint.joint_net.2.weight", (V + 1, J), "mat", 1 / J))
    s.append(("joint.joint_net.2.bias", (V + 1,), "bias", 0.02))
    return s


def make_tensor(seed: int, name: str, shape: tuple, kind: str, scale: float) -> np.ndarray:
    g = _rng(seed, name)
    x = g.standard_normal(int(np.prod(shape)), dtype=np.float32)
    if kind == "mat":
        x *= np.float32(np.sqrt(scale))
    elif kind == "gamma":
        x = np.float32(1.0) + np.float32(scale) * x
    else:
        x *= np.float32(scale)
    return x


def make_config(d: dict) -> dict:
    return {
        "encoder": {
            "feat_in": d["feat_in"], "n_layers": d["n_layers"], "d_model": d["d_model"],
            "n_heads": d["n_heads"], "ff_expansion_factor": d["ff_expansion_factor"],
            "subsampling_factor": d["subsampling_factor"],
            "subsampling_conv_channels": d["subsampling_conv_channels"],
            "conv_kernel_size": d["conv_kernel_size"], "att_context_size": ATT_CONTEXT,
        },
        "preprocessor": {"sample_rate": 16000, "features": d["feat_in"]},
        "prompt": {"num_prompts": d["num_prompts"], "prompt_hidden": d["prompt_hidden"],
                   "prompt_dictionary": {l: i for i, l in enumerate(LANGS)}},
        "decoder": {"pred_hidden": d["pred_hidden"], "pred_rnn_layers": 2, "vocab_size": d["vocab_size"]},
        "joint": {"joint_hidden": d["joint_hidden"], "num_classes": d["vocab_size"]},
        "max_symbols": d["max_symbols"],
        "default_att_context_size": [56, 6],
        "vocabulary": _vocab(d["vocab_size"]),
    }


def write_model(out_dir: str, dims: dict | None = None, seed: int = 0, blank_bias: float = 0.0,
                label_shift: float = 0.0) -> str:
    """Write config.json + model.safetensors into out_dir (skipped if an identical one is there)."""
    d = dict(FULL_DIMS if dims is None else dims)
    key = [d, seed, blank_bias] + ([label_shift] if label_shift else [])
    tag = hashlib.sha1(json.dumps(key, sort_keys=True).encode()).hexdigest()[:16]
    os.makedirs(out_dir, exist_ok=True)
    stamp = os.path.join(out_dir, "synth.tag")
    if os.path.exists(stamp) and open(stamp).read() == tag and os.path.exists(os.path.join(out_dir, "model.safetensors")):
        return out_dir
    specs = sorted(tensor_specs(d), key=lambda t: t[0])
    header, off = {}, 0
    for name, shape, _, _ in specs:
        n = int(np.prod(shape)) * 2
        header[name] = {"dtype": "BF16", "shape": list(shape), "data_offsets": [off, off + n]}
        off += n
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    blank = d["vocab_size"]
    tmp = os.path.join(out_dir, "model.safetensors.tmp")
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for name, shape, kind, scale in specs:
            x = make_tensor(seed, name, shape, kind, scale)
            if name == "joint.joint_net.2.bias":
                x[blank] += np.float32(blank_bias)
                x[:blank] -= np.float32(label_shift)
            f.write(f32_to_bf16(x).tobytes())
    os.replace(tmp, os.path.join(out_dir, "model.safetensors"))
    with open(os.path.join(out_dir, "config.json"), "w") as f:
        json.dump(make_config(d), f, ensure_ascii=False)
    with open(stamp, "w") as f:
        f.write(tag)
    return out_dir


def make_audio(seconds: float, seed: int = 0, rate: int = 16000) -> np.ndarray:
    """Pink noise at -20 dBFS RMS plus random linear sine chirps, float32 mono."""
    n = int(round(seconds * rate))
    g = np.random.default_rng([seed, 0xA0D10])
    white = g.standard_normal(n)
    spec = np.fft.rfft(white)
    f = np.arange(spec.size, dtype=np.float64)
    f[0] = 1.0
    pink = np.fft.irfft(spec / np.sqrt(f), n)
    pink *= 0.1 / max(np.sqrt(np.mean(pink * pink)), 1e-12)
    x = pink
    t = np.arange(n) / rate
    for _ in range(max(1, int(seconds * 1.5))):
        t0 = g.uniform(0, max(seconds - 0.2, 0.01))
        dur = g.uniform(0.15, 0.9)
        f0, f1 = g.uniform(150, 3500, size=2)
        amp = g.uniform(0.03, 0.2)
        m = (t >= t0) & (t < t0 + dur)
        tt = t[m] - t0
        phase = 2 * np.pi * (f0 * tt + 0.5 * (f1 - f0) / dur * tt * tt)
        env = np.sin(np.pi * tt / dur) ** 2
        x[m] += amp * env * np.sin(phase)
    return x.astype(np.float32)


def load_safetensors(path: str) -> dict[str, tuple[np.ndarray, tuple]]:
    """Minimal read-only reader: name -> (raw uint16 bf16 view, shape).  Memory-mapped."""
    with open(path, "rb") as f:
        hlen = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(hlen))
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    base = 8 + hlen
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        a, b = meta["data_offsets"]
        assert meta["dtype"] == "BF16", name
        out[name] = (mm[base + a: base + b].view(np.uint16), tuple(meta["shape"]))
    return out


if __name__ == "__main__":
    import argparse
    import time

    ap = argparse.ArgumentParser()
    ap.add_argument("out_dir")
    ap.add_argument("--tiny", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--blank-bias", type=float, default=0.0)
    a = ap.parse_args()
    t0 = time.time()
    write_model(a.out_dir, TINY_DIMS if a.tiny else FULL_DIMS, a.seed, a.blank_bias)
    print(f"wrote {a.out_dir} in {time.time() - t0:.1f}s")
