#!/usr/bin/env python3
"""Streaming ASR benchmark on one MI355X.

Workload (default): one stream at 80 ms latency (1 encoder frame per chunk, every GEMM an M=1
weight-streaming GEMV) over 10 s of seeded 16 kHz synthetic audio, FastConformer 0.6B + RNNT with
seeded random-init bf16 weights.  A step is one pass of that clip through the public C API
(nemoasr_reset + nemoasr_feed in chunk-sized pieces, like the reference's file mode,
src/main.c:234-246); value = RTFx = audio seconds / wall seconds over the timed steps.

A second leg runs the batched multi-stream path (include/nemoasr_batch.h): by default 64 streams
at 560 ms (M = 448 encoder rows per step), each stream with its own seeded 20 s clip and a start
offset of 0-7 chunks of pre-filled caches; it reports aggregate RTFx, p50 step latency (one chunk of
every stream, from the step's start to its tokens: front end + encoder + RNNT loop), the step period
(the RNNT loop of a step overlaps the next step's front end and encoder, so steps start faster than
they finish), the encoder's GEMM TFLOP/s per step and the MFMA roofline of the many-row GEMM kernels.

Also reported: p50 chunk latency (encoder step + its decoder round trips), the per-chunk HBM rate
of the encoder (1,176,502,272 bytes of bf16 weights streamed per chunk / chunk GPU time), the
roofline of the dominant kernel (algorithmic bytes / mean launch time, hipEvents around every
launch of that kernel on its stream during a direct-launch replay of the same clip), and the CPU
baseline: the oracle's C restatement on a bounded sample of the same clip on this host's cores.
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "nemo-c_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

import numpy as np  # noqa: E402

METRIC = "RTFx (audio-s/s) + p50 chunk ms at 1 and 64 streams; achieved HBM GB/s"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
LAT_RIGHT = {80: 0, 160: 1, 320: 3, 560: 6, 1120: 13}
DOMINANT = {80: "gemv_*", 160: "gemv_*", 320: "gemm_fr*", 560: "gemm_fr*", 1120: "gemm_fr*"}


def weight_bytes_per_chunk(cfg: dict) -> int:
    """bf16 bytes of every matrix a chunk streams once (prompt W0: its d_model used columns)."""
    e, p, j = cfg["encoder"], cfg["prompt"], cfg["joint"]
    D, FF, CH, nl = e["d_model"], e["d_model"] * e["ff_expansion_factor"], e["subsampling_conv_channels"], e["n_layers"]
    f3 = e["feat_in"]
    for _ in range(3):
        f3 = f3 // 2 + 1
    layer = 4 * FF * D + 3 * D * D + D * D + 2 * D * D + D * D
    params = nl * layer + 2 * CH * CH + D * CH * f3 + 2 * p["prompt_hidden"] * D + j["joint_hidden"] * D
    return 2 * params


def gemm_params_per_row(cfg: dict) -> int:
    """Weights every encoder row multiplies in the block, prompt and joint.enc GEMMs (a batched step
    does 2 * M * this many flops in them)."""
    e, p, j = cfg["encoder"], cfg["prompt"], cfg["joint"]
    D, FF, nl = e["d_model"], e["d_model"] * e["ff_expansion_factor"], e["n_layers"]
    layer = 4 * FF * D + 3 * D * D + D * D + 2 * D * D + D * D
    return nl * layer + 2 * p["prompt_hidden"] * D + j["joint_hidden"] * D


def batch_leg(a, nemoasr, synth, mdir, cfg):
    """Many streams through the batch API; see the module docstring."""
    S, lat, right = a.batch_streams, a.batch_latency, LAT_RIGHT[a.batch_latency]
    piece = (right + 1) * 8 * 160
    nsamp = int(round(a.batch_seconds * 16000))
    clips = [synth.make_audio(a.batch_seconds, seed=1000 + s) for s in range(S)]
    offs = [s % (a.batch_offsets + 1) for s in range(S)]
    pre = [synth.make_audio(max(o, 1) * piece / 16000.0, seed=2000 + s)[: o * piece] for s, o in enumerate(offs)]
    b = nemoasr.Batch(mdir, a.batch_lang, lat, S)
    b.use_graphs(not a.no_graphs)

    def run_once():
        for s in range(S):
            b.reset_stream(s)
            if offs[s]:
                b.push(s, pre[s])
        b.run()  # caches pre-filled to each stream's start offset
        st0, n0 = b.stats(), b.step_ms().size
        t0 = time.perf_counter()
        for i in range(0, nsamp, piece):
            fin = i + piece >= nsamp
            for s in range(S):
                b.push(s, clips[s][i:i + piece], final=fin)
            b.step()
        b.run()
        wall = time.perf_counter() - t0
        st1 = b.stats()
        d = {k: st1[k] - st0[k] for k in st1}
        return wall, b.step_ms()[n0:], d

    for _ in range(a.warmup):
        run_once()
    walls, sms, tot = [], [], None
    for _ in range(a.steps):
        w, sm, d = run_once()
        walls.append(w)
        sms.append(sm)
        tot = d if tot is None else {k: tot[k] + d[k] for k in d}
    wall = sum(walls)
    sm = np.concatenate(sms)
    rtfx = a.steps * S * nsamp / 16000.0 / wall
    flops_rows = 2.0 * gemm_params_per_row(cfg) * tot["rows"]
    enc_tflops = flops_rows / (tot["encoder_gpu_ms"] * 1e-3) / 1e12 if tot["encoder_gpu_ms"] > 0 else 0.0

    # many-row GEMM kernels timed one by one during a direct-launch pass of the same workload
    b.use_graphs(False)
    b.time_kernel("gemm_m*", 32768)
    run_once()
    kms, kn, _, kfl = b.kernel_ms()
    b.time_kernel(None, 0)
    achieved = kfl / (kms * kn * 1e-3) / 1e12 if kn and kms > 0 else 0.0
    b.close()
    steps = max(int(tot["steps"]), 1)
    return {
        "workload": f"{S} streams, {lat} ms latency ({right + 1} encoder frames/chunk/stream, M = {S * (right + 1)} rows "
                    f"per steady step), {a.batch_seconds:g} s of 16 kHz audio per stream (own seed), start offsets "
                    f"0-{a.batch_offsets} chunks of pre-filled caches, prompt {a.batch_lang}",
        "streams": S, "latency_ms": lat, "rtfx": round(rtfx, 2), "audio_s_per_pass": S * nsamp / 16000.0,
        "wall_s_per_pass": round(wall / a.steps, 4),
        "p50_step_ms": round(float(np.median(sm)), 3), "p90_step_ms": round(float(np.percentile(sm, 90)), 3),
        "step_period_ms": round(wall / steps * 1e3, 3),
        "steps_per_pass": int(tot["steps"] / a.steps), "rows_per_step": round(tot["rows"] / steps, 1),
        "frontend_ms_per_step": round(tot["frontend_ms"] / steps, 3),
        "encoder_ms_per_step": round(tot["encoder_ms"] / steps, 3),
        "encoder_gpu_ms_per_step": round(tot["encoder_gpu_ms"] / steps, 3),
        "decoder_ms_per_step": round(tot["decoder_ms"] / steps, 3),
        "joint_round_trips_per_step": round(tot["joint_steps"] / steps, 2),
        "tokens_per_pass": int(tot["tokens"] / a.steps),
        "encoder_gemm_tflops": round(enc_tflops, 1),
        "encoder_gemm_frac_of_bf16_peak": round(enc_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "graphs": not a.no_graphs,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None, "kernel": "gemm_m*",
                     "launches": kn, "mean_launch_us": round(kms * 1e3, 3),
                     "note": "algorithmic 2*M*N*K flops; the f32 activations enter the MFMAs as bf16 hi + lo "
                             "halves, so the kernels issue twice these MFMA flops"},
    }


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--latency", type=int, default=80, choices=sorted(LAT_RIGHT))
    ap.add_argument("--seconds", type=float, default=10.0)
    ap.add_argument("--cpu-sample-s", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graphs", action="store_true")
    ap.add_argument("--kernel", default=None, help="kernel whose launches are timed for the roofline")
    ap.add_argument("--batch-streams", type=int, default=64, help="0 skips the multi-stream leg")
    ap.add_argument("--batch-latency", type=int, default=560, choices=sorted(LAT_RIGHT))
    ap.add_argument("--batch-seconds", type=float, default=20.0)
    ap.add_argument("--batch-offsets", type=int, default=7, help="start offsets 0..this many chunks")
    ap.add_argument("--batch-lang", default="en-US")
    ap.add_argument("--batch-blank-bias", type=float, default=0.0,
                    help="added to the blank logit's bias of the checkpoint for the multi-stream leg")
    ap.add_argument("--batch-only", action="store_true")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="first run one device copy of this many MiB (a known-size reference for HBM counters)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs one stream set on one GPU; --gpus {a.gpus} is not supported "
              "(independent streams shard by stream across GPUs with no communication)", file=sys.stderr)
        sys.exit(2)

    import nemoasr
    import synth

    cache = os.environ.get("NEMO_MODEL_CACHE", "/tmp/nemo_models")
    mdir = synth.write_model(os.path.join(cache, "full_s0_b0"), synth.FULL_DIMS, 0, 0.0)
    cfg = json.load(open(os.path.join(mdir, "config.json")))

    def run_batch():
        bb = a.batch_blank_bias
        bdir = mdir if bb == 0 else synth.write_model(os.path.join(cache, f"full_s0_b{bb:g}"), synth.FULL_DIMS, 0, bb)
        r = batch_leg(a, nemoasr, synth, bdir, cfg)
        r["blank_bias"] = bb
        return r

    if a.batch_only:
        print(json.dumps({"batch": run_batch()}), flush=True)
        return
    audio = synth.make_audio(a.seconds, seed=0)
    audio_s = audio.size / 16000.0
    right = LAT_RIGHT[a.latency]
    piece = (right + 1) * 8 * 160

    s = nemoasr.Session(mdir, "en-US", a.latency)
    s.use_graphs(not a.no_graphs)
    if a.copy_calib_mib:
        g = nemoasr.Gpu()
        nb = a.copy_calib_mib << 20
        src, dst = g.alloc(nb), g.alloc(nb)
        g.begin()
        g.check(nemoasr.lib().nk_copy(g.h, src.ptr, dst.ptr, nb // 4))
        g.end()
        g.close()

    def clip():
        s.reset("en-US", a.latency)
        s.use_graphs(not a.no_graphs)
        t0 = time.perf_counter()
        for i in range(0, audio.size, piece):
            s.feed(audio[i:i + piece], final=i + piece >= audio.size)
        return time.perf_counter() - t0

    for _ in range(a.warmup):
        clip()
    times, chunk_ms, enc_gpu, chunks, toks, steps = [], [], 0.0, 0, 0, 0
    for _ in range(a.steps):
        times.append(clip())
        chunk_ms.append(s.chunk_ms())
        st = s.stats()
        enc_gpu += nemoasr.lib().nemoasr_debug_encoder_gpu_ms(s.h)
        chunks += st["chunks"]
        toks += st["tokens"]
        steps += s.joint_steps
    wall = sum(times)
    rtfx = a.steps * audio_s / wall
    cms = np.concatenate(chunk_ms)
    wb = weight_bytes_per_chunk(cfg)
    enc_ms_per_chunk = enc_gpu / max(chunks, 1)

    # dominant kernel: hipEvents around each of its launches during a direct-launch replay
    kname = a.kernel or DOMINANT.get(a.latency, "gemm_fr*")
    s.reset("en-US", a.latency)
    s.use_graphs(False)
    s.time_kernel(kname, 32768)
    for i in range(0, audio.size, piece):
        s.feed(audio[i:i + piece], final=i + piece >= audio.size)
    kms, kn, kbytes = s.kernel_ms()
    s.time_kernel(None, 0)
    achieved = (kbytes / max(kn, 1)) / (kms * 1e-3) / 1e9 if kn and kms > 0 else 0.0
    gpu_name = s.gpu_name
    s.close()
    batch = run_batch() if a.batch_streams > 0 else None

    cpu = None
    if not a.no_cpu:
        import mel_ref
        import oracle

        n = cpu_threads()
        oracle.lib().or_set_threads(n)
        om = oracle.Model(mdir, "en-US")
        sample = audio[: int(a.cpu_sample_s * 16000)]
        t0 = time.perf_counter()
        o = oracle.Session(om, right)
        o.feed_mel(mel_ref.logmel(sample), final=True)
        dt = time.perf_counter() - t0
        cpu = {"value": round(sample.size / 16000.0 / dt, 4), "unit": "audio-s/s", "cores": n, "kind": "port",
               "sample": f"first {a.cpu_sample_s:g} s of the same clip at {a.latency} ms latency through the oracle's "
                         f"C restatement (log-mel + encoder + greedy RNNT), {n} threads, {o.chunks} chunks"}

    out = {
        "metric": METRIC, "value": round(rtfx, 3), "unit": "audio-s/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(1e3 * wall / a.steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded random-init bf16 weights (seed 0), seeded pink noise -20 dBFS + sine chirps",
        "config": {
            "workload": f"1 stream, {a.latency} ms latency ({right + 1} encoder frame(s)/chunk), {audio_s:g} s of 16 kHz "
                        "audio, FastConformer 0.6B (24 x d1024, FF 4096, 8 heads) + RNNT (2 x LSTM 640, vocab 1024+blank)",
            "latency_ms": a.latency, "streams": 1, "audio_s": audio_s, "graphs": not a.no_graphs,
            "weights": "bf16", "activations": "f32",
            "chunks_per_clip": int(chunks / a.steps), "tokens_per_clip": int(toks / a.steps),
            "joint_round_trips_per_clip": int(steps / a.steps),
            "p50_chunk_ms": round(float(np.median(cms)), 4), "p90_chunk_ms": round(float(np.percentile(cms, 90)), 4),
            "encoder_gpu_ms_per_chunk": round(enc_ms_per_chunk, 4),
            "encoder_weight_bytes_per_chunk": wb,
            "encoder_chunk_hbm_gbs": round(wb / (enc_ms_per_chunk * 1e-3) / 1e9, 1) if enc_ms_per_chunk > 0 else None,
            "gpu": gpu_name,
        },
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": kname,
                     "launches": kn, "mean_launch_us": round(kms * 1e3, 3),
                     "bytes_per_launch": round(kbytes / max(kn, 1))},
        "cpu_baseline": cpu,
        "batch": batch,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
