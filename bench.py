#!/usr/bin/env python3
"""Streaming ASR benchmark on one MI355X.

Headline (value): one stream at 80 ms latency (1 encoder frame per chunk, every GEMM an M=1
weight-streaming GEMV) over 10 s of seeded 16 kHz synthetic audio, FastConformer 0.6B + RNNT with
seeded random-init bf16 weights.  A step is one pass of that clip through the public C API
(nemoasr_reset + nemoasr_feed in chunk-sized pieces, like the reference's file mode,
src/main.c:234-246); value = RTFx = audio seconds / wall seconds over the timed steps.

Legs in the same JSON line (each with its own roofline of its dominant kernel):
  S560   one stream, 560 ms, 10 s, en-US;
  S1120  one stream, 1120 ms, 30 s, en-US, joint bias skewed to P(blank) ~ 0.5 (the token loop);
  B64    64 streams, 560 ms, 20 s each, start offsets 0-7 chunks of pre-filled caches;
  B256   256 streams, 1120 ms, 60 s each, prompt auto, offsets 0-4 chunks, P(blank) ~ 0.7.
P(blank) is measured and reported as blank decisions / all greedy decisions, counted as
frames / (frames + tokens) (a frame ends on a blank unless it reaches max_symbols).

Per single-stream leg: RTFx, p50/p90 chunk latency (encoder step + its decoder round trips), the
encoder's HBM rate (1,176,502,272 bytes of bf16 weights streamed per chunk / chunk GPU time) and the
roofline of the dominant kernel class (algorithmic bytes / mean launch duration from hipEvents
stamped by the dispatch itself around every launch of the class on the library's stream, during a
direct-launch replay of the same clip).  Per batch leg: aggregate RTFx, p50 step latency (one chunk
of every stream, from the step's start to its tokens), the step period, and the MFMA roofline of the
encoder's many-row GEMM kernels (algorithmic 2*M*N*K flops / dispatch-stamped durations, from a
direct-launch pass in which each step's greedy loop is drained before the next step starts, so that
the durations are the kernels' own and not shared with the overlapping loop of the timed passes).

CPU baseline: the oracle's C restatement (log-mel + encoder + greedy RNNT) on bounded samples of the
headline clip and of every leg's workload on this host's cores, at one thread and at all threads
given to this process: RTFx and the median chunk time (batch legs: streams one after another, the
step time being the stream count times the chunk time).
"""
import argparse
import glob
import json
import os
import re
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
# dominant kernel class per latency: one-row chunks run every conformer block in one persistent
# launch (enc_chain); two-row chunks stream each matrix in a GEMV, longer chunks in few-row GEMMs
DOMINANT = {80: "enc_chain", 160: "gemv_*", 320: "gemm_fr*", 560: "gemm_fr*", 1120: "gemm_fr*"}
# joint-bias skews (blank_bias, label_shift) of the checkpoints for the skewed legs, calibrated on
# those legs' own workloads by bisection on label_shift (MI355X): S1120 gives P(blank) 0.500
# (376 tokens over 376 frames), B256 0.701
SKEW_S1120 = (2.0, 0.0188)
SKEW_B256 = (2.0, 0.0619)
# HBM traffic per launch of the headline's dominant kernel class, from rocprofv3 FETCH_SIZE and
# WRITE_SIZE runs of this benchmark's headline workload (profiles/stream80_hbm_traffic.md)
PROFILES = os.path.join(REPO, "profiles")


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


def model(synth, skew=(0.0, 0.0)):
    cache = os.environ.get("NEMO_MODEL_CACHE", "/tmp/nemo_models")
    bb, ls = skew
    tag = f"full_s0_b{bb:g}" + (f"_l{ls:g}" if ls else "")
    return synth.write_model(os.path.join(cache, tag), synth.FULL_DIMS, 0, bb, ls)


def p_blank(frames, tokens):
    return round(frames / (frames + tokens), 4) if frames + tokens else None


def traffic_from_profile(kernel: str, leg: str = ""):
    """HBM bytes per launch (FETCH + WRITE, scaled by the copy calibration) that a committed PMC
    summary under profiles/ records for this kernel class (key "leg:class" for the extra legs,
    the class alone for the headline stream), or None."""
    key = f"{leg}:{kernel}" if leg else kernel
    pat = re.compile(r"traffic_bytes_per_launch\[" + re.escape(key) + r"\]\s*=\s*([0-9.eE+]+)")
    for path in sorted(glob.glob(os.path.join(PROFILES, "*.md"))):
        try:
            m = pat.search(open(path).read())
        except OSError:
            continue
        if m:
            return float(m.group(1))
    return None


def single_leg(a, nemoasr, synth, mdir, cfg, latency, seconds, lang="en-US", steps=None, warmup=None, frames_fn=None):
    """One stream through the public API: see the module docstring."""
    steps = a.steps if steps is None else steps
    warmup = a.warmup if warmup is None else warmup
    audio = synth.make_audio(seconds, seed=0)
    audio_s = audio.size / 16000.0
    right = LAT_RIGHT[latency]
    piece = (right + 1) * 8 * 160
    s = nemoasr.Session(mdir, lang, latency)

    def clip():
        s.reset(lang, latency)
        s.use_graphs(not a.no_graphs)
        t0 = time.perf_counter()
        for i in range(0, audio.size, piece):
            s.feed(audio[i:i + piece], final=i + piece >= audio.size)
        return time.perf_counter() - t0

    for _ in range(warmup):
        clip()
    times, chunk_ms, enc_gpu, chunks, toks, trips = [], [], 0.0, 0, 0, 0
    for _ in range(steps):
        times.append(clip())
        chunk_ms.append(s.chunk_ms())
        st = s.stats()
        enc_gpu += nemoasr.lib().nemoasr_debug_encoder_gpu_ms(s.h)
        chunks += st["chunks"]
        toks += st["tokens"]
        trips += s.joint_steps
    wall = sum(times)
    cms = np.concatenate(chunk_ms)
    wb = weight_bytes_per_chunk(cfg)
    enc_ms = enc_gpu / max(chunks, 1)
    # dominant kernel class: hipEvents around each of its launches during a direct-launch replay
    kname = DOMINANT.get(latency, "gemm_fr*")
    s.reset(lang, latency)
    s.use_graphs(False)
    s.time_kernel(kname, 32768)
    for i in range(0, audio.size, piece):
        s.feed(audio[i:i + piece], final=i + piece >= audio.size)
    kms, kn, kbytes = s.kernel_ms()
    s.time_kernel(None, 0)
    achieved = (kbytes / max(kn, 1)) / (kms * 1e-3) / 1e9 if kn and kms > 0 else 0.0
    gpu_name = s.gpu_name
    s.close()
    # a freshly opened session: open time (model load + warm-up, which captures the session's chunk
    # and decoder graphs) and its first chunk's latency
    s = nemoasr.Session(mdir, lang, latency)
    open_ms = s.load_ms
    for i in range(0, min(audio.size, 4 * piece), piece):
        s.feed(audio[i:i + piece])
    first = s.chunk_ms()
    s.close()
    frames = frames_fn(audio.size)
    return {
        "workload": f"1 stream, {latency} ms latency ({right + 1} encoder frame(s)/chunk), {audio_s:g} s of 16 kHz "
                    f"audio, prompt {lang}",
        "latency_ms": latency, "audio_s": audio_s, "rtfx": round(steps * audio_s / wall, 3),
        "ms_per_pass": round(1e3 * wall / steps, 3),
        "chunks_per_clip": int(chunks / steps), "frames_per_clip": frames, "tokens_per_clip": int(toks / steps),
        "p_blank": p_blank(frames, toks / steps),
        "joint_round_trips_per_clip": int(trips / steps),
        "p50_chunk_ms": round(float(np.median(cms)), 4), "p90_chunk_ms": round(float(np.percentile(cms, 90)), 4),
        "first_chunk_ms": round(float(first[0]), 4) if first.size else None, "open_ms": round(open_ms, 1),
        "encoder_gpu_ms_per_chunk": round(enc_ms, 4), "encoder_weight_bytes_per_chunk": wb,
        "encoder_chunk_hbm_gbs": round(wb / (enc_ms * 1e-3) / 1e9, 1) if enc_ms > 0 else None,
        "graphs": not a.no_graphs, "gpu": gpu_name,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile(kname, "" if latency == 80 else f"S{latency}"), "kernel": kname,
                     "launches": kn,
                     "mean_launch_us": round(kms * 1e3, 3), "bytes_per_launch": round(kbytes / max(kn, 1))},
    }


def batch_leg(a, nemoasr, synth, mdir, cfg, S, lat, seconds, offsets, lang):
    """Many streams through the batch API; see the module docstring."""
    right = LAT_RIGHT[lat]
    piece = (right + 1) * 8 * 160
    nsamp = int(round(seconds * 16000))
    clips = [synth.make_audio(seconds, seed=1000 + s) for s in range(S)]
    offs = [s % (offsets + 1) for s in range(S)]
    pre = [synth.make_audio(max(o, 1) * piece / 16000.0, seed=2000 + s)[: o * piece] for s, o in enumerate(offs)]
    b = nemoasr.Batch(mdir, lang, lat, S)
    b.use_graphs(not a.no_graphs)

    def run_once(serial=False):
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
            if serial:  # wait for this step's greedy loop: the next step's encoder runs alone
                b.tokens(0)
        b.run()
        wall = time.perf_counter() - t0
        st1 = b.stats()
        return wall, b.step_ms()[n0:], {k: st1[k] - st0[k] for k in st1}

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
    # the encoder's many-row GEMM kernels timed one by one during a direct-launch pass of the same
    # workload, each step's greedy loop (its own stream, overlapping the next step's encoder in the
    # timed passes) drained first, so that the durations are the kernels' own
    b.use_graphs(False)
    b.time_kernel("gemm_m*", 32768)
    run_once(serial=True)
    kms, kn, _, kfl = b.kernel_ms()
    b.time_kernel(None, 0)
    achieved = kfl / (kms * kn * 1e-3) / 1e12 if kn and kms > 0 else 0.0
    b.close()
    steps = max(int(tot["steps"]), 1)
    return {
        "workload": f"{S} streams, {lat} ms latency ({right + 1} encoder frames/chunk/stream, M = {S * (right + 1)} rows "
                    f"per steady step), {seconds:g} s of 16 kHz audio per stream (own seed), start offsets "
                    f"0-{offsets} chunks of pre-filled caches, prompt {lang}",
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
        "p_blank": p_blank(tot["rows"], tot["tokens"]),
        "encoder_gemm_tflops": round(enc_tflops, 1),
        "encoder_gemm_frac_of_bf16_peak": round(enc_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "graphs": not a.no_graphs,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic_from_profile("gemm_m*", f"B{S}"),
                     "kernel": "gemm_m*",
                     "launches": kn, "mean_launch_us": round(kms * 1e3, 3),
                     "note": "algorithmic 2*M*N*K flops; the f32 activations enter the MFMAs as bf16 hi + lo "
                             "halves, so the kernels issue twice these MFMA flops"},
    }


def cpu_threads() -> int:
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


_ORACLE_MODELS = {}


def cpu_sample(mdir, lang, latency, clips, threads, what):
    """The oracle's C restatement (log-mel + encoder + greedy RNNT) on `clips` (one stream after
    another, each fed one chunk of mel rows at a time) with `threads` threads: RTFx over the sample
    and the median chunk time (one chunk's encoder step and its greedy decode)."""
    import mel_ref
    import oracle

    oracle.lib().or_set_threads(threads)
    key = (mdir, lang)
    if key not in _ORACLE_MODELS:
        _ORACLE_MODELS[key] = oracle.Model(mdir, lang)
    om = _ORACLE_MODELS[key]
    right = LAT_RIGHT[latency]
    cm = 8 * (right + 1)
    chunk_ms, wall, chunks = [], 0.0, 0
    for clip in clips:
        t0 = time.perf_counter()
        mel = mel_ref.logmel(clip)
        o = oracle.Session(om, right)
        for i in range(0, mel.shape[0], cm):
            tc = time.perf_counter()
            o.feed_mel(mel[i:i + cm], final=i + cm >= mel.shape[0])
            if i + cm <= mel.shape[0]:
                chunk_ms.append(1e3 * (time.perf_counter() - tc))
        wall += time.perf_counter() - t0
        chunks += o.chunks
    audio_s = sum(c.size for c in clips) / 16000.0
    return {"value": round(audio_s / wall, 4), "unit": "audio-s/s", "cores": threads, "kind": "port",
            "p50_chunk_ms": round(float(np.median(chunk_ms)), 2) if chunk_ms else None,
            "sample": f"{what}: {audio_s:g} s of audio through the oracle's C restatement (log-mel + encoder + greedy "
                      f"RNNT) at {latency} ms latency, {threads} thread(s), {chunks} chunks, {wall:.1f} s",
            "seconds": round(wall, 2)}


def cpu_baselines(synth, mdir, a, want):
    """Bounded CPU samples of the headline and of every leg, at all threads given to this process
    and at one thread (a few seconds of CPU work each).  Batch legs: streams one after another (the
    oracle has no batching); their p50 step is the stream count times the median chunk time."""
    n = cpu_threads()
    out = {}
    head_audio = synth.make_audio(a.seconds, seed=0)
    chunk_s = {80: 0.08, 560: 0.56, 1120: 1.12}
    cases = {"S80": (mdir, "en-US", a.latency, [head_audio[: int(a.cpu_sample_s * 16000)]],
                     [head_audio[: int(a.cpu1_sample_s * 16000)]], "first %s s of the headline clip" % a.cpu_sample_s,
                     1)}
    if "S560" in want:
        clip = synth.make_audio(10.0, seed=0)
        cases["S560"] = (mdir, "en-US", 560, [clip[:int(3.4 * 16000)]], [clip[:int(0.6 * 16000)]],
                         "first seconds of the 560 ms leg's clip", 1)
    if "S1120" in want:
        clip = synth.make_audio(30.0, seed=0)
        cases["S1120"] = (model(synth, SKEW_S1120), "en-US", 1120, [clip[:int(3.4 * 16000)]],
                          [clip[:int(1.2 * 16000)]], "first seconds of the 1120 ms leg's clip (P(blank) 0.5 model)", 1)
    if "B64" in want:
        clips = [synth.make_audio(20.0, seed=1000 + s) for s in range(2)]
        cases["B64"] = (mdir, "en-US", 560, [c[:int(1.2 * 16000)] for c in clips], [clips[0][:int(0.6 * 16000)]],
                        "first seconds of streams 0-1 of the 64-stream leg", 64)
    if "B256" in want:
        clips = [synth.make_audio(60.0, seed=1000 + s) for s in range(2)]
        cases["B256"] = (model(synth, SKEW_B256), "auto", 1120, [c[:int(2.3 * 16000)] for c in clips],
                         [clips[0][:int(1.2 * 16000)]], "first seconds of streams 0-1 of the 256-stream leg (auto, "
                                                        "P(blank) 0.7 model)", 256)
    # a batch leg's one-thread chunk costs what the single-stream leg of its latency and model size
    # costs, whose one-thread sample it reuses
    same = {"B64": "S560", "B256": "S1120"}
    for leg, (md, lang, lat, many, one, what, streams) in cases.items():
        full = cpu_sample(md, lang, lat, many, n, what)
        if leg in same and same[leg] in out:
            single = dict(out[same[leg]]["single_thread"])
            single["sample"] = f"the {same[leg]} leg's one-thread sample (same latency and model size): " + single["sample"]
        else:
            single = cpu_sample(md, lang, lat, one, 1, what)
        for r in (full, single):
            if streams > 1 and r["p50_chunk_ms"] is not None:
                r["p50_step_ms"] = round(streams * r["p50_chunk_ms"], 1)
        full["single_thread"] = single
        out[leg] = full
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--latency", type=int, default=80, choices=sorted(LAT_RIGHT))
    ap.add_argument("--seconds", type=float, default=10.0)
    ap.add_argument("--cpu-sample-s", type=float, default=6.0, help="audio seconds of the all-threads CPU sample")
    ap.add_argument("--cpu1-sample-s", type=float, default=1.0, help="audio seconds of the one-thread CPU sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graphs", action="store_true")
    ap.add_argument("--legs", default="S560,S1120,B64,B256", help="comma list of extra legs (empty: none)")
    ap.add_argument("--legs-only", action="store_true",
                    help="profiling: skip the headline stream and print {'legs': ...} only")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="profiling: first run one f32 copy of this many MiB (the HBM counter calibration)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs one stream set on one GPU; --gpus {a.gpus} is not supported "
              "(independent streams shard by stream across GPUs with no communication)", file=sys.stderr)
        sys.exit(2)

    import nemoasr
    import synth

    if a.no_graphs:
        # direct launches from each session's open on (its warm-up included)
        nemoasr.lib().nemoasr_debug_default_graphs(0)

    def sub3(nsamp):  # encoder frames of a clip: mel frames (centred, 10 ms hop) subsampled x8
        n = nsamp // 160 + 1
        for _ in range(3):
            n = n // 2 + 1
        return n

    if a.copy_calib_mib > 0:  # one copy_f32 dispatch of known size: n floats read, n floats written
        g = nemoasr.Gpu()
        n = a.copy_calib_mib << 18
        src, dst = g.alloc(4 * n), g.alloc(4 * n)
        g.begin()
        g.check(nemoasr.lib().nk_copy(g.h, src.ptr, dst.ptr, n))
        g.end()
        g.close()

    mdir = model(synth)
    cfg = json.load(open(os.path.join(mdir, "config.json")))
    head = None if a.legs_only else single_leg(a, nemoasr, synth, mdir, cfg, a.latency, a.seconds, frames_fn=sub3)
    legs = {}
    want = [x for x in a.legs.split(",") if x]
    if "S560" in want:
        legs["S560"] = single_leg(a, nemoasr, synth, mdir, cfg, 560, 10.0, frames_fn=sub3)
    if "S1120" in want:
        legs["S1120"] = single_leg(a, nemoasr, synth, model(synth, SKEW_S1120), cfg, 1120, 30.0, frames_fn=sub3)
        legs["S1120"]["skew"] = {"blank_bias": SKEW_S1120[0], "label_shift": SKEW_S1120[1]}
    if "B64" in want:
        legs["B64"] = batch_leg(a, nemoasr, synth, mdir, cfg, 64, 560, 20.0, 7, "en-US")
    if "B256" in want:
        legs["B256"] = batch_leg(a, nemoasr, synth, model(synth, SKEW_B256), cfg, 256, 1120, 60.0, 4, "auto")
        legs["B256"]["skew"] = {"blank_bias": SKEW_B256[0], "label_shift": SKEW_B256[1]}

    if head is None:
        print(json.dumps({"legs": legs}), flush=True)
        return

    cpu = None
    if not a.no_cpu:
        base = cpu_baselines(synth, mdir, a, want)
        cpu = base.pop("S80")
        cpu["cpu_model"] = cpu_model()
        cpu["nproc"] = os.cpu_count()
        for leg, b in base.items():
            legs[leg]["cpu_baseline"] = b

    out = {
        "metric": METRIC, "value": head["rtfx"], "unit": "audio-s/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": head["ms_per_pass"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded random-init bf16 weights (seed 0), seeded pink noise -20 dBFS + sine chirps",
        "config": dict(head, workload=head["workload"] + ", FastConformer 0.6B (24 x d1024, FF 4096, 8 heads) + RNNT "
                                                         "(2 x LSTM 640, vocab 1024+blank)",
                       streams=1, weights="bf16", activations="f32"),
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "legs": legs,
    }
    out["config"].pop("roofline")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
