#!/usr/bin/env python3
"""Kernel micro-benchmark of the streaming hot path on one MI355X (the methodology of the
reference's tools/kbench.c:140-195: every GEMM shape of a chunk against HBM-resident weights).

For each shape it reports
  graph_us   launch-to-launch time of the kernel replayed back to back inside a hipGraph (the
             way a chunk runs), with a fresh weight matrix per launch so nothing is served from
             cache;
  kernel_us  mean execution time of the same launches from dispatch-stamped events (what
             rocprofv3 reports as the kernel duration);
  GB/s       weight bytes / kernel_us and / graph_us.
Plus a large device copy (HBM read + write bandwidth reference) and the per-row kernels.

Usage: python kbench.py [--rows 1,7,14] [--reps 3] [--json out.json]
       python kbench.py --no-gemm --rows 0 --split-rows 448,1792,3584 --tiles=-1,2,1 --ksplits=-1,0,1
"""
import argparse
import ctypes as C
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import nemoasr  # noqa: E402

# (label, N, K, act, accumulate, alpha, ln_mode, ldw, bias) as the chunk calls them
SHAPES = [
    ("ff_up+ln2", 4096, 1024, 1, 0, 1.0, 2, None, False),
    ("ff_down", 1024, 4096, 0, 1, 0.5, 0, None, False),
    ("qkv+ln", 3072, 1024, 0, 0, 1.0, 1, None, False),
    ("out_proj", 1024, 1024, 0, 1, 1.0, 0, None, False),
    ("pw1_glu+ln", 2048, 1024, 3, 0, 1.0, 1, None, False),
    ("pw2", 1024, 1024, 0, 1, 1.0, 0, None, False),
    ("prompt_w0+ln", 2048, 1024, 2, 0, 1.0, 1, 1152, True),
    ("prompt_w2", 1024, 2048, 0, 0, 1.0, 0, None, True),
    ("joint_enc", 640, 1024, 0, 0, 1.0, 0, None, True),
    ("lstm", 2560, 640, 0, 1, 1.0, 0, None, False),
]


def bench_gemm(gpu, M, N, K, act, acc, alpha, ln_mode, ldw, has_bias, copies, reps):
    L = nemoasr.lib()
    ldw = ldw or K
    rng = np.random.default_rng([M, N, K])
    nout = N // 2 if act == 3 else N
    W = (rng.standard_normal((N, ldw)).astype(np.float32) / np.float32(np.sqrt(K))).view(np.uint32) >> 16
    W = W.astype(np.uint16)
    dWs = [gpu.put(W) for _ in range(copies)]
    dA = gpu.put(rng.standard_normal((M, K)).astype(np.float32))
    dC = gpu.put(np.zeros((M, nout), np.float32))
    dB = gpu.put((0.1 * rng.standard_normal(N)).astype(np.float32))
    g = [gpu.put((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)) for _ in range(4)]
    dT = gpu.alloc(M * K * 4)
    dO = gpu.alloc(M * K * 4)

    def launch(i):
        return L.nk_gemm_ln(gpu.h, dA.ptr, K, dWs[i % copies].ptr, ldw, dB.ptr if has_bias else None, dC.ptr, nout, None, M, N, K, act, acc,
                            alpha, ln_mode, g[0].ptr, g[1].ptr, g[2].ptr, g[3].ptr, dO.ptr if ln_mode == 2 else None,
                            dT.ptr, 1e-5)

    name = L.nk_gemm_kernel_name(M, N, K, act).decode()
    if ln_mode and name.startswith("gemm_fr") and K == 1024:
        name = "gemm_fr_ln*"  # the LayerNorm-fused few-row kernels (nk_gemm_kernel_name names the plain GEMM's)
    # graph replay
    gpu.begin()
    gpu.check(L.gpu_capture_begin(gpu.h))
    for i in range(copies):
        gpu.check(launch(i))
    gr = L.gpu_capture_end(gpu.h)
    gpu.end()
    if not gr:
        raise RuntimeError(L.gpu_last_error(gpu.h).decode())
    best = 1e30
    for _ in range(reps + 1):
        gpu.begin()
        gpu.check(L.gpu_graph_launch(gpu.h, gr))
        best = min(best, gpu.end())
    L.gpu_graph_free(gr)
    graph_us = best * 1e3 / copies
    # dispatch-stamped kernel durations (direct launches)
    L.gpu_timing_set(gpu.h, b"gemm_fr*" if name.startswith("gemm_fr") else name.encode(), 4096)
    gpu.begin()
    for i in range(copies * reps):
        gpu.check(launch(i))
    gpu.end()
    ms, cnt, by = C.c_double(), C.c_int(), C.c_double()
    L.gpu_timing_collect(gpu.h, C.byref(ms), C.byref(cnt), C.byref(by))
    L.gpu_timing_set(gpu.h, None, 0)
    for b in dWs + [dA, dC, dB, dT, dO] + g:
        b.free()
    return name, graph_us, ms.value * 1e3, cnt.value


def graph_us(gpu, launch, copies, reps):
    """launch-to-launch time of `copies` launches replayed back to back in one hipGraph"""
    L = nemoasr.lib()
    gpu.begin()
    gpu.check(L.gpu_capture_begin(gpu.h))
    for i in range(copies):
        gpu.check(launch(i))
    gr = L.gpu_capture_end(gpu.h)
    gpu.end()
    if not gr:
        raise RuntimeError(L.gpu_last_error(gpu.h).decode())
    best = 1e30
    for _ in range(reps + 1):
        gpu.begin()
        gpu.check(L.gpu_graph_launch(gpu.h, gr))
        best = min(best, gpu.end())
    L.gpu_graph_free(gr)
    return best * 1e3 / copies


def bench_attention(gpu, c, cache, use_desc, copies, reps):
    """relative-position attention of one layer (8 heads x 128) over cache + c keys; a distinct
    K/V cache and position table per launch, as the 24 layers of a chunk"""
    L = nemoasr.lib()
    H, dh, D, Lmax = 8, 128, 1024, 72
    Lw = cache + c
    rng = np.random.default_rng([c, cache])
    pos = cache + 8
    kvs = [gpu.put(rng.standard_normal((pos + c, 3 * D)).astype(np.float32)) for _ in range(copies)]
    Ps = [gpu.put(rng.standard_normal((2 * Lmax - 1, D)).astype(np.float32)) for _ in range(copies)]
    bu, bv, dO = gpu.put(np.zeros(D, np.float32)), gpu.put(np.zeros(D, np.float32)), gpu.alloc(c * D * 4)
    desc = np.zeros(20, np.int32)
    desc[:4] = [pos, cache, Lw, c]
    ddesc = gpu.put(desc)
    row = 3 * D * 4
    scale = float(1.0 / np.sqrt(dh))

    def launch(i):
        kv, P = kvs[i % copies], Ps[i % copies]
        if use_desc:
            return L.nk_attention_rel_desc(gpu.h, kv.ptr, 3 * D, ddesc.ptr, P.ptr, bu.ptr, bv.ptr, dO.ptr, c, Lmax, H, dh,
                                           D, scale)
        return L.nk_attention_rel(gpu.h, kv.at(pos * row), 3 * D, kv.at((pos - cache) * row + D * 4),
                                  kv.at((pos - cache) * row + 2 * D * 4), 3 * D, P.ptr, bu.ptr, bv.ptr, dO.ptr, c, Lw,
                                  Lmax, H, dh, D, scale)

    us = graph_us(gpu, launch, copies, reps)
    for b in kvs + Ps + [bu, bv, dO, ddesc]:
        b.free()
    return us


def bench_dwconv(gpu, c, use_desc, copies, reps):
    L = nemoasr.lib()
    D, taps = 1024, 9
    rng = np.random.default_rng(c)
    dins = [gpu.put(rng.standard_normal((taps - 1 + c + 8, D)).astype(np.float32)) for _ in range(copies)]
    Ws = [gpu.put((rng.standard_normal((D, taps)) / 3).astype(np.float32)) for _ in range(copies)]
    g, b, dY = gpu.put(np.ones(D, np.float32)), gpu.put(np.zeros(D, np.float32)), gpu.alloc(c * D * 4)
    desc = np.zeros(20, np.int32)
    desc[:4] = [taps - 1 + 8, 0, c, c]
    ddesc = gpu.put(desc)

    def launch(i):
        if use_desc:
            return L.nk_dwconv_ln_silu_desc(gpu.h, dins[i % copies].ptr, ddesc.ptr, Ws[i % copies].ptr, g.ptr, b.ptr,
                                            dY.ptr, c, D, taps, 1e-5)
        return L.nk_dwconv_ln_silu(gpu.h, dins[i % copies].at(8 * D * 4), Ws[i % copies].ptr, g.ptr, b.ptr, dY.ptr, c,
                                   D, taps, 1e-5)

    us = graph_us(gpu, launch, copies, reps)
    for x in dins + Ws + [g, b, dY, ddesc]:
        x.free()
    return us


# the batched encoder's many-row GEMMs on split-row activations (K bf16 hi then K lo per row), as
# batch.c calls them: (label, N, K, act, kind) with kind "so" split-row output, "f" f32 output,
# "r" residual update left pending (nk_gemm_resid)
SPLIT_SHAPES = [("ff_up", 4096, 1024, 1, "so"), ("ff_down", 1024, 4096, 0, "r"), ("qkv", 3072, 1024, 0, "f"),
                ("pw1_glu", 2048, 1024, 3, "f"), ("out/pw2", 1024, 1024, 0, "r")]


def split_rows(x):
    """f32 rows -> split rows (RNE bf16 hi, then RNE bf16 of the remainder)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    hi = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = (x - (hi.astype(np.uint32) << 16).view(np.float32)).astype(np.float32).view(np.uint32)
    lo = ((r + 0x7FFF + ((r >> 16) & 1)) >> 16).astype(np.uint16)
    return np.concatenate([hi, lo], axis=1)


def bench_split(gpu, M, N, K, act, kind, copies, launches):
    """Mean kernel time (dispatch-stamped events, direct launches) and total flops of `launches`
    launches cycling `copies` weight matrices."""
    L = nemoasr.lib()
    rng = np.random.default_rng(1)
    A2 = gpu.put(split_rows(rng.standard_normal((M, K)).astype(np.float32)))
    Ws = [gpu.put(((rng.standard_normal((N, K)) * 0.03).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
          for _ in range(copies)]
    nout = N // 2 if act == 3 else N
    Cb = gpu.alloc(M * nout * 4 * (2 if kind == "so" else 1))
    pend = nemoasr.Resid()
    L.gpu_timing_set(gpu.h, b"gemm_mx*", launches)
    gpu.begin()
    for r in range(launches):
        W = Ws[r % copies].ptr
        if kind == "so":
            rc = L.nk_gemm_split(gpu.h, None, A2.ptr, 2 * K, W, K, None, None, Cb.ptr, 2 * nout, None, M, N, K, act, 0, 1.0)
        elif kind == "f":
            rc = L.nk_gemm_split(gpu.h, None, A2.ptr, 2 * K, W, K, None, Cb.ptr, None, nout, None, M, N, K, act, 0, 1.0)
        else:
            rc = L.nk_gemm_resid(gpu.h, None, A2.ptr, 2 * K, W, K, Cb.ptr, N, M, N, K, 1.0, C.byref(pend))
        gpu.check(rc)
    gpu.end()
    ms, cnt, by = C.c_double(), C.c_int(), C.c_double()
    L.gpu_timing_collect(gpu.h, C.byref(ms), C.byref(cnt), C.byref(by))
    fl = L.gpu_timing_last_flops(gpu.h)
    for b in Ws + [A2, Cb]:
        b.free()
    gpu._bufs = []
    return ms.value * 1e3, fl / max(cnt.value, 1)


def bench_floor(gpu, copies, reps):
    """The launch floor under both timings: a 256-float copy (one workgroup) replayed in a graph
    (graph_us) and timed by dispatch-stamped events around each direct launch (kernel_us), the
    method of bench.py's roofline; the fixed cost every GEMV measurement above includes."""
    L = nemoasr.lib()
    src, dst = gpu.alloc(1024 * copies), gpu.alloc(1024 * copies)
    gus = graph_us(gpu, lambda i: L.nk_copy(gpu.h, src.at(1024 * i), dst.at(1024 * i), 256), copies, reps)
    L.gpu_timing_set(gpu.h, b"copy_f32", 4096)
    gpu.begin()
    for i in range(copies * 4):
        gpu.check(L.nk_copy(gpu.h, src.at(1024 * (i % copies)), dst.at(1024 * (i % copies)), 256))
    gpu.end()
    ms, cnt, by = C.c_double(), C.c_int(), C.c_double()
    L.gpu_timing_collect(gpu.h, C.byref(ms), C.byref(cnt), C.byref(by))
    L.gpu_timing_set(gpu.h, None, 0)
    src.free()
    dst.free()
    return gus, ms.value * 1e3


def bench_copy(gpu, nbytes, reps):
    L = nemoasr.lib()
    n = nbytes // 4
    src, dst = gpu.alloc(nbytes), gpu.alloc(nbytes)
    best = 1e30
    for _ in range(reps + 1):
        gpu.begin()
        gpu.check(L.nk_copy(gpu.h, src.ptr, dst.ptr, n))
        best = min(best, gpu.end())
    src.free()
    dst.free()
    return best * 1e3


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--rows", default="1,7,14")
    ap.add_argument("--rows-force", default="0", help="few-row kernel selections to compare (nk_gemm_force: 0 policy, "
                    "2 few-row MFMA, 4 weight-streaming GEMV where it applies), e.g. 0,2")
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--copies", type=int, default=48, help="distinct weight matrices cycled per replay")
    ap.add_argument("--json", default=None)
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--batch-rows", default="", help="many-row (batched streams) GEMM sizes, e.g. 448,3584")
    ap.add_argument("--batch-force", default="0", help="kernel selections to compare (nk_gemm_force), e.g. 0,5")
    ap.add_argument("--split-rows", default="", help="many-row GEMMs on split-row activations, e.g. 448,1792,3584")
    ap.add_argument("--tiles", default="-1", help="many-row tiles to compare (nk_gemm_mx_tile: -1 policy, "
                                                  "0 128x128, 1 64x128, 2 64x64), e.g. -1,2,1")
    ap.add_argument("--ksplits", default="-1", help="residual K split modes to compare (nk_gemm_ksplit), e.g. -1,0,1")
    a = ap.parse_args()
    gpu = nemoasr.Gpu()
    print(f"device: {gpu.name}", flush=True)
    out = {"device": gpu.name, "gemm": [], "copy": None}
    cb = 256 << 20
    cu = bench_copy(gpu, cb, a.reps)
    out["copy"] = {"bytes": cb, "us": cu, "gbs_rw": 2 * cb / (cu * 1e-6) / 1e9}
    print(f"copy {cb >> 20} MiB: {cu:.1f} us, {2 * cb / (cu * 1e-6) / 1e9:.0f} GB/s read+write", flush=True)
    fg, fk = bench_floor(gpu, 48, a.reps)
    out["floor"] = {"graph_us": round(fg, 3), "kernel_us": round(fk, 3)}
    print(f"launch floor (1 KB copy): graph {fg:7.2f} us  kernel {fk:7.2f} us", flush=True)
    for M, force in ([] if a.no_gemm else [(int(x), int(f)) for x in a.rows.split(",") for f in a.rows_force.split(",")]):
        for (label, N, K, act, acc, alpha, ln, ldw, hb) in SHAPES:
            if label == "lstm" and M > 1:
                continue
            nemoasr.lib().nk_gemm_force(force)
            name, gus, kus, cnt = bench_gemm(gpu, M, N, K, act, acc, alpha, ln, ldw, hb, a.copies, a.reps)
            nemoasr.lib().nk_gemm_force(0)
            wb = 2.0 * N * K
            rec = {"M": M, "shape": label, "N": N, "K": K, "kernel": name, "graph_us": round(gus, 3),
                   "kernel_us": round(kus, 3), "weight_bytes": wb, "gbs_kernel": round(wb / (kus * 1e-6) / 1e9, 1),
                   "gbs_graph": round(wb / (gus * 1e-6) / 1e9, 1), "timed_launches": cnt}
            out["gemm"].append(rec)
            print(f"M={M:2d} {label:14s} {name:22s} graph {gus:7.2f} us ({rec['gbs_graph']:7.1f} GB/s)  "
                  f"kernel {kus:7.2f} us ({rec['gbs_kernel']:7.1f} GB/s)", flush=True)
    out["batched"] = []
    for M, force in [(int(x), int(f)) for x in a.batch_rows.split(",") if x for f in a.batch_force.split(",")]:
        nemoasr.lib().nk_gemm_force(force)
        tot_us, tot_fl = 0.0, 0.0
        for (label, N, K, act, acc, alpha, ln, ldw, hb) in SHAPES:
            if label == "lstm":
                continue
            name, gus, kus, cnt = bench_gemm(gpu, M, N, K, act, acc, alpha, 0, ldw, hb, 8, a.reps)
            fl = 2.0 * M * N * K
            per_layer = {"ff_up+ln2": 2, "ff_down": 2, "qkv+ln": 1, "out_proj": 1, "pw1_glu+ln": 1, "pw2": 1}.get(label, 0)
            cnt_chunk = 24 * per_layer if per_layer else 1
            tot_us += gus * cnt_chunk
            tot_fl += fl * cnt_chunk
            rec = {"M": M, "shape": label, "N": N, "K": K, "kernel": name, "graph_us": round(gus, 3),
                   "tflops": round(fl / (gus * 1e-6) / 1e12, 1), "mfma_frac": round(fl / (gus * 1e-6) / 2.5e15, 4)}
            rec["force"] = force
            out["batched"].append(rec)
            print(f"M={M:5d} f{force} {label:14s} {name:18s} graph {gus:8.2f} us  {rec['tflops']:7.1f} TFLOP/s "
                  f"({rec['mfma_frac']:.3f} of 2.5 PF bf16; issued MFMA work is 2x: A = hi + lo)", flush=True)
        nemoasr.lib().nk_gemm_force(0)
        print(f"M={M:5d} f{force} chunk GEMMs (24 layers + prompt + joint.enc, no LN launches): {tot_us / 1e3:.3f} ms, "
              f"{tot_fl / (tot_us * 1e-6) / 1e12:.1f} TFLOP/s = {tot_fl / (tot_us * 1e-6) / 2.5e15:.3f} of peak", flush=True)
    out["split"] = []
    L = nemoasr.lib()
    for M in [int(x) for x in a.split_rows.split(",") if x]:
        for (label, N, K, act, kind) in SPLIT_SHAPES:
            for tile in [int(t) for t in a.tiles.split(",")]:
                for ks in ([int(k) for k in a.ksplits.split(",")] if kind == "r" else [-1]):
                    L.nk_gemm_mx_tile(tile)
                    L.nk_gemm_ksplit(ks)
                    us, fl = bench_split(gpu, M, N, K, act, kind, 8, 64)
                    tf = fl / (us * 1e-6) / 1e12
                    out["split"].append({"M": M, "shape": label, "N": N, "K": K, "tile": tile, "ksplit": ks,
                                         "kernel_us": round(us, 3), "tflops": round(tf, 1)})
                    print(f"M={M:5d} {label:8s} tile {tile:2d} ksplit {ks:2d}  kernel {us:7.2f} us  {tf:6.1f} TFLOP/s "
                          f"({tf / 2500:.3f} of 2.5 PF bf16)", flush=True)
            L.nk_gemm_mx_tile(-1)
            L.nk_gemm_ksplit(-1)
    out["rows"] = []
    for c in [int(x) for x in a.rows.split(",") if 0 < int(x) <= 16]:
        for desc in (0, 1):
            us = bench_attention(gpu, c, 56, desc, 24, a.reps)
            out["rows"].append({"kernel": "attention_rel", "c": c, "cache": 56, "desc": desc, "graph_us": round(us, 3)})
            print(f"c={c:2d} attention_rel cache 56 desc={desc} graph {us:7.2f} us", flush=True)
        for desc in (0, 1):
            us = bench_dwconv(gpu, c, desc, 24, a.reps)
            out["rows"].append({"kernel": "dwconv_ln_silu", "c": c, "desc": desc, "graph_us": round(us, 3)})
            print(f"c={c:2d} dwconv_ln_silu  desc={desc} graph {us:7.2f} us", flush=True)
    gpu.close()
    if a.json:
        with open(a.json, "w") as f:
            json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
