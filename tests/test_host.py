"""Host side of the path on the CPU (no GPU calls).

- The product library loads and exports every function include/*.h declares.
- The product's streaming log-mel front end, resampler, encoder-step bookkeeping and piece text
  agree with the oracle, and, where oracle/_ref was built from the reference's own sources
  (src/mel.c, src/resample.c, src/tokenizer.c, src/json.c), with the reference itself.  The same
  comparison pins oracle/mel_ref.py to the reference's front end.
- nemoasr_open fails with a message, not a fallback, when no GPU is present.
"""
import ctypes as C
import glob
import os
import re

import numpy as np
import pytest

import mel_ref
import oracle
import synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SO = os.path.join(REPO, "oracle", "_ref", "libref_host.so")
_f32p = C.POINTER(C.c_float)


def product():
    import nemoasr

    return nemoasr.lib()


def ref_lib():
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (the reference sources are not present)")
    L = C.CDLL(REF_SO)
    L.mel_create.restype = C.c_void_p
    L.mel_destroy.argtypes = [C.c_void_p]
    L.mel_push.argtypes = [C.c_void_p, _f32p, C.c_size_t, C.c_int, C.POINTER(_f32p), C.POINTER(C.c_size_t)]
    L.resampler_create.restype = C.c_void_p
    L.resampler_create.argtypes = [C.c_int, C.c_int]
    L.resampler_destroy.argtypes = [C.c_void_p]
    L.resampler_process.restype = C.c_size_t
    L.resampler_process.argtypes = [C.c_void_p, _f32p, C.c_size_t, _f32p, C.c_size_t]
    L.resampler_flush.restype = C.c_size_t
    L.resampler_flush.argtypes = [C.c_void_p, _f32p, C.c_size_t]
    L.tok_text.restype = C.c_void_p
    L.tok_text.argtypes = [C.c_void_p, C.c_int]
    return L


# ---- exports -----------------------------------------------------------------------------------
def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\([^;{]*\)\s*;", text, flags=re.M):
            if not m.group(0).lstrip().startswith(("typedef", "return")):
                names.add(m.group(1))
    return sorted(names)


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(names) > 40 and "nemoasr_open" in names and "nk_gemm" in names
    L = product()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_every_kernel_takes_one_argument_block():
    """gpu_launch hands each kernel one by-value argument block (kernelParams = { &block }), so every
    kernel in the gfx950 code object must declare exactly one explicit argument; a second one would
    be read from an unset pointer.  Read from the metadata of the code object built here."""
    import shutil
    import subprocess
    import yaml

    co = os.path.join(REPO, "nemo-c_amd", "build", "nk_all.hsaco")
    llvm = "/opt/rocm/llvm/bin"
    if not os.path.exists(co) or not shutil.which(os.path.join(llvm, "llvm-readelf")):
        pytest.skip("code object or LLVM tools not present")
    elf = os.path.join(REPO, "nemo-c_amd", "build", "nk_all.gfx950.elf")
    subprocess.run([os.path.join(llvm, "clang-offload-bundler"), "--unbundle", "--type=o", f"--input={co}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={elf}"], check=True)
    notes = subprocess.run([os.path.join(llvm, "llvm-readelf"), "--notes", elf], check=True, capture_output=True,
                           text=True).stdout
    meta = yaml.safe_load(notes[notes.index("---"):notes.index("\n...", notes.index("---"))])
    kernels = meta["amdhsa.kernels"]
    assert len(kernels) > 100
    bad = {k[".name"]: len([a for a in k.get(".args", []) if not a[".value_kind"].startswith("hidden")])
           for k in kernels}
    bad = {n: c for n, c in bad.items() if c != 1}
    assert not bad, bad


def test_reference_runtime_header_compiles_and_links(tmp_path):
    """include/nemo_gpu.h and include/nemo_kernel_params.h: a host unit written the way the
    reference's launchers are (src/model.c:70-111: GemmParams by value, GPU_BUF / GPU_BYTES,
    gpu_dispatch_groups_fc with function constants) compiles with gcc, the parameter blocks have the
    reference's layout (src/kernel_params.h:22-32), and the program links against the library and
    runs (gpu_create takes the reference's source argument and fails cleanly without a GPU)."""
    import shutil
    import subprocess

    if not shutil.which("gcc"):
        pytest.skip("gcc not present")
    src = tmp_path / "refhost.c"
    src.write_text(r"""
#include <stddef.h>
#include <stdio.h>
#include "nemo_gpu.h"
#include "nemo_kernel_params.h"
_Static_assert(sizeof(GemmParams) == 40 && offsetof(GemmParams, has_bias) == 24 && offsetof(GemmParams, alpha) == 36, "GemmParams");
_Static_assert(sizeof(LnParams) == 12 && offsetof(LnParams, eps) == 8, "LnParams");
_Static_assert(sizeof(AttnParams) == 36 && offsetof(AttnParams, ldk) == 28 && offsetof(AttnParams, scale) == 32, "AttnParams");
_Static_assert(sizeof(GluParams) == 8 && sizeof(DwParams) == 16 && offsetof(DwParams, eps) == 12, "Glu/Dw");
_Static_assert(sizeof(Conv2dParams) == 20 && sizeof(FlatParams) == 12 && sizeof(CountParams) == 4, "conv");
_Static_assert(sizeof(FillParams) == 8 && sizeof(LstmParams) == 4 && sizeof(JointParams) == 16, "misc");
_Static_assert(sizeof(gpu_arg_t) == 4 * sizeof(void *), "gpu_arg_t");
static int k_gemm_like(gpu_t *g, gpu_buf_t *A, gpu_buf_t *W, gpu_buf_t *C) {
    GemmParams p = { 7, 4096, 1024, 1024, 1024, 4096, 0, 1, 0, 1.0f };
    gpu_arg_t args[5] = { GPU_BUF(A, 0), GPU_BUF(W, 0), GPU_BUF(A, 0), GPU_BUF(C, 0), GPU_BYTES(&p) };
    uint32_t fc[7] = { 7, 0, 0, 1, 2, 8, 32 };
    return gpu_dispatch_groups_fc(g, "gemm_mma", fc, 7, args, 5, 256, 1, 1, 256, 1, 1);
}
int main(void) {
    char err[256] = "";
    gpu_t *g = gpu_create("metal source text", err, sizeof err);
    if (g) { gpu_buf_t *b = gpu_buf_alloc(g, 64); (void)gpu_buf_ptr(b); (void)k_gemm_like; gpu_buf_free(b); gpu_destroy(g); return 2; }
    printf("%s\n", err);
    return err[0] ? 0 : 1;
}
""")
    exe = tmp_path / "refhost"
    pkg = os.path.join(REPO, "nemo-c_amd")
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe),
                    "-L", pkg, "-lnemoasr_hip", f"-Wl,-rpath,{pkg}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    if r.returncode == 2:
        pytest.skip("a GPU is present: the no-device path is not exercised")
    assert r.returncode == 0, r.stdout + r.stderr


def test_open_without_gpu_fails_loudly(tiny_model_dir):
    import torch

    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present")
    L = product()
    err = C.create_string_buffer(512)
    h = L.nemoasr_open(tiny_model_dir.encode(), b"en-US", 560, 16000, err, 512)
    assert not h
    assert err.value, "nemoasr_open must say why it failed"
    L.nemoasr_batch_open.restype = C.c_void_p
    err = C.create_string_buffer(512)
    h = L.nemoasr_batch_open(tiny_model_dir.encode(), b"en-US", 560, 8, err, 512)
    assert not h
    assert err.value, "nemoasr_batch_open must say why it failed"


def test_batch_open_rejects_bad_arguments(tiny_model_dir):
    L = product()
    L.nemoasr_batch_open.restype = C.c_void_p
    for lat, n in ((500, 4), (560, 0), (560, 5000)):
        err = C.create_string_buffer(512)
        assert not L.nemoasr_batch_open(tiny_model_dir.encode(), b"en-US", lat, n, err, 512)
        assert err.value


# ---- log-mel front end -------------------------------------------------------------------------
def product_mel(x, pieces):
    L = product()
    m = L.melfe_create()
    out, pos = [], 0
    for i, n in enumerate(pieces):
        seg = np.ascontiguousarray(x[pos:pos + n], np.float32)
        pos += n
        fr, nf = _f32p(), C.c_size_t()
        L.melfe_push(m, seg.ctypes.data_as(_f32p), seg.size, int(pos >= x.size), C.byref(fr), C.byref(nf))
        if nf.value:
            out.append(np.ctypeslib.as_array(fr, shape=(nf.value * 128,)).reshape(-1, 128).copy())
    L.melfe_destroy(m)
    return np.concatenate(out) if out else np.zeros((0, 128), np.float32)


def ref_mel(R, x, pieces):
    m = R.mel_create()
    out, pos = [], 0
    for n in pieces:
        seg = np.ascontiguousarray(x[pos:pos + n], np.float32)
        pos += n
        fr, nf = _f32p(), C.c_size_t()
        R.mel_push(m, seg.ctypes.data_as(_f32p), seg.size, int(pos >= x.size), C.byref(fr), C.byref(nf))
        if nf.value:
            out.append(np.ctypeslib.as_array(fr, shape=(nf.value * 128,)).reshape(-1, 128).copy())
    R.mel_destroy(m)
    return np.concatenate(out) if out else np.zeros((0, 128), np.float32)


def split(n, sizes):
    out, i = [], 0
    while n > 0:
        k = min(n, sizes[i % len(sizes)])
        out.append(k)
        n -= k
        i += 1
    return out or [0]


MEL_TOL = 1e-3  # absolute, the reference's own front-end gate (tools/compare.py:19-21)


@pytest.mark.parametrize("seconds,sizes", [(1.0, [16000]), (2.3, [1600]), (1.7, [1, 159, 4000, 77]), (0.02, [320])])
def test_mel_product_vs_oracle(seconds, sizes):
    x = synth.make_audio(seconds, seed=21)
    got = product_mel(x, split(x.size, sizes))
    ref = mel_ref.logmel(x, final=True)
    assert got.shape == ref.shape
    assert np.max(np.abs(got - ref)) < MEL_TOL


@pytest.mark.parametrize("seconds,sizes", [(1.0, [16000]), (2.3, [1600]), (1.7, [1, 159, 4000, 77]), (0.02, [320])])
def test_mel_reference_pins_oracle_and_product(seconds, sizes):
    R = ref_lib()
    x = synth.make_audio(seconds, seed=22)
    ref = ref_mel(R, x, split(x.size, sizes))
    orc = mel_ref.logmel(x, final=True)
    got = product_mel(x, split(x.size, sizes))
    assert ref.shape == orc.shape == got.shape
    assert np.max(np.abs(orc - ref)) < MEL_TOL
    assert np.max(np.abs(got - ref)) < 1e-5  # measured: bit-identical on these clips


def test_mel_partial_stream_matches_reference():
    """Without the final flush only fully-covered frames come out, in both implementations."""
    R = ref_lib()
    x = synth.make_audio(1.0, seed=23)[:12345]
    m1, m2 = R.mel_create(), product().melfe_create()
    seg = np.ascontiguousarray(x, np.float32)
    f1, n1, f2, n2 = _f32p(), C.c_size_t(), _f32p(), C.c_size_t()
    R.mel_push(m1, seg.ctypes.data_as(_f32p), seg.size, 0, C.byref(f1), C.byref(n1))
    product().melfe_push(m2, seg.ctypes.data_as(_f32p), seg.size, 0, C.byref(f2), C.byref(n2))
    assert n1.value == n2.value > 0
    a = np.ctypeslib.as_array(f1, shape=(n1.value * 128,))
    b = np.ctypeslib.as_array(f2, shape=(n2.value * 128,))
    assert np.max(np.abs(a - b)) < MEL_TOL
    R.mel_destroy(m1)
    product().melfe_destroy(m2)


# ---- resampler ---------------------------------------------------------------------------------
def run_resampler(create, process, flush, destroy, x, rate, pieces):
    r = create(rate, 16000)
    out = []
    buf = np.zeros(1 << 20, np.float32)
    pos = 0
    for n in pieces:
        seg = np.ascontiguousarray(x[pos:pos + n], np.float32)
        pos += n
        k = process(r, seg.ctypes.data_as(_f32p), seg.size, buf.ctypes.data_as(_f32p), buf.size)
        out.append(buf[:k].copy())
    k = flush(r, buf.ctypes.data_as(_f32p), buf.size)
    out.append(buf[:k].copy())
    destroy(r)
    return np.concatenate(out)


@pytest.mark.parametrize("rate", [8000, 22050, 44100, 48000])
def test_resampler_matches_reference(rate):
    R = ref_lib()
    L = product()
    rng = np.random.default_rng(rate)
    x = (0.1 * rng.standard_normal(int(0.7 * rate))).astype(np.float32)
    pieces = split(x.size, [rate // 10, 333, 1])
    ref = run_resampler(R.resampler_create, R.resampler_process, R.resampler_flush, R.resampler_destroy, x, rate, pieces)
    got = run_resampler(L.rsmp_create, L.rsmp_process, L.rsmp_flush, L.rsmp_destroy, x, rate, pieces)
    assert got.shape == ref.shape
    assert np.max(np.abs(got - ref)) < 1e-5


# ---- token text --------------------------------------------------------------------------------
PIECES = ["▁the", "s", "▁", "<unk>", "<pad>", "<s>", "</s>", "<en-US>", "<de-DE>", "<xx>", "▁▁a▁b", "ab▁", "<0x41>",
          "é", "▁日本", "<en-us>", "<en-USA>"]


def test_piece_text_matches_reference():
    R = ref_lib()
    L = product()
    arr = (C.c_char_p * len(PIECES))(*[p.encode() for p in PIECES])

    class Vocab(C.Structure):
        _fields_ = [("pieces", C.POINTER(C.c_char_p)), ("count", C.c_int)]

    v = Vocab(C.cast(arr, C.POINTER(C.c_char_p)), len(PIECES))
    libc = C.CDLL(None)
    libc.free.argtypes = [C.c_void_p]
    for i, p in enumerate(PIECES):
        t = R.tok_text(C.byref(v), i)
        want = C.string_at(t)
        libc.free(t)
        out = C.create_string_buffer(256)
        assert L.nemo_piece_text(p.encode(), 0, out, 256) == 0
        assert out.value == want, p


# ---- encoder-step bookkeeping ------------------------------------------------------------------
@pytest.mark.parametrize("chunk_mel", [8, 56, 112])
def test_enc_plan_product_vs_oracle(chunk_mel):
    L = product()
    for n in (1, 7, 8, 9, 63, 200):
        for batch in (1, 13, 1000):
            b = oracle.EncBook(0, 0, 0, 0, 0)
            st = [0, 0, 0, 0, 0]
            fed = 0
            while True:
                if fed < n:
                    k = min(batch, n - fed)
                    fed += k
                    b.pending_n += k
                    st[0] += k
                final = fed >= n
                while True:
                    p = oracle.enc_plan(b, final, chunk_mel)
                    plan = (C.c_int * 8)()
                    so = (C.c_int * 5)()
                    ran = L.nemo_enc_plan(plan, st[0], st[1], st[2], st[3], st[4], int(final), chunk_mel, 8, 16, so)
                    assert ran == p.ran
                    assert list(plan) == [p.ran, p.take, p.nwin, p.lo, p.hi, p.c, p.include_boundary, p.T3]
                    st = list(so)
                    assert st == [b.pending_n, b.consumed, b.emitted, b.mel_cache_n, b.closed]
                    if not ran:
                        break
                if final and b.closed:
                    break


class _CkTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int), ("numel", C.c_size_t), ("at", C.c_uint64),
                ("bytes", C.c_uint64)]


def _ckpt_lib():
    L = product()
    L.ckpt_open.restype = C.c_void_p
    L.ckpt_open.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
    L.ckpt_close.argtypes = [C.c_void_p]
    L.ckpt_count.restype = C.c_size_t
    L.ckpt_count.argtypes = [C.c_void_p]
    L.ckpt_find.restype = C.POINTER(_CkTensor)
    L.ckpt_find.argtypes = [C.c_void_p, C.c_char_p]
    L.ckpt_read.argtypes = [C.c_void_p, C.POINTER(_CkTensor), C.c_void_p]
    return L


def _write_st(path, header: dict, payload: bytes):
    import json
    import struct

    hj = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)) + hj + payload)


def test_checkpoint_index_reads_tensors(tmp_path):
    """The product's checkpoint index (pread, sorted lookup) gives every tensor of a synthetic
    checkpoint with the shape, dtype and bytes a plain reader finds."""
    from conftest import model_dir

    L = _ckpt_lib()
    path = os.path.join(model_dir("tiny"), "model.safetensors")
    ref = synth.load_safetensors(path)
    err = C.create_string_buffer(256)
    h = L.ckpt_open(path.encode(), err, 256)
    assert h, err.value
    try:
        assert L.ckpt_count(h) == len(ref)
        for name in sorted(ref)[::7] + ["prompt_kernel.0.weight", "joint.joint_net.2.bias"]:
            raw, shape = ref[name]
            t = L.ckpt_find(h, name.encode())
            assert t and t.contents.dtype == 0 and t.contents.numel == int(np.prod(shape))
            out = np.empty(raw.size, np.uint16)
            assert L.ckpt_read(h, t, out.ctypes.data) == 0
            np.testing.assert_array_equal(out, raw)
        assert not L.ckpt_find(h, b"no.such.tensor")
        assert not L.ckpt_find(h, b"")
    finally:
        L.ckpt_close(h)


@pytest.mark.parametrize("case", ["past_end", "length_mismatch", "header_length", "duplicate", "not_object"])
def test_checkpoint_index_rejects_bad_files(tmp_path, case):
    L = _ckpt_lib()
    p = str(tmp_path / "bad.safetensors")
    ok = {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 12]}
    if case == "past_end":
        _write_st(p, {"a": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 12]}}, b"\0" * 8)
    elif case == "length_mismatch":
        _write_st(p, {"a": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 12]}}, b"\0" * 12)
    elif case == "header_length":
        with open(p, "wb") as f:
            f.write((1 << 40).to_bytes(8, "little") + b"{}")
    elif case == "duplicate":
        import struct

        hj = b'{"a": ' + str(ok).replace("'", '"').encode() + b', "a": ' + str(ok).replace("'", '"').encode() + b"}"
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", len(hj)) + hj + b"\0" * 12)
    else:
        with open(p, "wb") as f:
            f.write((2).to_bytes(8, "little") + b"[]")
    err = C.create_string_buffer(256)
    assert not L.ckpt_open(p.encode(), err, 256)
    assert err.value, case


def test_default_model_dir(tmp_path, monkeypatch):
    """nemoasr_default_model_dir: the Hugging Face cache snapshot that holds model.safetensors
    (src/nemoasr.h:23-25), -1 when there is none."""
    L = product()
    L.nemoasr_default_model_dir.restype = C.c_int
    L.nemoasr_default_model_dir.argtypes = [C.c_char_p, C.c_size_t]
    monkeypatch.setenv("HOME", str(tmp_path))
    out = C.create_string_buffer(4096)
    assert L.nemoasr_default_model_dir(out, 4096) == -1
    snaps = tmp_path / ".cache/huggingface/hub/models--mlx-community--nemotron-3.5-asr-streaming-0.6b/snapshots"
    (snaps / "aaa").mkdir(parents=True)  # a snapshot without the weights is skipped
    (snaps / "bbb").mkdir()
    (snaps / "bbb" / "model.safetensors").write_bytes(b"")
    assert L.nemoasr_default_model_dir(out, 4096) == 0
    assert out.value.decode() == str(snaps / "bbb")
    assert L.nemoasr_default_model_dir(out, 8) == -1  # does not fit
