"""ctypes binding of libnemoasr_hip.so for tests, the benchmark and smoke checks.

Exposes the public API (include/nemoasr.h), the multi-stream batch API (include/nemoasr_batch.h),
the test hooks (include/nemoasr_debug.h), the
kernel-level C ABI (include/nemo_kernels.h) and the exported host helpers
(include/nemoasr_host.h).  Loading the library needs no GPU; creating a session or a device
context does, and fails loudly without one — there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnemoasr_hip.so")

_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int)
_u16p = C.POINTER(C.c_uint16)
_vp = C.c_void_p
_u32 = C.c_uint32

_lib = None

# exported entry points: name -> (restype, argtypes)
API = {
    # include/nemoasr.h
    "nemoasr_default_model_dir": (C.c_int, [C.c_char_p, C.c_size_t]),
    "nemoasr_open": (_vp, [C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.c_char_p, C.c_size_t]),
    "nemoasr_close": (None, [_vp]),
    "nemoasr_feed": (_vp, [_vp, _f32p, C.c_size_t, C.c_int, C.c_char_p, C.c_size_t]),
    "nemoasr_free": (None, [_vp]),
    "nemoasr_reset": (C.c_int, [_vp, C.c_char_p, C.c_int, C.c_char_p, C.c_size_t]),
    "nemoasr_prepare_latency": (C.c_int, [_vp, C.c_int, C.c_char_p, C.c_size_t]),
    "nemoasr_load_ms": (C.c_double, [_vp]),
    "nemoasr_gpu_name": (C.c_char_p, [_vp]),
    "nemoasr_latency_ms": (C.c_int, [_vp]),
    "nemoasr_stats": (None, [_vp, _vp]),
    # include/nemoasr_batch.h
    "nemoasr_batch_open": (_vp, [C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.c_char_p, C.c_size_t]),
    "nemoasr_batch_close": (None, [_vp]),
    "nemoasr_batch_streams": (C.c_int, [_vp]),
    "nemoasr_batch_push": (C.c_int, [_vp, C.c_int, _f32p, C.c_size_t, C.c_int, C.c_char_p, C.c_size_t]),
    "nemoasr_batch_push_mel": (C.c_int, [_vp, C.c_int, _f32p, C.c_size_t, C.c_int, C.c_char_p, C.c_size_t]),
    "nemoasr_batch_step": (C.c_int, [_vp, C.c_char_p, C.c_size_t]),
    "nemoasr_batch_run": (C.c_int, [_vp, C.c_char_p, C.c_size_t]),
    "nemoasr_batch_tokens": (_i32p, [_vp, C.c_int, C.POINTER(C.c_size_t)]),
    "nemoasr_batch_text": (_vp, [_vp, C.c_int]),
    "nemoasr_batch_reset_stream": (C.c_int, [_vp, C.c_int, C.c_char_p, C.c_size_t]),
    "nemoasr_batch_stats": (None, [_vp, _vp]),
    "nemoasr_batch_step_ms": (C.POINTER(C.c_double), [_vp, C.POINTER(C.c_size_t)]),
    "nemoasr_batch_debug_use_graphs": (None, [_vp, C.c_int]),
    "nemoasr_batch_debug_gpu_frontend": (C.c_int, [_vp, C.c_int]),
    "nemoasr_batch_debug_set_dump": (None, [_vp, C.c_int]),
    "nemoasr_batch_debug_device_decoder": (C.c_int, [_vp, C.c_int]),
    "nemoasr_batch_debug_joint_enc": (_f32p, [_vp, C.c_int, C.POINTER(C.c_size_t)]),
    "nemoasr_batch_debug_time_kernel": (C.c_int, [_vp, C.c_char_p, C.c_int]),
    "nemoasr_batch_debug_kernel_ms": (C.c_int, [_vp, C.POINTER(C.c_double), C.POINTER(C.c_int),
                                                C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    # include/nemoasr_debug.h
    "nemoasr_debug_feed_mel": (C.c_int, [_vp, _f32p, C.c_size_t, C.c_int, C.c_char_p, C.c_size_t]),
    "nemoasr_debug_tokens": (_i32p, [_vp, C.POINTER(C.c_size_t)]),
    "nemoasr_debug_set_dump": (None, [_vp, C.c_int]),
    "nemoasr_debug_frames": (C.c_size_t, [_vp]),
    "nemoasr_debug_dump_layers": (_f32p, [_vp]),
    "nemoasr_debug_dump_prompted": (_f32p, [_vp]),
    "nemoasr_debug_dump_mel": (_f32p, [_vp, C.POINTER(C.c_size_t)]),
    "nemoasr_debug_dump_joint_enc": (_f32p, [_vp]),
    "nemoasr_debug_use_graphs": (None, [_vp, C.c_int]),
    "nemoasr_debug_fuse": (None, [_vp, C.c_int]),
    "nemoasr_debug_chain": (None, [_vp, C.c_int]),
    "nemoasr_debug_default_graphs": (None, [C.c_int]),
    "nemoasr_debug_chain_usable": (C.c_int, [_vp]),
    "nemoasr_debug_chain_spin": (None, [_vp, C.c_uint]),
    "nemoasr_debug_joint_steps": (C.c_size_t, [_vp]),
    "nemoasr_debug_encoder_gpu_ms": (C.c_double, [_vp]),
    "nemoasr_debug_chunk_ms": (C.POINTER(C.c_double), [_vp, C.POINTER(C.c_size_t)]),
    "nemoasr_debug_time_kernel": (C.c_int, [_vp, C.c_char_p, C.c_int]),
    "nemoasr_debug_kernel_ms": (C.c_int, [_vp, C.POINTER(C.c_double), C.POINTER(C.c_int), C.POINTER(C.c_double)]),
    "nemoasr_debug_weight_bytes": (C.c_size_t, [_vp]),
    "nemoasr_debug_launches": (C.c_uint64, [_vp]),
    # include/nemo_kernels.h
    "gpu_create": (_vp, [C.c_char_p, C.c_char_p, C.c_size_t]),
    "gpu_destroy": (None, [_vp]),
    "gpu_device_name": (C.c_char_p, [_vp]),
    "gpu_buf_alloc": (_vp, [_vp, C.c_size_t]),
    "gpu_buf_free": (None, [_vp]),
    "gpu_buf_dptr": (_vp, [_vp]),
    "gpu_buf_len": (C.c_size_t, [_vp]),
    "gpu_upload": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
    "gpu_download": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
    "gpu_begin": (C.c_int, [_vp]),
    "gpu_end": (C.c_int, [_vp, C.c_char_p, C.c_size_t]),
    "gpu_last_ms": (C.c_double, [_vp]),
    "gpu_last_error": (C.c_char_p, [_vp]),
    "gpu_timing_set": (C.c_int, [_vp, C.c_char_p, C.c_int]),
    "gpu_timing_collect": (C.c_int, [_vp, C.POINTER(C.c_double), C.POINTER(C.c_int), C.POINTER(C.c_double)]),
    "gpu_timing_last_flops": (C.c_double, [_vp]),
    "gpu_launch_count": (C.c_uint64, [_vp]),
    "gpu_capture_begin": (C.c_int, [_vp]),
    "gpu_capture_end": (_vp, [_vp]),
    "gpu_graph_launch": (C.c_int, [_vp, _vp]),
    "gpu_graph_free": (None, [_vp]),
    "nk_gemm": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32, C.c_int, C.c_int, C.c_float]),
    "nk_gemm_rows": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _u32, _vp, _u32, _u32, _u32, C.c_int, C.c_int,
                               C.c_float]),
    "nk_gemm_ln": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _u32, _vp, _u32, _u32, _u32, C.c_int, C.c_int,
                             C.c_float, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp, C.c_float]),
    "nk_gemm_force": (C.c_int, [C.c_int]),
    "nk_gemm_ksplit": (C.c_int, [C.c_int]),
    "nk_gemm_mx_tile": (C.c_int, [C.c_int]),
    "nk_gemm_fr_ksplit": (C.c_int, [C.c_int]),
    "nk_gemm_split": (C.c_int, [_vp, _vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32, C.c_int,
                                C.c_int, C.c_float]),
    "nk_gemm_split_noalloc": (C.c_int, [_vp, _vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32,
                                        C.c_int, C.c_int, C.c_float]),
    "nk_layernorm2_split": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, C.c_float]),
    "nk_gemm_resid": (C.c_int, [_vp, _vp, _vp, _u32, _vp, _u32, _vp, _u32, _u32, _u32, _u32, C.c_float, _vp]),
    "nk_resid_fold": (C.c_int, [_vp, _vp, _u32, _u32, _u32, _vp]),
    "nk_gemm_pend": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _u32, _u32, _u32, _u32, C.c_float, _vp]),
    "nk_gemm_ln_pend": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _u32, _vp, _u32, _u32, _u32, C.c_int, C.c_int,
                                  C.c_float, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _vp]),
    "nk_attention_out_desc_pend": (C.c_int, [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, C.c_float,
                                             _vp, _u32, C.c_float, _vp]),
    "nk_attention_rel_chunks_split": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                                _u32, C.c_float]),
    "nk_dwconv_ln_silu_rows_split": (C.c_int, [_vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _u32, C.c_float]),
    "nk_gemm_argmax": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32, _u32]),
    "nk_gemm_argmax_rows": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp, _u32]),
    "nk_gemm_kernel_name": (C.c_char_p, [_u32, _u32, _u32, C.c_int]),
    "nk_layernorm": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, C.c_float]),
    "nk_layernorm2": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, C.c_float]),
    "nk_attention_rel": (C.c_int, [_vp, _vp, _u32, _vp, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
                                   _u32, C.c_float]),
    "nk_attention_rel_desc": (C.c_int, [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
                                        C.c_float]),
    "nk_dwconv_ln_silu": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, C.c_float]),
    "nk_dwconv_ln_silu_desc": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, C.c_float]),
    "nk_attention_out_desc": (C.c_int, [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, C.c_float,
                                        _vp, _u32, _vp, _u32, C.c_float]),
    "nk_dwconv_pw_desc": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _u32, _vp, _u32, _u32, _u32, _u32,
                                    C.c_int, C.c_float]),
    "nk_fuse_shape": (C.c_int, [C.c_int, C.c_int]),
    "nk_mel_frames": (C.c_int, [_vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "nk_scatter_rows": (C.c_int, [_vp, _vp, _u32, _vp, _vp, _u32, _u32, _u32]),
    "nk_conv2d_c1_s2_relu": (C.c_int, [_vp, _vp, _vp, _vp, _vp] + [_u32] * 5),
    "nk_dwconv2d_s2": (C.c_int, [_vp, _vp, _vp, _vp, _vp] + [_u32] * 5),
    "nk_flatten_cf": (C.c_int, [_vp, _vp, _vp, _u32, _u32, _u32]),
    "nk_copy": (C.c_int, [_vp, _vp, _vp, _u32]),
    "nk_copy2d": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _u32, _u32]),
    "nk_fill": (C.c_int, [_vp, _vp, _u32, C.c_float]),
    "nk_compact": (C.c_int, [_vp, _vp, C.c_uint64, _u32, _u32, _u32, _u32, _u32]),
    "nk_attention_rel_rows": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                        C.c_float]),
    "nk_attention_rel_chunks": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                          C.c_float]),
    "nk_dwconv_ln_silu_rows": (C.c_int, [_vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, C.c_float]),
    "nk_conv2d_c1_s2_relu_b": (C.c_int, [_vp, _vp, _vp, _vp, _vp] + [_u32] * 6),
    "nk_dwconv2d_s2_b": (C.c_int, [_vp, _vp, _vp, _vp, _vp] + [_u32] * 6),
    "nk_conv2d_c1_dw_s2_b": (C.c_int, [_vp] * 7 + [_u32] * 8),
    "nk_flatten_cf_b": (C.c_int, [_vp, _vp, _vp, _u32, _u32, _u32, _u32]),
    "nk_gather_rows": (C.c_int, [_vp, _vp, _u32, _vp, _vp, _u32, _u32, _u32]),
    "nk_lstm_input_rows": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32]),
    "nk_lstm_cell_rows": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32]),
    "nk_joint_in_rows": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32]),
    "nk_argmax_rows": (C.c_int, [_vp, _vp, _u32, _u32, _u32, _vp]),
    "nk_glu": (C.c_int, [_vp, _vp, _vp, _u32, _u32]),
    "nk_lstm_cell": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _u32]),
    "nk_joint_partial": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32]),
    "nk_argmax_reduce": (C.c_int, [_vp, _vp, _vp, _vp, _u32, _u32]),
    # include/nemo_gpu.h (the reference's runtime interface; gpu_arg_t arrays are GpuArg below)
    "gpu_buf_ptr": (_vp, [_vp]),
    "gpu_dispatch": (C.c_int, [_vp, C.c_char_p, _vp, C.c_int] + [_u32] * 6),
    "gpu_dispatch_groups": (C.c_int, [_vp, C.c_char_p, _vp, C.c_int] + [_u32] * 6),
    "gpu_dispatch_groups_fc": (C.c_int, [_vp, C.c_char_p, _vp, C.c_int, _vp, C.c_int] + [_u32] * 6),
    # include/nemoasr_host.h
    "melfe_create": (_vp, []),
    "melfe_destroy": (None, [_vp]),
    "melfe_push": (None, [_vp, _f32p, C.c_size_t, C.c_int, C.POINTER(_f32p), C.POINTER(C.c_size_t)]),
    "melfe_samples": (C.c_size_t, [_vp]),
    "melfe_frames": (C.c_size_t, [_vp]),
    "rsmp_create": (_vp, [C.c_int, C.c_int]),
    "rsmp_destroy": (None, [_vp]),
    "rsmp_process": (C.c_size_t, [_vp, _f32p, C.c_size_t, _f32p, C.c_size_t]),
    "rsmp_flush": (C.c_size_t, [_vp, _f32p, C.c_size_t]),
    "nemo_enc_plan": (C.c_int, [_i32p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_int, _i32p]),
    "nemo_piece_text": (C.c_int, [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t]),
}


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() or make -C nemo-c_amd")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in API.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def fp(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


class GpuArg(C.Structure):
    """gpu_arg_t of include/nemo_gpu.h (src/gpu.h:10-15): a buffer + byte offset, or inline bytes."""
    _fields_ = [("buf", C.c_void_p), ("offset", C.c_size_t), ("bytes", C.c_void_p), ("size", C.c_size_t)]


def gpu_args(*items):
    """A gpu_arg_t array from (buffer handle, byte offset) pairs and ctypes parameter blocks (kept
    alive by the returned tuple's second element)."""
    arr = (GpuArg * len(items))()
    keep = []
    for i, it in enumerate(items):
        if isinstance(it, tuple):
            arr[i].buf, arr[i].offset = it[0], it[1]
        else:
            keep.append(it)
            arr[i].bytes, arr[i].size = C.cast(C.pointer(it), C.c_void_p), C.sizeof(it)
    return arr, keep


class Resid(C.Structure):
    """nk_resid_t: a pending residual update (partial rows in the context's scratch)."""
    _fields_ = [("parts", C.c_void_p), ("nparts", C.c_uint32), ("alpha", C.c_float)]


class Gpu:
    """Device context of the kernel-level C ABI (one stream)."""

    def __init__(self):
        err = C.create_string_buffer(512)
        self.h = lib().gpu_create(None, err, 512)
        if not self.h:
            raise RuntimeError("gpu_create: " + err.value.decode())
        self._bufs = []

    @property
    def name(self) -> str:
        return lib().gpu_device_name(self.h).decode()

    def alloc(self, nbytes: int) -> "Buf":
        b = lib().gpu_buf_alloc(self.h, max(int(nbytes), 1))
        if not b:
            raise MemoryError(nbytes)
        buf = Buf(self, b, int(nbytes))
        self._bufs.append(buf)
        return buf

    def put(self, a: np.ndarray) -> "Buf":
        a = np.ascontiguousarray(a)
        b = self.alloc(a.nbytes)
        b.write(a)
        return b

    def begin(self):
        if lib().gpu_begin(self.h):
            raise RuntimeError(lib().gpu_last_error(self.h).decode())

    def end(self) -> float:
        err = C.create_string_buffer(512)
        if lib().gpu_end(self.h, err, 512):
            raise RuntimeError(err.value.decode())
        return lib().gpu_last_ms(self.h)

    def check(self, rc: int):
        if rc:
            raise RuntimeError(lib().gpu_last_error(self.h).decode())

    def close(self):
        for b in self._bufs:
            b.free()
        self._bufs = []
        if self.h:
            lib().gpu_destroy(self.h)
            self.h = None


class Buf:
    def __init__(self, gpu: Gpu, h, nbytes: int):
        self.gpu, self.h, self.nbytes = gpu, h, nbytes

    @property
    def ptr(self) -> int:
        return lib().gpu_buf_dptr(self.h)

    def at(self, byte_offset: int) -> int:
        return self.ptr + int(byte_offset)

    def write(self, a: np.ndarray, byte_offset: int = 0):
        a = np.ascontiguousarray(a)
        assert byte_offset + a.nbytes <= self.nbytes
        self.gpu.check(lib().gpu_upload(self.gpu.h, self.at(byte_offset), a.ctypes.data, a.nbytes))

    def read(self, shape, dtype=np.float32, byte_offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert byte_offset + out.nbytes <= self.nbytes
        self.gpu.check(lib().gpu_download(self.gpu.h, out.ctypes.data, self.at(byte_offset), out.nbytes))
        return out

    def free(self):
        if self.h:
            lib().gpu_buf_free(self.h)
            self.h = None


class Session:
    """One streaming session through the public C API (include/nemoasr.h)."""

    def __init__(self, model_dir: str, language: str = "en-US", latency_ms: int = 560, input_rate: int = 16000):
        err = C.create_string_buffer(1024)
        self.h = lib().nemoasr_open(model_dir.encode(), language.encode(), latency_ms, input_rate, err, 1024)
        if not self.h:
            raise RuntimeError("nemoasr_open: " + err.value.decode())

    def feed(self, audio: np.ndarray, final: bool = False) -> str:
        a = np.ascontiguousarray(audio, dtype=np.float32)
        err = C.create_string_buffer(1024)
        p = lib().nemoasr_feed(self.h, fp(a), a.size, int(final), err, 1024)
        if err.value:
            raise RuntimeError("nemoasr_feed: " + err.value.decode())
        if not p:
            return ""
        s = C.cast(p, C.c_char_p).value.decode("utf-8", "replace")
        lib().nemoasr_free(p)
        return s

    def feed_mel(self, mel: np.ndarray, final: bool = False) -> int:
        m = np.ascontiguousarray(mel, dtype=np.float32).reshape(-1, 128)
        err = C.create_string_buffer(1024)
        n = lib().nemoasr_debug_feed_mel(self.h, fp(m), m.shape[0], int(final), err, 1024)
        if n < 0:
            raise RuntimeError("feed_mel: " + err.value.decode())
        return n

    def reset(self, language: str | None, latency_ms: int):
        err = C.create_string_buffer(1024)
        if lib().nemoasr_reset(self.h, language.encode() if language else None, latency_ms, err, 1024):
            raise RuntimeError("nemoasr_reset: " + err.value.decode())

    def tokens(self) -> list[int]:
        n = C.c_size_t()
        p = lib().nemoasr_debug_tokens(self.h, C.byref(n))
        return np.ctypeslib.as_array(p, shape=(n.value,)).tolist() if n.value else []

    def set_dump(self, on: bool):
        lib().nemoasr_debug_set_dump(self.h, int(on))

    def use_graphs(self, on: bool):
        lib().nemoasr_debug_use_graphs(self.h, int(on))

    def fuse(self, on: bool):
        lib().nemoasr_debug_fuse(self.h, int(on))

    def chain(self, on: bool):
        """One-row chunks: every conformer block in one persistent launch (default, where usable)
        or the per-kernel sequence."""
        lib().nemoasr_debug_chain(self.h, int(on))

    def chain_usable(self) -> bool:
        return bool(lib().nemoasr_debug_chain_usable(self.h))

    def chain_spin(self, spin_max: int):
        """Polls a chain hand-off may spend before the launch gives up (0: the default)."""
        lib().nemoasr_debug_chain_spin(self.h, int(spin_max))

    def dumps(self, n_layers: int, d_model: int, joint_hidden: int):
        F = lib().nemoasr_debug_frames(self.h)
        if F == 0:
            return (np.zeros((0, n_layers, d_model), np.float32), np.zeros((0, d_model), np.float32),
                    np.zeros((0, joint_hidden), np.float32))
        lay = np.ctypeslib.as_array(lib().nemoasr_debug_dump_layers(self.h), shape=(F * n_layers * d_model,))
        pr = np.ctypeslib.as_array(lib().nemoasr_debug_dump_prompted(self.h), shape=(F * d_model,))
        je = np.ctypeslib.as_array(lib().nemoasr_debug_dump_joint_enc(self.h), shape=(F * joint_hidden,))
        return (lay.reshape(F, n_layers, d_model).copy(), pr.reshape(F, d_model).copy(), je.reshape(F, joint_hidden).copy())

    def mel_dump(self) -> np.ndarray:
        """Log-mel frames (n, 128) the front end produced from fed audio while dumps were on."""
        n = C.c_size_t()
        p = lib().nemoasr_debug_dump_mel(self.h, C.byref(n))
        if not n.value:
            return np.zeros((0, 128), np.float32)
        return np.ctypeslib.as_array(p, shape=(n.value * 128,)).reshape(n.value, 128).copy()

    def stats(self) -> dict:
        class St(C.Structure):
            _fields_ = [("audio_seconds", C.c_double), ("chunks", C.c_size_t), ("tokens", C.c_size_t),
                        ("encoder_ms", C.c_double), ("decoder_ms", C.c_double)]
        st = St()
        lib().nemoasr_stats(self.h, C.byref(st))
        return {k: getattr(st, k) for k, _ in St._fields_}

    def chunk_ms(self) -> np.ndarray:
        n = C.c_size_t()
        p = lib().nemoasr_debug_chunk_ms(self.h, C.byref(n))
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy() if n.value else np.zeros(0)

    @property
    def joint_steps(self) -> int:
        return lib().nemoasr_debug_joint_steps(self.h)

    @property
    def gpu_name(self) -> str:
        return lib().nemoasr_gpu_name(self.h).decode()

    @property
    def load_ms(self) -> float:
        return lib().nemoasr_load_ms(self.h)

    def launches(self) -> int:
        """Kernel launches (direct and captured) issued on the session's device so far."""
        return int(lib().nemoasr_debug_launches(self.h))

    def time_kernel(self, name: str | None, max_launches: int = 4096):
        lib().nemoasr_debug_time_kernel(self.h, name.encode() if name else None, max_launches)

    def kernel_ms(self):
        """(mean ms per launch, launches, summed algorithmic bytes) of the timed kernel."""
        ms, n, by = C.c_double(), C.c_int(), C.c_double()
        lib().nemoasr_debug_kernel_ms(self.h, C.byref(ms), C.byref(n), C.byref(by))
        return ms.value, n.value, by.value

    def close(self):
        if self.h:
            lib().nemoasr_close(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Batch:
    """Many streams on one model (include/nemoasr_batch.h)."""

    def __init__(self, model_dir: str, language: str = "en-US", latency_ms: int = 560, streams: int = 64):
        err = C.create_string_buffer(1024)
        self.h = lib().nemoasr_batch_open(model_dir.encode(), language.encode(), latency_ms, streams, err, 1024)
        if not self.h:
            raise RuntimeError("nemoasr_batch_open: " + err.value.decode())
        self.n = streams

    def _check(self, rc: int, what: str, err) -> int:
        if rc < 0:
            raise RuntimeError(f"{what}: " + err.value.decode())
        return rc

    def push(self, stream: int, audio: np.ndarray, final: bool = False):
        a = np.ascontiguousarray(audio, dtype=np.float32)
        err = C.create_string_buffer(1024)
        self._check(lib().nemoasr_batch_push(self.h, stream, fp(a), a.size, int(final), err, 1024), "push", err)

    def push_mel(self, stream: int, mel: np.ndarray, final: bool = False):
        m = np.ascontiguousarray(mel, dtype=np.float32).reshape(-1, 128)
        err = C.create_string_buffer(1024)
        self._check(lib().nemoasr_batch_push_mel(self.h, stream, fp(m), m.shape[0], int(final), err, 1024),
                    "push_mel", err)

    def step(self) -> int:
        err = C.create_string_buffer(1024)
        return self._check(lib().nemoasr_batch_step(self.h, err, 1024), "step", err)

    def run(self) -> int:
        err = C.create_string_buffer(1024)
        return self._check(lib().nemoasr_batch_run(self.h, err, 1024), "run", err)

    def tokens(self, stream: int) -> list[int]:
        n = C.c_size_t()
        p = lib().nemoasr_batch_tokens(self.h, stream, C.byref(n))
        return np.ctypeslib.as_array(p, shape=(n.value,)).tolist() if n.value else []

    def text(self, stream: int) -> str:
        p = lib().nemoasr_batch_text(self.h, stream)
        if not p:
            return ""
        s = C.cast(p, C.c_char_p).value.decode("utf-8", "replace")
        lib().nemoasr_free(p)
        return s

    def reset_stream(self, stream: int):
        err = C.create_string_buffer(1024)
        self._check(lib().nemoasr_batch_reset_stream(self.h, stream, err, 1024), "reset_stream", err)

    def stats(self) -> dict:
        class St(C.Structure):
            _fields_ = [("steps", C.c_size_t), ("chunks", C.c_size_t), ("rows", C.c_size_t),
                        ("joint_steps", C.c_size_t), ("tokens", C.c_size_t), ("frontend_ms", C.c_double),
                        ("encoder_ms", C.c_double), ("decoder_ms", C.c_double), ("encoder_gpu_ms", C.c_double)]
        st = St()
        lib().nemoasr_batch_stats(self.h, C.byref(st))
        return {k: getattr(st, k) for k, _ in St._fields_}

    def step_ms(self) -> np.ndarray:
        n = C.c_size_t()
        p = lib().nemoasr_batch_step_ms(self.h, C.byref(n))
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy() if n.value else np.zeros(0)

    def use_graphs(self, on: bool):
        lib().nemoasr_batch_debug_use_graphs(self.h, int(on))

    def gpu_frontend(self, on: bool):
        if lib().nemoasr_batch_debug_gpu_frontend(self.h, int(on)):
            raise RuntimeError("front end can only be chosen before any input")

    def set_dump(self, on: bool):
        lib().nemoasr_batch_debug_set_dump(self.h, int(on))

    def device_decoder(self, on: bool):
        if lib().nemoasr_batch_debug_device_decoder(self.h, int(on)):
            raise RuntimeError("greedy loop can only be chosen before any input")

    def joint_enc(self, stream: int, joint_hidden: int) -> np.ndarray:
        n = C.c_size_t()
        p = lib().nemoasr_batch_debug_joint_enc(self.h, stream, C.byref(n))
        if not n.value:
            return np.zeros((0, joint_hidden), np.float32)
        return np.ctypeslib.as_array(p, shape=(n.value * joint_hidden,)).reshape(n.value, joint_hidden).copy()

    def time_kernel(self, name: str | None, max_launches: int = 32768):
        lib().nemoasr_batch_debug_time_kernel(self.h, name.encode() if name else None, max_launches)

    def kernel_ms(self):
        """(mean ms per launch, launches, summed algorithmic bytes, summed flops) of the timed kernel."""
        ms, n, by, fl = C.c_double(), C.c_int(), C.c_double(), C.c_double()
        lib().nemoasr_batch_debug_kernel_ms(self.h, C.byref(ms), C.byref(n), C.byref(by), C.byref(fl))
        return ms.value, n.value, by.value, fl.value

    def close(self):
        if self.h:
            lib().nemoasr_batch_close(self.h)
            self.h = None

    def __del__(self):
        self.close()
