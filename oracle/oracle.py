"""ORACLE — test infrastructure only.

ctypes binding of liboracle.so (the CPU restatement in oracle/*.c) plus a loader that reads the
checkpoint with its own small safetensors reader and config.json with the json module, so that
nothing of the product's loader is shared with the checker.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_u16p = C.POINTER(C.c_uint16)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int)


class Dims(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "n_layers", "d_model", "n_heads", "head_dim", "d_ff", "subsampling", "sub_channels", "conv_kernel", "feat_in",
        "num_prompts", "prompt_hidden", "pred_hidden", "vocab_size", "blank_id", "joint_hidden", "num_classes",
        "max_symbols", "att_left", "max_right")] + [("ln_eps", C.c_float)]


_G_FIELDS = ["conv0_w", "conv0_b", "conv2_w", "conv2_b", "conv3_w", "conv3_b", "conv5_w", "conv5_b", "conv6_w", "conv6_b",
             "pre_out_w", "pre_out_b", "prompt_w0", "prompt_b0", "prompt_w2", "prompt_b2"]


class GlobalW(C.Structure):
    _fields_ = ([(n, _u16p) for n in _G_FIELDS]
                + [("lstm_wx", _u16p * 2), ("lstm_wh", _u16p * 2), ("lstm_b", _u16p * 2), ("embed", _u16p)]
                + [(n, _u16p) for n in ("joint_enc_w", "joint_enc_b", "joint_pred_w", "joint_pred_b", "joint_out_w",
                                        "joint_out_b")])


_L_FIELDS = ["ff1_w1", "ff1_w2", "ff2_w1", "ff2_w2", "wq", "wk", "wv", "wo", "wpos", "pw1", "pw2",
             "ln_ff1_g", "ln_ff1_b", "ln_att_g", "ln_att_b", "ln_conv_g", "ln_conv_b", "ln_ff2_g", "ln_ff2_b",
             "ln_out_g", "ln_out_b", "bn_g", "bn_b", "dw_w", "bias_u", "bias_v"]


class LayerW(C.Structure):
    _fields_ = [(n, _u16p) for n in _L_FIELDS]


class EncBook(C.Structure):
    _fields_ = [("pending_n", C.c_size_t), ("consumed", C.c_size_t), ("emitted", C.c_size_t),
                ("mel_cache_n", C.c_int), ("closed", C.c_int)]


class EncPlan(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("ran", "take", "nwin", "lo", "hi", "c", "include_boundary", "T3")]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run make -C oracle)")
        L = C.CDLL(LIB_PATH)
        L.or_gemm.argtypes = [_f32p, C.c_long, _u16p, C.c_long, _f32p, _f32p, C.c_long, C.c_int, C.c_int, C.c_int,
                              C.c_int, C.c_int, C.c_float]
        L.or_layernorm.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_float]
        L.or_layernorm2.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_float]
        L.or_attention_rel.argtypes = [_f32p, C.c_long, _f32p, _f32p, C.c_long, _f32p, _f32p, _f32p, _f32p, C.c_int,
                                       C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        L.or_dwconv_ln_silu.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_float]
        for fn in ("or_conv2d_c1_s2_relu", "or_dwconv2d_s2"):
            getattr(L, fn).argtypes = [_f32p, _f32p, _f32p, _f32p] + [C.c_int] * 5
        L.or_flatten_cf.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.or_lstm_cell.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int]
        L.or_joint_argmax.argtypes = [_f32p, _f32p, _u16p, _f32p, C.c_int, C.c_int, _f32p, _f32p]
        L.or_joint_argmax.restype = C.c_int
        L.or_ptab.argtypes = [_u16p, C.c_int, C.c_int, _f32p]
        L.or_sigmoid.argtypes = [C.c_float]
        L.or_sigmoid.restype = C.c_float
        L.or_silu.argtypes = [C.c_float]
        L.or_silu.restype = C.c_float
        L.or_model_create.argtypes = [C.POINTER(Dims), C.POINTER(GlobalW), C.POINTER(LayerW)]
        L.or_model_create.restype = C.c_void_p
        L.or_model_free.argtypes = [C.c_void_p]
        L.or_model_set_language.argtypes = [C.c_void_p, C.c_int]
        L.or_model_ptab.argtypes = [C.c_void_p, C.c_int]
        L.or_model_ptab.restype = _f32p
        L.or_model_lmax.argtypes = [C.c_void_p]
        L.or_session_create.argtypes = [C.c_void_p, C.c_int]
        L.or_session_create.restype = C.c_void_p
        for fn in ("or_session_free", "or_session_reset"):
            getattr(L, fn).argtypes = [C.c_void_p]
        L.or_session_set_dump.argtypes = [C.c_void_p, C.c_int]
        L.or_session_feed_mel.argtypes = [C.c_void_p, _f32p, C.c_size_t, C.c_int, _i32p, C.c_int]
        for fn in ("or_session_chunks", "or_session_frames", "or_session_joint_steps"):
            getattr(L, fn).argtypes = [C.c_void_p]
            getattr(L, fn).restype = C.c_size_t
        for fn in ("or_session_dump_layers", "or_session_dump_prompted", "or_session_dump_joint_enc"):
            getattr(L, fn).argtypes = [C.c_void_p]
            getattr(L, fn).restype = _f32p
        L.or_session_dump_chunk_rows.argtypes = [C.c_void_p]
        L.or_session_dump_chunk_rows.restype = _i32p
        L.or_session_joint_log.argtypes = [C.c_void_p, C.POINTER(_i32p), C.POINTER(_f32p)]
        L.or_session_joint_log.restype = C.c_size_t
        L.or_session_token_margins.argtypes = [C.c_void_p, C.POINTER(_f32p), C.POINTER(C.c_float)]
        L.or_session_token_margins.restype = C.c_size_t
        L.or_set_gemm_a_mode.argtypes = [C.c_int]
        L.or_set_gemm_a_mode.restype = None
        L.or_session_decisions.argtypes = [C.c_void_p, C.POINTER(_i32p), C.POINTER(_i32p), C.POINTER(_f32p)]
        L.or_session_decisions.restype = C.c_size_t
        L.or_session_force.argtypes = [C.c_void_p, C.POINTER(C.c_size_t), _i32p, C.c_size_t]
        L.or_session_force.restype = None
        L.or_session_error.argtypes = [C.c_void_p]
        L.or_session_error.restype = C.c_char_p
        L.or_enc_plan.argtypes = [C.POINTER(EncBook), C.c_int, C.c_int, C.c_int, C.c_int]
        L.or_enc_plan.restype = EncPlan
        L.or_set_threads.argtypes = [C.c_int]
        _lib = L
    return _lib


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def fp(a: np.ndarray):
    return a.ctypes.data_as(_f32p) if a is not None else None


def up(a: np.ndarray):
    return a.ctypes.data_as(_u16p)


def bf16_to_f32(u: np.ndarray) -> np.ndarray:
    return (np.asarray(u).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


# ---- kernel-level wrappers --------------------------------------------------------------------
def gemm(A, W_bf16, bias=None, act=0, accumulate=False, alpha=1.0, C0=None, ldw=None, K=None):
    A = f32(A)
    M = A.shape[0]
    N = W_bf16.shape[0]
    K = A.shape[1] if K is None else K
    ldw = W_bf16.shape[1] if ldw is None else ldw
    nout = N // 2 if act == 3 else N
    out = f32(C0).copy() if C0 is not None else np.zeros((M, nout), np.float32)
    b = f32(bias) if bias is not None else None
    W = np.ascontiguousarray(W_bf16, dtype=np.uint16)
    lib().or_gemm(fp(A), A.shape[1], up(W), ldw, fp(b), fp(out), nout, M, N, K, act, int(accumulate), alpha)
    return out


def layernorm(X, g, b, eps=1e-5):
    X = f32(X)
    Y = np.empty_like(X)
    lib().or_layernorm(fp(X), fp(f32(g)), fp(f32(b)), fp(Y), X.shape[0], X.shape[1], eps)
    return Y


def layernorm2(X, g1, b1, g2, b2, eps=1e-5):
    X = f32(X)
    Y1, Y2 = np.empty_like(X), np.empty_like(X)
    lib().or_layernorm2(fp(X), fp(f32(g1)), fp(f32(b1)), fp(f32(g2)), fp(f32(b2)), fp(Y1), fp(Y2), X.shape[0],
                        X.shape[1], eps)
    return Y1, Y2


def attention_rel(Q, K, V, P, bu, bv, c, L, Lmax, H, dh):
    """Q [c][ldq], K/V [L][ldk] (head h at columns h*dh..), P [2Lmax-1][D]."""
    Q, K, V, P = f32(Q), f32(K), f32(V), f32(P)
    D = H * dh
    O = np.zeros((c, D), np.float32)
    lib().or_attention_rel(fp(Q), Q.shape[1], fp(K), fp(V), K.shape[1], fp(P), fp(f32(bu)), fp(f32(bv)), fp(O), c, L,
                           Lmax, H, dh, D, float(np.float32(1.0) / np.sqrt(np.float32(dh))))
    return O


def dwconv_ln_silu(din, W, g, b, c, eps=1e-5):
    din, W = f32(din), f32(W)
    D, taps = W.shape
    Y = np.zeros((c, D), np.float32)
    lib().or_dwconv_ln_silu(fp(din), fp(W), fp(f32(g)), fp(f32(b)), fp(Y), c, D, taps, eps)
    return Y


def sub_len(n):
    return n // 2 + 1


def conv2d_c1_s2_relu(X, W, bias):
    X = f32(X)
    T, F = X.shape
    Cc = W.shape[0]
    T1, F1 = sub_len(T), F // 2 + 1
    Y = np.zeros((T1, F1, Cc), np.float32)
    lib().or_conv2d_c1_s2_relu(fp(X), fp(f32(W)), fp(f32(bias)), fp(Y), T, F, T1, F1, Cc)
    return Y


def dwconv2d_s2(X, W, bias):
    X = f32(X)
    T, F, Cc = X.shape
    T1, F1 = T // 2 + 1, F // 2 + 1
    Y = np.zeros((T1, F1, Cc), np.float32)
    lib().or_dwconv2d_s2(fp(X), fp(f32(W)), fp(f32(bias)), fp(Y), T, F, T1, F1, Cc)
    return Y


def flatten_cf(X):
    X = f32(X)
    T, F, Cc = X.shape
    Y = np.zeros((T, Cc * F), np.float32)
    lib().or_flatten_cf(fp(X), fp(Y), T, F, Cc)
    return Y


def lstm_cell(gates, c_in):
    gates, c_in = f32(gates), f32(c_in)
    H = c_in.size
    c_out, h_out = np.zeros(H, np.float32), np.zeros(H, np.float32)
    lib().or_lstm_cell(fp(gates), fp(c_in), fp(c_out), fp(h_out), H)
    return c_out, h_out


def joint_argmax(enc, pred, W_bf16, bias):
    enc, pred, bias = f32(enc), f32(pred), f32(bias)
    V, H = W_bf16.shape
    W = np.ascontiguousarray(W_bf16, dtype=np.uint16)
    bv = C.c_float()
    logits = np.zeros(V, np.float32)
    i = lib().or_joint_argmax(fp(enc), fp(pred), up(W), fp(bias), V, H, C.byref(bv), fp(logits))
    return i, bv.value, logits


def ptab(wpos_bf16, D, Lmax):
    W = np.ascontiguousarray(wpos_bf16, dtype=np.uint16)
    out = np.zeros((2 * Lmax - 1, D), np.float32)
    lib().or_ptab(up(W), D, Lmax, fp(out))
    return out


def enc_plan(book: EncBook, final: bool, chunk_mel: int, subsampling: int = 8, mel_cache: int = 16) -> EncPlan:
    return lib().or_enc_plan(C.byref(book), int(final), chunk_mel, subsampling, mel_cache)


# ---- checkpoint -------------------------------------------------------------------------------
def read_safetensors(path: str) -> dict:
    with open(path, "rb") as f:
        hlen = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(hlen))
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        a, b = meta["data_offsets"]
        if meta["dtype"] != "BF16":
            raise ValueError(f"{name} is not BF16")
        out[name] = np.asarray(mm[8 + hlen + a: 8 + hlen + b].view(np.uint16)).reshape(meta["shape"])
    return out


def read_config(model_dir: str) -> dict:
    with open(os.path.join(model_dir, "config.json")) as f:
        return json.load(f)


def dims_from_config(cfg: dict) -> Dims:
    e, p, d, j = cfg["encoder"], cfg["prompt"], cfg["decoder"], cfg["joint"]
    rights = [r for _, r in e["att_context_size"]]
    return Dims(n_layers=e["n_layers"], d_model=e["d_model"], n_heads=e["n_heads"],
                head_dim=e["d_model"] // e["n_heads"], d_ff=e["d_model"] * e["ff_expansion_factor"],
                subsampling=e["subsampling_factor"], sub_channels=e["subsampling_conv_channels"],
                conv_kernel=e["conv_kernel_size"], feat_in=e["feat_in"], num_prompts=p["num_prompts"],
                prompt_hidden=p["prompt_hidden"], pred_hidden=d["pred_hidden"], vocab_size=d["vocab_size"],
                blank_id=d["vocab_size"], joint_hidden=j["joint_hidden"], num_classes=j["num_classes"] + 1,
                max_symbols=cfg.get("max_symbols", 10), att_left=e["att_context_size"][-1][0],
                max_right=max(rights), ln_eps=1e-5)


class Model:
    """The oracle model: weights memory-mapped from the checkpoint, small params widened in C."""

    def __init__(self, model_dir: str, language: str = "en-US"):
        self.dir = model_dir
        self.cfg = read_config(model_dir)
        self.t = read_safetensors(os.path.join(model_dir, "model.safetensors"))
        self.dims = dims_from_config(self.cfg)
        t = self.t
        pe = "encoder.pre_encode."
        gw = GlobalW()
        names = {"conv0_w": pe + "conv.0.weight", "conv0_b": pe + "conv.0.bias", "conv2_w": pe + "conv.2.weight",
                 "conv2_b": pe + "conv.2.bias", "conv3_w": pe + "conv.3.weight", "conv3_b": pe + "conv.3.bias",
                 "conv5_w": pe + "conv.5.weight", "conv5_b": pe + "conv.5.bias", "conv6_w": pe + "conv.6.weight",
                 "conv6_b": pe + "conv.6.bias", "pre_out_w": pe + "out.weight", "pre_out_b": pe + "out.bias",
                 "prompt_w0": "prompt_kernel.0.weight", "prompt_b0": "prompt_kernel.0.bias",
                 "prompt_w2": "prompt_kernel.2.weight", "prompt_b2": "prompt_kernel.2.bias",
                 "embed": "decoder.prediction.embed.weight", "joint_enc_w": "joint.enc.weight",
                 "joint_enc_b": "joint.enc.bias", "joint_pred_w": "joint.pred.weight",
                 "joint_pred_b": "joint.pred.bias", "joint_out_w": "joint.joint_net.2.weight",
                 "joint_out_b": "joint.joint_net.2.bias"}
        self._keep = []
        for f, n in names.items():
            setattr(gw, f, self._p(n))
        for l in range(2):
            q = f"decoder.prediction.dec_rnn.lstm.{l}."
            gw.lstm_wx[l] = self._p(q + "Wx")
            gw.lstm_wh[l] = self._p(q + "Wh")
            gw.lstm_b[l] = self._p(q + "bias")
        nl = self.dims.n_layers
        layers = (LayerW * nl)()
        lmap = {"ff1_w1": "feed_forward1.linear1.weight", "ff1_w2": "feed_forward1.linear2.weight",
                "ff2_w1": "feed_forward2.linear1.weight", "ff2_w2": "feed_forward2.linear2.weight",
                "wq": "self_attn.linear_q.weight", "wk": "self_attn.linear_k.weight",
                "wv": "self_attn.linear_v.weight", "wo": "self_attn.linear_out.weight",
                "wpos": "self_attn.linear_pos.weight", "pw1": "conv.pointwise_conv1.weight",
                "pw2": "conv.pointwise_conv2.weight", "ln_ff1_g": "norm_feed_forward1.weight",
                "ln_ff1_b": "norm_feed_forward1.bias", "ln_att_g": "norm_self_att.weight",
                "ln_att_b": "norm_self_att.bias", "ln_conv_g": "norm_conv.weight", "ln_conv_b": "norm_conv.bias",
                "ln_ff2_g": "norm_feed_forward2.weight", "ln_ff2_b": "norm_feed_forward2.bias",
                "ln_out_g": "norm_out.weight", "ln_out_b": "norm_out.bias", "bn_g": "conv.batch_norm.weight",
                "bn_b": "conv.batch_norm.bias", "dw_w": "conv.depthwise_conv.weight",
                "bias_u": "self_attn.pos_bias_u", "bias_v": "self_attn.pos_bias_v"}
        for l in range(nl):
            for f, n in lmap.items():
                setattr(layers[l], f, self._p(f"encoder.layers.{l}.{n}"))
        self.handle = lib().or_model_create(C.byref(self.dims), C.byref(gw), layers)
        self.set_language(language)

    def _p(self, name):
        a = np.ascontiguousarray(self.t[name])
        self._keep.append(a)
        return up(a)

    def set_language(self, language: str):
        idx = self.cfg["prompt"]["prompt_dictionary"][language]
        if lib().or_model_set_language(self.handle, idx) != 0:
            raise ValueError(language)

    @property
    def lmax(self) -> int:
        return lib().or_model_lmax(self.handle)

    def ptab(self, layer: int) -> np.ndarray:
        P = 2 * self.lmax - 1
        p = lib().or_model_ptab(self.handle, layer)
        return np.ctypeslib.as_array(p, shape=(P * self.dims.d_model,)).reshape(P, self.dims.d_model).copy()

    def __del__(self):
        if getattr(self, "handle", None):
            lib().or_model_free(self.handle)
            self.handle = None


class Session:
    """Streaming encoder + greedy RNNT decoder over mel frames (oracle)."""

    def __init__(self, model: Model, right: int, dump: bool = False):
        self.model = model
        self.right = right
        self.h = lib().or_session_create(model.handle, right)
        lib().or_session_set_dump(self.h, int(dump))
        self.tokens: list[int] = []
        self._mel: list[np.ndarray] = []

    def feed_mel(self, mel: np.ndarray, final: bool = False) -> list[int]:
        mel = f32(mel).reshape(-1, self.model.dims.feat_in)
        self._mel.append(mel.copy())
        buf = np.zeros(1 << 20, np.int32)
        n = lib().or_session_feed_mel(self.h, fp(mel), mel.shape[0], int(final), buf.ctypes.data_as(_i32p), buf.size)
        if n < 0:
            raise RuntimeError(lib().or_session_error(self.h).decode())
        out = buf[:n].tolist()
        self.tokens += out
        return out

    def reset(self):
        lib().or_session_reset(self.h)
        self.tokens = []
        self._mel = []

    def replayer(self):
        """rerun(forced) for the tests' token check: a fresh session of the same model and latency
        decodes the mel rows fed since reset in one piece (feed granularity does not change the
        decode) with committed decisions forced; returns (tokens, outcomes, runner-ups, margins,
        blank id)."""
        nm = self.model.dims.feat_in
        mel = np.concatenate(self._mel) if self._mel else np.zeros((0, nm), np.float32)
        model, right = self.model, self.right

        def run(forced):
            o = Session(model, right)
            o.force(forced)
            o.feed_mel(mel, final=True)
            best, second, margin = o.decisions()
            return list(o.tokens), best, second, margin, model.dims.blank_id

        return run

    @property
    def frames(self) -> int:
        return lib().or_session_frames(self.h)

    @property
    def chunks(self) -> int:
        return lib().or_session_chunks(self.h)

    @property
    def joint_steps(self) -> int:
        return lib().or_session_joint_steps(self.h)

    def dumps(self):
        d = self.model.dims
        F = self.frames
        nl, D, J = d.n_layers, d.d_model, d.joint_hidden
        if F == 0:
            return np.zeros((0, nl, D), np.float32), np.zeros((0, D), np.float32), np.zeros((0, J), np.float32), []
        lay = np.ctypeslib.as_array(lib().or_session_dump_layers(self.h), shape=(F * nl * D,)).reshape(F, nl, D).copy()
        pr = np.ctypeslib.as_array(lib().or_session_dump_prompted(self.h), shape=(F * D,)).reshape(F, D).copy()
        je = np.ctypeslib.as_array(lib().or_session_dump_joint_enc(self.h), shape=(F * J,)).reshape(F, J).copy()
        rows = np.ctypeslib.as_array(lib().or_session_dump_chunk_rows(self.h), shape=(self.chunks,)).tolist()
        return lay, pr, je, rows

    def joint_log(self):
        b, m = _i32p(), _f32p()
        n = lib().or_session_joint_log(self.h, C.byref(b), C.byref(m))
        if n == 0:
            return np.zeros(0, np.int32), np.zeros(0, np.float32)
        return (np.ctypeslib.as_array(b, shape=(n,)).copy(), np.ctypeslib.as_array(m, shape=(n,)).copy())

    def token_margins(self) -> np.ndarray:
        """Per emitted token k, the smallest top-2 joint margin over the greedy decisions that
        produced it (blank frames since token k-1, then the emitting frame); one extra last entry
        for the decisions after the last token (inf when there are none)."""
        m, tail = _f32p(), C.c_float()
        n = lib().or_session_token_margins(self.h, C.byref(m), C.byref(tail))
        head = np.ctypeslib.as_array(m, shape=(n,)).copy() if n else np.zeros(0, np.float32)
        return np.append(head, np.float32(tail.value))

    def decisions(self):
        """Committed greedy decisions since reset: (outcome, runner-up index, top-2 margin) arrays.
        A decision is one frame's blank or one emitted token (src/decoder.c:107-123)."""
        b, s2, m = _i32p(), _i32p(), _f32p()
        n = lib().or_session_decisions(self.h, C.byref(b), C.byref(s2), C.byref(m))
        if n == 0:
            return np.zeros(0, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32)
        return (np.ctypeslib.as_array(b, shape=(n,)).copy(), np.ctypeslib.as_array(s2, shape=(n,)).copy(),
                np.ctypeslib.as_array(m, shape=(n,)).copy())

    def force(self, forced: dict):
        """Force committed decision j to token forced[j] in the following decodes (the other side of
        a float tie)."""
        at = sorted(forced)
        arr_at = (C.c_size_t * max(1, len(at)))(*at)
        arr_tok = np.array([forced[j] for j in at] or [0], np.int32)
        lib().or_session_force(self.h, arr_at, arr_tok.ctypes.data_as(_i32p), len(at))

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_session_free(self.h)
            self.h = None
