"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, and only there as the checker / the CPU
baseline. The product package textsift_amd never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
i32p = C.POINTER(C.c_int32)
f32p = C.POINTER(C.c_float)


class Config(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden", "heads", "kv_heads", "head_dim", "window", "dff", "experts",
                                           "topk", "classes", "vocab", "layers")] + [
        ("eps", C.c_float),
        ("rope_theta", C.c_double), ("rope_factor", C.c_double),
        ("rope_beta_fast", C.c_double), ("rope_beta_slow", C.c_double),
        ("rope_orig_max", C.c_uint32), ("rope_truncate", C.c_uint32)]


class QWeight(C.Structure):
    _fields_ = [("int4", u8p), ("scales", u16p), ("zp", u8p), ("bias", u16p)]


class Layer(C.Structure):
    _fields_ = [("input_ln", u16p), ("post_ln", u16p), ("q", QWeight), ("k", QWeight), ("v", QWeight),
                ("o", QWeight), ("sinks", f32p), ("router", QWeight), ("gate_up", QWeight), ("down", QWeight)]


class Model(C.Structure):
    _fields_ = [("embed_int4", u8p), ("embed_scales", u16p), ("embed_zp", u8p), ("layers", C.POINTER(Layer)),
                ("final_ln", u16p), ("score", QWeight)]


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _lib.pfo_fp16_to_f32.restype = C.c_float
        _lib.pfo_fp16_to_f32.argtypes = [C.c_uint16]
        _lib.pfo_f32_to_fp16.restype = C.c_uint16
        _lib.pfo_f32_to_fp16.argtypes = [C.c_float]
        _lib.pfo_exp_approx.restype = C.c_float
        _lib.pfo_exp_approx.argtypes = [C.c_float]
        _lib.pfo_rms_norm.argtypes = [C.c_void_p] * 3 + [C.c_uint32] * 2 + [C.c_float]
        _lib.pfo_rms_norm_fp16_to_f32.argtypes = [C.c_void_p] * 3 + [C.c_uint32] * 2 + [C.c_float]
        _lib.pfo_add_rmsnorm_fp16_to_f32.argtypes = [C.c_void_p] * 5 + [C.c_uint32] * 2 + [C.c_float]
        _lib.pfo_topk_partial_f32.argtypes = [C.c_void_p] * 3 + [C.c_uint32] * 3
        _lib.pfo_matmul_int4block.argtypes = [C.c_int, C.c_int] + [C.c_void_p] * 6 + [C.c_uint32] * 3
        _lib.pfo_swiglu_clamp_f32.argtypes = [C.c_void_p] * 2 + [C.c_uint32] * 2
        _lib.pfo_softmax_f32.argtypes = [C.c_void_p] * 2 + [C.c_uint32] * 2
        _lib.pfo_add_fp16.argtypes = [C.c_void_p] * 3 + [C.c_uint32]
        _lib.pfo_scatter_add_weighted_f32.argtypes = [C.c_void_p] * 4 + [C.c_uint32] * 2
        _lib.pfo_cast_f32_to_fp16_scaled.argtypes = [C.c_void_p] * 2 + [C.c_uint32, C.c_float]
        _lib.pfo_banded_attention.argtypes = [C.c_void_p] * 6 + [C.c_uint32] * 7
        _lib.pfo_banded_attention_wgsl.argtypes = [C.c_void_p] * 6 + [C.c_uint32] * 5
        _lib.pfo_f2h_ieee.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        _lib.pfo_rope_apply.argtypes = [C.c_void_p] * 3 + [C.c_uint32] * 3
        _lib.pfo_embed_lookup_int4.argtypes = [C.c_void_p] * 5 + [C.c_uint32] * 3
        _lib.pfo_rope_tables.argtypes = [C.POINTER(Config), C.c_uint32, C.c_void_p, C.c_void_p]
        _lib.pfo_router_select.argtypes = [C.c_void_p] * 3 + [C.c_uint32] * 3
        _lib.pfo_expert_dispatch.argtypes = [C.POINTER(Config), C.POINTER(Layer)] + [C.c_void_p] * 4 + [
            C.c_uint32, C.c_int]
        _lib.pfo_model_forward.argtypes = [C.POINTER(Config), C.POINTER(Model), C.c_void_p, C.c_void_p,
                                           C.c_uint32, C.c_int, C.c_void_p]
        _lib.pfo_model_forward_route.argtypes = [C.POINTER(Config), C.POINTER(Model), C.c_void_p, C.c_void_p,
                                                 C.c_uint32, C.c_int, C.c_void_p, C.c_void_p]
        _lib.pfo_block_forward.argtypes = [C.POINTER(Config), C.POINTER(Layer)] + [C.c_void_p] * 5 + [
            C.c_uint32, C.c_int]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def make_config(cfg, layers=None, experts=None, vocab=None) -> Config:
    r = cfg.rope
    return Config(cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.sliding_window,
                  cfg.intermediate_size, cfg.num_experts if experts is None else experts, cfg.num_experts_per_tok,
                  cfg.num_classes, cfg.vocab_size if vocab is None else vocab,
                  cfg.num_layers if layers is None else layers, cfg.rms_norm_eps, r.theta, r.factor, r.beta_fast,
                  r.beta_slow, r.original_max_position_embeddings, int(r.truncate))


# ---------------- element-wise / kernel wrappers ----------------

def fp16_to_f32(bits):
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().pfo_fp16_to_f32_n(_p(bits), _p(out), C.c_size_t(bits.size))
    return out


def f32_to_fp16(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().pfo_f32_to_fp16_n(_p(x), _p(out), C.c_size_t(x.size))
    return out


def matmul(x, w_int4, scales, zp, bias, N, D, x_f32, out_f32):
    x = _c(x, np.float32 if x_f32 else np.uint16)
    T = x.size // D
    out = np.empty((T, N), np.float32 if out_f32 else np.uint16)
    w_int4, scales, bias = _c(w_int4, np.uint8), _c(scales, np.uint16), _c(bias, np.uint16)
    zp = None if zp is None else _c(zp, np.uint8)
    lib().pfo_matmul_int4block(int(x_f32), int(out_f32), _p(x), _p(w_int4), _p(scales), _p(zp), _p(bias),
                               _p(out), T, N, D)
    return out


def embed_lookup(int4, scales, zp, ids, V, D):
    ids = _c(ids, np.int32)
    out = np.empty((ids.size, D), np.uint16)
    int4, scales, zp = _c(int4, np.uint8), _c(scales, np.uint16), _c(zp, np.uint8)
    lib().pfo_embed_lookup_int4(_p(int4), _p(scales), _p(zp), _p(ids), _p(out), ids.size, V, D)
    return out


def rms_norm(x, gamma, T, D, eps):
    x, gamma = _c(x, np.uint16), _c(gamma, np.uint16)
    out = np.empty((T, D), np.uint16)
    lib().pfo_rms_norm(_p(x), _p(gamma), _p(out), T, D, eps)
    return out


def rms_norm_f32(x, gamma, T, D, eps):
    x, gamma = _c(x, np.uint16), _c(gamma, np.uint16)
    out = np.empty((T, D), np.float32)
    lib().pfo_rms_norm_fp16_to_f32(_p(x), _p(gamma), _p(out), T, D, eps)
    return out


def add_rmsnorm_f32(a, b, gamma, T, D, eps):
    a, b, gamma = _c(a, np.uint16), _c(b, np.uint16), _c(gamma, np.uint16)
    s = np.empty((T, D), np.uint16)
    n = np.empty((T, D), np.float32)
    lib().pfo_add_rmsnorm_fp16_to_f32(_p(a), _p(b), _p(gamma), _p(s), _p(n), T, D, eps)
    return s, n


def topk(x, rows, cols, k):
    x = _c(x, np.float32)
    idx = np.empty((rows, k), np.int32)
    val = np.empty((rows, k), np.float32)
    lib().pfo_topk_partial_f32(_p(x), _p(idx), _p(val), rows, cols, k)
    return idx, val


def softmax(x, rows, cols):
    x = _c(x, np.float32)
    out = np.empty((rows, cols), np.float32)
    lib().pfo_softmax_f32(_p(x), _p(out), rows, cols)
    return out


def swiglu(gu, T, D):
    gu = _c(gu, np.float32)
    out = np.empty((T, D), np.float32)
    lib().pfo_swiglu_clamp_f32(_p(gu), _p(out), T, D)
    return out


def add_fp16(a, b):
    a, b = _c(a, np.uint16), _c(b, np.uint16)
    out = np.empty(a.shape, np.uint16)
    lib().pfo_add_fp16(_p(a), _p(b), _p(out), a.size)
    return out


def cast_scaled(src, scale):
    src = _c(src, np.float32)
    out = np.empty(src.shape, np.uint16)
    lib().pfo_cast_f32_to_fp16_scaled(_p(src), _p(out), src.size, scale)
    return out


def banded_attention(q, k, v, sinks, mask, T, Hq, Hkv, hd, window, h0=0, h1=None):
    q, k, v = _c(q, np.uint16), _c(k, np.uint16), _c(v, np.uint16)
    sinks = _c(sinks, np.float32)
    mask = None if mask is None else _c(mask, np.uint8)
    out = np.zeros((T, Hq * hd), np.uint16)
    lib().pfo_banded_attention(_p(q), _p(k), _p(v), _p(sinks), _p(mask), _p(out), T, Hq, Hkv, hd, window, h0,
                               Hq if h1 is None else h1)
    return out


def f2h_ieee(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().pfo_f2h_ieee(_p(x), _p(out), x.size)
    return out


def banded_attention_wgsl(q, k, v, sinks, mask, T, Hq, Hkv, hd, window):
    """The reference's GPU-path attention (native/shaders/banded_attention.wgsl)."""
    q, k, v = _c(q, np.uint16), _c(k, np.uint16), _c(v, np.uint16)
    sinks = _c(sinks, np.float32)
    mask = None if mask is None else _c(mask, np.uint8)
    out = np.zeros((T, Hq * hd), np.uint16)
    lib().pfo_banded_attention_wgsl(_p(q), _p(k), _p(v), _p(sinks), _p(mask), _p(out), T, Hq, Hkv, hd, window)
    return out


def rope_apply(qk, cos_t, sin_t, T, H, hd):
    qk = _c(qk, np.uint16).copy()
    cos_t, sin_t = _c(cos_t, np.uint16), _c(sin_t, np.uint16)
    lib().pfo_rope_apply(_p(qk), _p(cos_t), _p(sin_t), T, H, hd)
    return qk


def rope_tables(cfg, T):
    c = make_config(cfg)
    half = cfg.head_dim // 2
    cs = np.empty((T, half), np.uint16)
    sn = np.empty((T, half), np.uint16)
    lib().pfo_rope_tables(C.byref(c), T, _p(cs), _p(sn))
    return cs, sn


def router_select(logits, T, E, K):
    logits = _c(logits, np.float32)
    idx = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    lib().pfo_router_select(_p(logits), _p(idx), _p(w), T, E, K)
    return idx, w


# ---------------- model-level wrappers ----------------

class _Keep:
    """Keeps the numpy buffers a ctypes struct points into alive."""

    def __init__(self):
        self.refs = []

    def p(self, a, dtype):
        if a is None:
            return None
        a = _c(a, dtype)
        self.refs.append(a)
        return a.ctypes.data_as(C.c_void_p)


def _qw(keep, w, prefix, zp_present=True):
    return QWeight(C.cast(keep.p(w[prefix + ".int4"], np.uint8), u8p),
                   C.cast(keep.p(w[prefix + ".scales"], np.uint16), u16p),
                   C.cast(keep.p(w.get(prefix + ".zp") if zp_present else None, np.uint8), u8p),
                   C.cast(keep.p(w[prefix + ".bias"], np.uint16), u16p))


def make_layer(keep, w, l):
    p = f"layers.{l}"
    return Layer(C.cast(keep.p(w[p + ".input_layernorm"], np.uint16), u16p),
                 C.cast(keep.p(w[p + ".post_attention_layernorm"], np.uint16), u16p),
                 _qw(keep, w, p + ".attn.q_proj"), _qw(keep, w, p + ".attn.k_proj"),
                 _qw(keep, w, p + ".attn.v_proj"), _qw(keep, w, p + ".attn.o_proj"),
                 C.cast(keep.p(w[p + ".attn.sinks"], np.float32), f32p),
                 _qw(keep, w, p + ".router"), _qw(keep, w, p + ".experts.gate_up"),
                 _qw(keep, w, p + ".experts.down"))


def model_forward(cfg, w, ids, mask=None, n_threads=1, num_layers=None, return_routing=False):
    """Oracle forward -> fp16 logit bits [T, classes] (WASM path, model.ts:50-105).
    return_routing: also every layer's routed expert ids, int32 [layers, T, topk]."""
    L = cfg.num_layers if num_layers is None else num_layers
    E = w["layers.0.router.int4"].shape[0]
    V = w["embed.int4"].shape[0]
    c = make_config(cfg, layers=L, experts=E, vocab=V)
    keep = _Keep()
    layers = (Layer * L)(*[make_layer(keep, w, l) for l in range(L)])
    m = Model(C.cast(keep.p(w["embed.int4"], np.uint8), u8p), C.cast(keep.p(w["embed.scales"], np.uint16), u16p),
              C.cast(keep.p(w["embed.zp"], np.uint8), u8p), layers,
              C.cast(keep.p(w["final_norm"], np.uint16), u16p), _qw(keep, w, "score"))
    ids = _c(ids, np.int32)
    T = ids.size
    mask = None if mask is None else _c(mask, np.uint8)
    out = np.empty((T, cfg.num_classes), np.uint16)
    route = np.empty((L, T, cfg.num_experts_per_tok), np.int32) if return_routing else None
    rc = lib().pfo_model_forward_route(C.byref(c), C.byref(m), _p(ids), _p(mask), T, n_threads, _p(out),
                                       _p(route))
    if rc != 0:
        raise RuntimeError("oracle model_forward failed")
    return (out, route) if return_routing else out


def expert_dispatch(cfg, w, l, hidden_f32, ridx, rw, n_slices=1):
    E = w[f"layers.{l}.experts.gate_up.int4"].shape[0]
    c = make_config(cfg, experts=E)
    keep = _Keep()
    layer = make_layer(keep, w, l)
    hidden_f32 = _c(hidden_f32, np.float32)
    T = hidden_f32.shape[0]
    ridx, rw = _c(ridx, np.int32), _c(rw, np.float32)
    out = np.empty((T, cfg.hidden_size), np.uint16)
    rc = lib().pfo_expert_dispatch(C.byref(c), C.byref(layer), _p(hidden_f32), _p(ridx), _p(rw), _p(out), T,
                                   n_slices)
    if rc != 0:
        raise RuntimeError("oracle expert_dispatch failed")
    return out
