"""ctypes binding of the C ABI in include/pfhip.h (textsift_amd/lib/libpfhip.so).

Loading fails loudly when the library has not been built: there is no CPU
fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

# PFHIP_LIBRARY names another build of the library (e.g. an installed copy)
LIB_PATH = os.environ.get("PFHIP_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                                                           "libpfhip.so")
ERR_CAP = 1024

_lib = None


class PfhipError(RuntimeError):
    pass


# pfhip_model_config.precision (include/pfhip.h)
PRECISION_FP16 = 0
PRECISION_SPLIT = 1


class ModelConfigC(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden", "heads", "kv_heads", "head_dim", "window", "dff", "experts",
                                           "topk", "classes", "vocab", "layers")] + [
        ("eps", C.c_float), ("rope_theta", C.c_double), ("rope_factor", C.c_double),
        ("rope_beta_fast", C.c_double), ("rope_beta_slow", C.c_double),
        ("rope_orig_max", C.c_uint32), ("rope_truncate", C.c_uint32), ("precision", C.c_uint32)]

    @classmethod
    def from_config(cls, cfg, num_layers=None, num_experts=None, vocab_size=None, precision=PRECISION_FP16):
        r = cfg.rope
        return cls(cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.sliding_window,
                   cfg.intermediate_size, cfg.num_experts if num_experts is None else num_experts,
                   cfg.num_experts_per_tok, cfg.num_classes, cfg.vocab_size if vocab_size is None else vocab_size,
                   cfg.num_layers if num_layers is None else num_layers, cfg.rms_norm_eps, r.theta, r.factor,
                   r.beta_fast, r.beta_slow, r.original_max_position_embeddings, int(r.truncate), int(precision))


# (name, restype, argtypes) of every exported entry point of include/pfhip.h
EXPORTS = [
    ("pfhip_version", C.c_char_p, []),
    ("pfhip_create_backend", C.c_void_p, [C.c_int, C.c_char_p, C.c_size_t]),
    ("pfhip_destroy_backend", None, [C.c_void_p]),
    ("pfhip_device_name", C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t]),
    ("pfhip_create_buffer", C.c_void_p, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]),
    ("pfhip_create_empty_buffer", C.c_void_p, [C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]),
    ("pfhip_release_buffer", None, [C.c_void_p, C.c_void_p]),
    ("pfhip_write_buffer", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_char_p,
                                     C.c_size_t]),
    ("pfhip_read_buffer", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_char_p,
                                    C.c_size_t]),
    ("pfhip_buffer_size", C.c_size_t, [C.c_void_p]),
    ("pfhip_buffer_device_ptr", C.c_void_p, [C.c_void_p]),
    ("pfhip_dispatch_one_shot", C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_size_t,
                                          C.c_void_p, C.c_char_p, C.c_size_t]),
    ("pfhip_begin_encoder", C.c_void_p, [C.c_void_p, C.c_char_p, C.c_size_t]),
    ("pfhip_enqueue_dispatch", C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_size_t,
                                         C.c_void_p, C.c_char_p, C.c_size_t]),
    ("pfhip_submit_and_readback", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_char_p,
                                            C.c_size_t]),
    ("pfhip_discard_encoder", None, [C.c_void_p]),
    ("pfhip_kernel_names", C.c_char_p, []),
    ("pfhip_model_create", C.c_void_p, [C.c_void_p, C.POINTER(ModelConfigC), C.c_char_p, C.c_size_t]),
    ("pfhip_model_destroy", None, [C.c_void_p]),
    ("pfhip_model_set_weight", C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]),
    ("pfhip_model_finalize", C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t]),
    ("pfhip_model_forward", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p,
                                      C.c_char_p, C.c_size_t]),
    ("pfhip_model_forward_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32,
                                             C.c_void_p, C.c_char_p, C.c_size_t]),
    ("pfhip_model_forward_device_noalloc", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32,
                                                     C.c_void_p, C.c_char_p, C.c_size_t]),
    ("pfhip_model_read_tap", C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]),
    ("pfhip_model_enable_taps", C.c_int, [C.c_void_p, C.c_int]),
    ("pfhip_model_enable_graphs", C.c_int, [C.c_void_p, C.c_int]),
    ("pfhip_rope_tables", C.c_int, [C.POINTER(ModelConfigC), C.c_uint32, C.c_void_p, C.c_void_p]),
    ("pfhip_profile_enable", C.c_int, [C.c_void_p, C.c_int]),
    ("pfhip_profile_select", C.c_int, [C.c_void_p, C.c_char_p]),
    ("pfhip_profile_reset", C.c_int, [C.c_void_p]),
    ("pfhip_profile_report", C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t]),
    ("pfhip_viterbi_decode", C.c_int, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p,
                                       C.c_void_p, C.c_uint32, C.c_char_p, C.c_size_t]),
]


def lib():
    """Loads libpfhip.so (no compute happens at load time)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise PfhipError(f"{LIB_PATH} is missing: build it with `python -m textsift_amd.build` "
                             "(there is no CPU fallback)")
        l = C.CDLL(LIB_PATH)
        for name, res, args in EXPORTS:
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _err():
    return C.create_string_buffer(ERR_CAP)


def _check(rc, err, what):
    if rc != 0:
        raise PfhipError(f"{what}: {err.value.decode(errors='replace')}")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class Buffer:
    def __init__(self, backend: "Backend", handle: int, size: int):
        self.backend, self.handle, self.size = backend, handle, size

    def write(self, data: np.ndarray, offset: int = 0):
        data = np.ascontiguousarray(data)
        e = _err()
        _check(lib().pfhip_write_buffer(self.backend.handle, self.handle, offset, _ptr(data), data.nbytes, e,
                                        ERR_CAP), e, "write_buffer")

    def read(self, dtype, count=None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.size - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        e = _err()
        _check(lib().pfhip_read_buffer(self.backend.handle, self.handle, offset, _ptr(out), out.nbytes, e, ERR_CAP),
               e, "read_buffer")
        return out

    def release(self):
        if self.handle:
            lib().pfhip_release_buffer(self.backend.handle, self.handle)
            self.handle = 0


class Backend:
    """One GPU (HIP device) with its own stream."""

    def __init__(self, device: int = 0):
        e = _err()
        h = lib().pfhip_create_backend(device, e, ERR_CAP)
        if not h:
            raise PfhipError(f"create_backend: {e.value.decode(errors='replace')}")
        self.handle = h

    @property
    def device_name(self) -> str:
        b = C.create_string_buffer(256)
        lib().pfhip_device_name(self.handle, b, 256)
        return b.value.decode()

    def buffer(self, data: np.ndarray | None = None, nbytes: int | None = None) -> Buffer:
        e = _err()
        if data is not None:
            data = np.ascontiguousarray(data)
            h = lib().pfhip_create_buffer(self.handle, _ptr(data), data.nbytes, e, ERR_CAP)
            n = data.nbytes
        else:
            h = lib().pfhip_create_empty_buffer(self.handle, nbytes, e, ERR_CAP)
            n = nbytes
        if not h:
            raise PfhipError(f"create_buffer: {e.value.decode(errors='replace')}")
        return Buffer(self, h, n)

    def dispatch(self, name: str, bindings, push: bytes | np.ndarray = b""):
        arr = (C.c_void_p * len(bindings))(*[b.handle for b in bindings])
        push = bytes(np.ascontiguousarray(push).tobytes()) if isinstance(push, np.ndarray) else bytes(push)
        pbuf = C.create_string_buffer(push, max(1, len(push)))
        grid = (C.c_uint32 * 3)(1, 1, 1)
        e = _err()
        _check(lib().pfhip_dispatch_one_shot(self.handle, name.encode(), arr, len(bindings), pbuf, len(push), grid, e,
                                             ERR_CAP), e, name)

    def profile(self, on: bool = True):
        lib().pfhip_profile_enable(self.handle, int(on))

    def profile_select(self, name: str | None):
        lib().pfhip_profile_select(self.handle, None if name is None else name.encode())

    def profile_reset(self):
        lib().pfhip_profile_reset(self.handle)

    def profile_report(self) -> dict:
        b = C.create_string_buffer(1 << 16)
        lib().pfhip_profile_report(self.handle, b, 1 << 16)
        out = {}
        for line in b.value.decode().splitlines():
            name, n, ms = line.split()
            out[name] = (int(n), float(ms))
        return out

    def close(self):
        if self.handle:
            lib().pfhip_destroy_backend(self.handle)
            self.handle = 0


class Model:
    """The whole forward (pfhip_model_*)."""

    def __init__(self, backend: Backend, cfg, num_layers=None, num_experts=None, vocab_size=None,
                 precision=PRECISION_FP16):
        self.backend = backend
        self.precision = int(precision)
        self.ccfg = ModelConfigC.from_config(cfg, num_layers, num_experts, vocab_size, precision)
        self.num_classes = cfg.num_classes
        e = _err()
        h = lib().pfhip_model_create(backend.handle, C.byref(self.ccfg), e, ERR_CAP)
        if not h:
            raise PfhipError(f"model_create: {e.value.decode(errors='replace')}")
        self.handle = h

    def set_weight(self, name: str, data: np.ndarray):
        data = np.ascontiguousarray(data)
        e = _err()
        _check(lib().pfhip_model_set_weight(self.handle, name.encode(), _ptr(data), data.nbytes, e, ERR_CAP), e,
               f"set_weight({name})")

    def finalize(self):
        e = _err()
        _check(lib().pfhip_model_finalize(self.handle, e, ERR_CAP), e, "finalize")

    def forward(self, ids: np.ndarray, mask: np.ndarray | None, batch: int, seq_len: int) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        if ids.size != batch * seq_len:
            raise PfhipError("ids length does not match batch * seq_len")
        m = None if mask is None else np.ascontiguousarray(mask, np.uint8)
        if m is not None and m.size != ids.size:
            raise PfhipError(f"attentionMask length {m.size} does not match tokenIds length {ids.size}")
        out = np.empty(ids.size * self.num_classes, np.float32)
        e = _err()
        _check(lib().pfhip_model_forward(self.handle, _ptr(ids), None if m is None else _ptr(m), batch, seq_len,
                                         _ptr(out), e, ERR_CAP), e, "forward")
        return out

    def forward_device(self, ids: Buffer, mask: Buffer | None, batch: int, seq_len: int, logits: Buffer):
        e = _err()
        _check(lib().pfhip_model_forward_device(self.handle, ids.handle, mask.handle if mask else None, batch, seq_len,
                                                logits.handle, e, ERR_CAP), e, "forward_device")

    def forward_device_noalloc(self, ids: Buffer, mask: Buffer | None, batch: int, seq_len: int, logits: Buffer):
        """pfhip_model_forward_device_noalloc: the same forward with its scratch
        in the library's fixed per-GPU array; allocates nothing."""
        e = _err()
        _check(lib().pfhip_model_forward_device_noalloc(self.handle, ids.handle, mask.handle if mask else None, batch,
                                                        seq_len, logits.handle, e, ERR_CAP), e,
               "forward_device_noalloc")

    def enable_taps(self, on: bool = True):
        lib().pfhip_model_enable_taps(self.handle, int(on))

    def enable_graphs(self, on: bool = True):
        """pfhip_model_enable_graphs: replay each (batch, seq_len, buffers)
        forward from a HIP graph after its first call (default on)."""
        lib().pfhip_model_enable_graphs(self.handle, int(on))

    def tap(self, name: str, dtype, count: int) -> np.ndarray:
        out = np.empty(count, np.dtype(dtype))
        e = _err()
        _check(lib().pfhip_model_read_tap(self.handle, name.encode(), _ptr(out), out.nbytes, e, ERR_CAP), e,
               f"tap({name})")
        return out

    def close(self):
        if self.handle:
            lib().pfhip_model_destroy(self.handle)
            self.handle = 0


def rope_tables(cfg, T: int):
    c = ModelConfigC.from_config(cfg)
    half = cfg.head_dim // 2
    cs = np.empty((T, half), np.uint16)
    sn = np.empty((T, half), np.uint16)
    if lib().pfhip_rope_tables(C.byref(c), T, _ptr(cs), _ptr(sn)) != 0:
        raise PfhipError("rope_tables failed")
    return cs, sn


def viterbi_decode(logits: np.ndarray, biases, seq_lens=None, n_threads: int = 0) -> np.ndarray:
    """BIOES Viterbi decode on the host (pfhip_viterbi_decode).
    logits: f32 [T, C] or [B, T, C]; biases: the six calibration biases;
    seq_lens: tokens to decode per sequence (default: all). Returns u8 tags
    of logits' leading shape (entries past a sequence's length are 0)."""
    lg = np.ascontiguousarray(logits, np.float32)
    single = lg.ndim == 2
    if single:
        lg = lg[None]
    if lg.ndim != 3:
        raise ValueError("viterbi_decode: logits must be [T, C] or [B, T, C]")
    B, T, Cn = lg.shape
    bias = np.ascontiguousarray(biases, np.float32).ravel()
    if bias.size != 6:
        raise ValueError("viterbi_decode: expected 6 calibration biases")
    lens = None
    if seq_lens is not None:
        lens = np.ascontiguousarray(np.broadcast_to(np.asarray(seq_lens, np.uint32), (B,)), np.uint32)
    tags = np.zeros((B, T), np.uint8)
    err = _err()
    rc = lib().pfhip_viterbi_decode(_ptr(lg), B, T, None if lens is None else _ptr(lens), Cn, _ptr(bias),
                                    _ptr(tags), n_threads, err, ERR_CAP)
    _check(rc, err, "viterbi_decode")
    return tags[0] if single else tags
