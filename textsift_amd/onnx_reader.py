"""ONNX q4f16 weights -> the backend's named weight tensors (host side).

Restates the reference's minimal ONNX reader and its weight mapping:

  parse_onnx_graph / resolve_tensor_bytes   browser/model/onnx-reader.ts:60-260
      a protobuf decoder for the subset the privacy-filter graph uses:
      ModelProto.graph (7) -> GraphProto.initializer (5) -> TensorProto
      dims (1, packed or not), data_type (2), float_data (4, packed), name (8),
      raw_data (9), external_data (13: location / offset / length),
      data_location (14); every other field is skipped by wire type.
  load_onnx_weights                         native/backend.ts:140-236
      ONNX initializer names -> NodeBackend buffer names, with its load
      transforms: router scales and bias f32 -> fp16 (backend.ts:239-263,
      round to nearest even, subnormals and underflow to signed zero),
      expert zero-points synthesised as 0x88 (the experts ship none),
      a zero fp16 classifier bias, the layer count probed from
      `model.layers.{L}.input_layernorm.weight`, sinks flattened to [Hq].

External data is memory-mapped, so the ~770 MB `.onnx_data` file is read
only where tensors live. The result feeds `HipBackend(weights)` directly.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

import numpy as np

# TensorProto.DataType codes used here (onnx-reader.ts:17-35)
FLOAT, UINT8, INT8, UINT16, INT16, INT32, INT64 = 1, 2, 3, 4, 5, 6, 7
FLOAT16, DOUBLE, UINT32, UINT64, BFLOAT16, UINT4, INT4 = 10, 11, 12, 13, 16, 21, 22


@dataclass
class OnnxTensorRef:
    name: str
    shape: tuple
    dtype: int
    inline: bytes | None      # the bytes when stored in the graph file
    ext_location: str = ""    # otherwise a range of the external data file
    ext_offset: int = 0
    ext_length: int = 0


class _Reader:
    __slots__ = ("b", "pos", "end")

    def __init__(self, b, pos=0, end=None):
        self.b = b
        self.pos = pos
        self.end = len(b) if end is None else end

    @property
    def eof(self):
        return self.pos >= self.end

    def varint(self) -> int:
        result, shift, b = 0, 0, self.b
        while self.pos < self.end:
            c = b[self.pos]
            self.pos += 1
            result |= (c & 0x7F) << shift
            if not c & 0x80:
                return result
            shift += 7
            if shift > 63:
                raise ValueError("ONNX: varint too long")
        raise ValueError("ONNX: varint truncated")

    def skip(self, wire: int):
        if wire == 0:
            self.varint()
        elif wire == 1:
            self.pos += 8
        elif wire == 2:
            n = self.varint()  # read before updating pos (the read moves it)
            self.pos += n
        elif wire == 5:
            self.pos += 4
        else:
            raise ValueError(f"ONNX: unknown wire type {wire}")
        if self.pos > self.end:
            raise ValueError("ONNX: field runs past the end of its message")

    def sub(self) -> "_Reader":
        n = self.varint()
        r = _Reader(self.b, self.pos, self.pos + n)
        if r.end > self.end:
            raise ValueError("ONNX: sub-message runs past the end of its parent")
        self.pos += n
        return r

    def raw(self) -> bytes:
        n = self.varint()
        if self.pos + n > self.end:
            raise ValueError("ONNX: bytes field runs past the end of its message")
        out = bytes(self.b[self.pos:self.pos + n])
        self.pos += n
        return out

    def str(self) -> str:
        return self.raw().decode("utf-8", errors="replace")


def _read_entry(r: _Reader):
    key = value = ""
    while not r.eof:
        tag = r.varint()
        field, wire = tag >> 3, tag & 7
        if field == 1 and wire == 2:
            key = r.str()
        elif field == 2 and wire == 2:
            value = r.str()
        else:
            r.skip(wire)
    return key, value


def _read_tensor(r: _Reader) -> OnnxTensorRef | None:
    name, dtype, dims = "", 0, []
    loc, off, length, external, inline = "", 0, 0, False, None
    while not r.eof:
        tag = r.varint()
        field, wire = tag >> 3, tag & 7
        if field == 8 and wire == 2:
            name = r.str()
        elif field == 2 and wire == 0:
            dtype = r.varint()
        elif field == 1 and wire == 0:
            dims.append(r.varint())
        elif field == 1 and wire == 2:
            s = r.sub()
            while not s.eof:
                dims.append(s.varint())
        elif field == 13 and wire == 2:
            k, v = _read_entry(r.sub())
            if k == "location":
                loc = v
            elif k == "offset":
                off = int(v)
            elif k == "length":
                length = int(v)
            external = True
        elif field == 14 and wire == 0:
            if r.varint() == 1:
                external = True
        elif field in (9, 4) and wire == 2:  # raw_data, or packed float_data (little-endian f32 bytes)
            inline = r.raw()
        else:
            r.skip(wire)
    if not name or (not external and inline is None):
        return None
    return OnnxTensorRef(name, tuple(dims), dtype, None if external else inline, loc, off, length)


def parse_onnx_graph(data) -> dict:
    """name -> OnnxTensorRef for every initializer of the graph."""
    mv = memoryview(data)
    r = _Reader(mv)
    out: dict = {}
    while not r.eof:
        tag = r.varint()
        field, wire = tag >> 3, tag & 7
        if field == 7 and wire == 2:
            g = r.sub()
            while not g.eof:
                t2 = g.varint()
                if (t2 >> 3) == 5 and (t2 & 7) == 2:
                    t = _read_tensor(g.sub())
                    if t is not None:
                        out[t.name] = t
                else:
                    g.skip(t2 & 7)
        else:
            r.skip(wire)
    return out


def resolve_tensor_bytes(t: OnnxTensorRef, ext_data) -> np.ndarray:
    """The tensor's bytes as a uint8 array (a view into ext_data when external)."""
    if t.inline is not None:
        return np.frombuffer(t.inline, np.uint8)
    if ext_data is None:
        raise ValueError(f'tensor "{t.name}" is external but no extData was provided')
    if t.ext_offset + t.ext_length > len(ext_data):
        raise ValueError(f'tensor "{t.name}": external range past the end of the data file')
    return np.asarray(ext_data[t.ext_offset:t.ext_offset + t.ext_length])


def f32_to_fp16_node(src: np.ndarray) -> np.ndarray:
    """NodeBackend's f32 -> fp16 (native/backend.ts:239-263): round to
    nearest even on the 13 dropped bits; f32 zero/subnormal exponents and
    fp16 underflow give signed zero; overflow gives inf; NaN keeps a quiet
    bit."""
    u = np.ascontiguousarray(src, np.float32).view(np.uint32).ravel()
    sign = ((u >> 16) & 0x8000).astype(np.uint32)
    exp = ((u >> 23) & 0xFF).astype(np.int32)
    mant = (u & 0x7FFFFF).astype(np.uint32)
    e = exp - 127 + 15
    m = mant >> 13
    rnd = (mant >> 12) & 1
    sticky = (mant & 0xFFF) != 0
    h = sign | (np.clip(e, 0, 31).astype(np.uint32) << 10) | m
    h = h + ((rnd == 1) & (sticky | ((m & 1) == 1))).astype(np.uint32)
    out = np.where(exp == 0xFF, sign | 0x7C00 | np.where(mant != 0, 0x200, 0),
                   np.where(exp == 0, sign,
                            np.where(e >= 0x1F, sign | 0x7C00,
                                     np.where(e <= 0, sign, h))))
    return (out & 0xFFFF).astype(np.uint16)


def _u16(b: np.ndarray) -> np.ndarray:
    return b.view(np.uint16)


def load_onnx_weights(onnx_path: str, data_path: str | None = None) -> dict:
    """NodeBackend-named weights (uploadWeights, native/backend.ts:140-236)
    from an ONNX q4f16 graph and its external data file (default: the
    graph's path + "_data", as `model_q4f16.onnx_data` sits next to
    `model_q4f16.onnx`)."""
    with open(onnx_path, "rb") as f:
        graph = parse_onnx_graph(f.read())
    if data_path is None:
        data_path = onnx_path + "_data"
    ext = np.memmap(data_path, np.uint8, mode="r") if os.path.exists(data_path) else None
    return weights_from_graph(graph, ext)


def weights_from_graph(graph: dict, ext) -> dict:
    def ref(name):
        t = graph.get(name)
        if t is None:
            raise KeyError(f'uploadWeights: missing ONNX tensor "{name}"')
        return t

    def raw(name):
        return resolve_tensor_bytes(ref(name), ext)

    def rows2(name, rows):
        return raw(name).reshape(rows, -1)

    w: dict = {}
    emb = ref("model_embed_tokens_weight_quant")
    V = emb.shape[0]
    w["embed.int4"] = rows2("model_embed_tokens_weight_quant", V)
    w["embed.scales"] = _u16(raw("model_embed_tokens_weight_scales")).reshape(V, -1)
    w["embed.zp"] = rows2("model_embed_tokens_weight_zp", V)

    num_layers = 0
    for L in range(64):
        if f"model.layers.{L}.input_layernorm.weight" in graph:
            num_layers = L + 1
    if num_layers == 0:
        raise ValueError("uploadWeights: no transformer layers found in ONNX")
    w["final_norm"] = _u16(raw(f"model.layers.{num_layers}.final_norm_layernorm.weight"))

    sq = ref("model_score_MatMul_weight_quant")
    C = sq.shape[0]
    w["score.int4"] = rows2("model_score_MatMul_weight_quant", C)
    w["score.scales"] = _u16(raw("model_score_MatMul_weight_scales")).reshape(C, -1)
    w["score.zp"] = rows2("model_score_MatMul_weight_zp", C)
    w["score.bias"] = np.zeros(C, np.uint16)  # no classifier bias in the graph

    for L in range(num_layers):
        for n in ("input_layernorm", "post_attention_layernorm"):
            w[f"layers.{L}.{n}"] = _u16(raw(f"model.layers.{L}.{n}.weight"))
        for proj in ("q_proj", "k_proj", "v_proj", "o_proj"):
            base = f"model_layers_{L}_attn_{proj}_MatMul"
            k = f"layers.{L}.attn.{proj}"
            N = ref(f"{base}_weight_quant").shape[0]
            w[f"{k}.int4"] = rows2(f"{base}_weight_quant", N)
            w[f"{k}.scales"] = _u16(raw(f"{base}_weight_scales")).reshape(N, -1)
            w[f"{k}.zp"] = rows2(f"{base}_weight_zp", N)
            w[f"{k}.bias"] = _u16(raw(f"model.layers.{L}.attn.{proj}.Add.bias"))
        w[f"layers.{L}.attn.sinks"] = raw(f"model.layers.{L}.attn.sinks").view(np.float32).ravel()
        rb = f"/model/layers_{L}/moe/router/MatMul"
        E = ref(f"{rb}_weight_fp32_quant").shape[0]
        w[f"layers.{L}.router.int4"] = rows2(f"{rb}_weight_fp32_quant", E)
        w[f"layers.{L}.router.scales"] = f32_to_fp16_node(raw(f"{rb}_weight_fp32_scales").view(np.float32)).reshape(E, -1)
        w[f"layers.{L}.router.zp"] = rows2(f"{rb}_weight_fp32_zp", E)
        w[f"layers.{L}.router.bias"] = f32_to_fp16_node(raw(f"/model/layers.{L}/moe/router/Add.bias_fp32").view(np.float32))
        for onnx_proj, key in (("gate_up_proj", "gate_up"), ("down_proj", "down")):
            eb = f"model_layers_{L}_moe_experts_{onnx_proj}"
            k = f"layers.{L}.experts.{key}"
            qs = ref(f"{eb}_weight_quant").shape     # [E, N, K/2]
            ss = ref(f"{eb}_weight_scales").shape    # [E, N, K/32]
            Ee, N, nb = qs[0], qs[1], ss[2]
            w[f"{k}.int4"] = raw(f"{eb}_weight_quant").reshape(Ee, N, -1)
            w[f"{k}.scales"] = _u16(raw(f"{eb}_weight_scales")).reshape(Ee, N, nb)
            w[f"{k}.zp"] = np.full((Ee, N, (nb + 1) // 2), 0x88, np.uint8)  # the experts are centred on 8
            w[f"{k}.bias"] = _u16(raw(f"model.layers.{L}.moe.experts.{onnx_proj}.bias")).reshape(Ee, N)
    return w
