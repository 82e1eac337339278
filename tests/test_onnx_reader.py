"""ONNX q4f16 reader and NodeBackend weight mapping (CPU only).

The real `model_q4f16.onnx` is not available, so the tests write ONNX files
of their own with the reference's initializer names, dtypes and shapes
(protobuf encoded here, independently of the reader), with some tensors
inline and some in an external data file, unknown fields of every wire
type, and both packed and unpacked dims; then check that the loaded
weights are byte-identical to the tensors written (after the reference's
load transforms).
"""
import numpy as np
import pytest

from textsift_amd import onnx_reader as ox
from textsift_amd import synth
from textsift_amd.backend import HipBackend
from textsift_amd.config import PF_CONFIG

L, E, V = 2, 8, 512


def _varint(n):
    out = bytearray()
    while True:
        b = n & 0x7F
        n >>= 7
        if n:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(field, wire):
    return _varint(field << 3 | wire)


def _ld(field, payload):
    return _key(field, 2) + _varint(len(payload)) + payload


class OnnxWriter:
    """Initializers of a GraphProto, inline or in an external data file."""

    def __init__(self):
        self.tensors = []
        self.ext = bytearray()

    def add(self, name, dtype, dims, data: bytes, external: bool, packed_dims: bool = True):
        t = b""
        if packed_dims:
            t += _ld(1, b"".join(_varint(d) for d in dims))
        else:
            t += b"".join(_key(1, 0) + _varint(d) for d in dims)
        t += _key(2, 0) + _varint(dtype)
        t += _key(3, 5) + b"\x01\x02\x03\x04"       # unknown fixed32 field
        t += _ld(8, name.encode())
        if external:
            off = len(self.ext)
            self.ext += data
            self.ext += b"\x00" * (-len(self.ext) % 64)  # the exporter aligns
            for k, v in (("location", "model.onnx_data"), ("offset", str(off)), ("length", str(len(data)))):
                t += _ld(13, _ld(1, k.encode()) + _key(3, 0) + _varint(7) + _ld(2, v.encode()))
            t += _key(14, 0) + _varint(1)
        else:
            t += _ld(9, data)
        t += _key(12, 1) + b"\x00" * 8               # unknown fixed64 field
        self.tensors.append(t)

    def model_bytes(self):
        graph = _ld(1, b"\x0a\x03abc") + _ld(2, b"main_graph")
        graph += b"".join(_ld(5, t) for t in self.tensors)
        graph += _ld(11, b"\x0a\x01x")             # a graph input, skipped
        return _key(1, 0) + _varint(8) + _ld(8, b"\x0a\x00\x10\x11") + _ld(7, graph) + _ld(2, b"textsift-test")


def write_model(w, path, num_layers=L):
    D, hq = PF_CONFIG.hidden_size, PF_CONFIG.num_heads
    ne = w["layers.0.router.int4"].shape[0]
    wr = OnnxWriter()
    big = lambda a: a.nbytes > 4096
    b = lambda a: np.ascontiguousarray(a).tobytes()

    def mm(base, key, rows, k, router=False):
        nb = k // 32
        sfx = "_weight_fp32" if router else "_weight"  # the router was quantised from an f32 MatMul
        q = w[f"{key}.int4"].reshape(rows, nb, 16)
        wr.add(f"{base}{sfx}_quant", ox.UINT8, q.shape, b(q), big(q))
        if router:  # the router's scales and bias are f32 in the graph
            sc = synth.fp16_bits_to_f32(w[f"{key}.scales"]).astype(np.float32).ravel()
            wr.add(f"{base}{sfx}_scales", ox.FLOAT, sc.shape, b(sc), big(sc), packed_dims=False)
        else:
            sc = w[f"{key}.scales"].ravel()
            wr.add(f"{base}{sfx}_scales", ox.FLOAT16, sc.shape, b(sc), big(sc))
        zp = w[f"{key}.zp"].ravel()
        wr.add(f"{base}{sfx}_zp", ox.UINT8, zp.shape, b(zp), big(zp))

    emb = w["embed.int4"]
    wr.add("model_embed_tokens_weight_quant", ox.UINT8, emb.shape, b(emb), True)
    wr.add("model_embed_tokens_weight_scales", ox.FLOAT16, w["embed.scales"].shape, b(w["embed.scales"]), True)
    wr.add("model_embed_tokens_weight_zp", ox.UINT8, w["embed.zp"].shape, b(w["embed.zp"]), False)
    mm("model_score_MatMul", "score", w["score.int4"].shape[0], D)
    wr.add(f"model.layers.{num_layers}.final_norm_layernorm.weight", ox.FLOAT16, (D,), b(w["final_norm"]), False)
    for l in range(num_layers):
        for n in ("input_layernorm", "post_attention_layernorm"):
            wr.add(f"model.layers.{l}.{n}.weight", ox.FLOAT16, (D,), b(w[f"layers.{l}.{n}"]), False)
        for proj in ("q_proj", "k_proj", "v_proj", "o_proj"):
            key = f"layers.{l}.attn.{proj}"
            rows = w[f"{key}.int4"].shape[0]
            mm(f"model_layers_{l}_attn_{proj}_MatMul", key, rows, w[f"{key}.int4"].shape[1] * 2)
            wr.add(f"model.layers.{l}.attn.{proj}.Add.bias", ox.FLOAT16, (rows,), b(w[f"{key}.bias"]), False)
        snk = w[f"layers.{l}.attn.sinks"].reshape(1, hq, 1, 1)
        wr.add(f"model.layers.{l}.attn.sinks", ox.FLOAT, snk.shape, b(snk), False)
        mm(f"/model/layers_{l}/moe/router/MatMul", f"layers.{l}.router", ne, D, router=True)
        rbias = synth.fp16_bits_to_f32(w[f"layers.{l}.router.bias"]).astype(np.float32)
        wr.add(f"/model/layers.{l}/moe/router/Add.bias_fp32", ox.FLOAT, rbias.shape, b(rbias), False)
        for onnx_proj, key in (("gate_up_proj", "gate_up"), ("down_proj", "down")):
            k = f"layers.{l}.experts.{key}"
            q, sc, bias = w[f"{k}.int4"], w[f"{k}.scales"], w[f"{k}.bias"]
            wr.add(f"model_layers_{l}_moe_experts_{onnx_proj}_weight_quant", ox.UINT8, q.shape, b(q), True)
            wr.add(f"model_layers_{l}_moe_experts_{onnx_proj}_weight_scales", ox.FLOAT16, sc.shape, b(sc), True)
            wr.add(f"model.layers.{l}.moe.experts.{onnx_proj}.bias", ox.FLOAT16, bias.shape, b(bias), False)
    with open(path, "wb") as f:
        f.write(wr.model_bytes())
    with open(str(path) + "_data", "wb") as f:
        f.write(bytes(wr.ext))


@pytest.fixture(scope="module")
def model_files(tmp_path_factory):
    w = synth.make_model_weights(PF_CONFIG, seed=31, num_layers=L, num_experts=E, vocab_size=V)
    path = tmp_path_factory.mktemp("onnx") / "model_q4f16.onnx"
    write_model(w, path)
    return w, str(path)


def test_loaded_weights_match_the_tensors_written(model_files):
    w, path = model_files
    got = ox.load_onnx_weights(path)
    assert set(got) == set(w)
    for k in w:
        a, b = np.ascontiguousarray(got[k]), np.ascontiguousarray(w[k])
        assert a.tobytes() == b.tobytes(), k
    # shapes the backend reads: experts from the router, vocab from the embed table
    be = HipBackend(got)
    assert (be.num_layers, be.num_experts, be.vocab_size) == (L, E, V)


def test_graph_parse_details(model_files):
    _, path = model_files
    with open(path, "rb") as f:
        g = ox.parse_onnx_graph(f.read())
    t = g["model_embed_tokens_weight_quant"]
    assert t.inline is None and t.ext_location == "model.onnx_data" and t.ext_length == V * 320
    assert t.shape == (V, 320) and t.dtype == ox.UINT8
    s = g["model.layers.0.attn.sinks"]
    assert s.inline is not None and s.shape == (1, PF_CONFIG.num_heads, 1, 1) and s.dtype == ox.FLOAT
    r = g["/model/layers_1/moe/router/MatMul_weight_fp32_scales"]
    assert r.shape == (E * 20,)  # unpacked dims
    with pytest.raises(ValueError, match="external but no extData"):
        ox.resolve_tensor_bytes(t, None)


def test_missing_tensor_and_truncation_errors(model_files, tmp_path):
    _, path = model_files
    with open(path, "rb") as f:
        g = ox.parse_onnx_graph(f.read())
    del g["model.layers.1.attn.o_proj.Add.bias"]
    ext = np.memmap(path + "_data", np.uint8, mode="r")
    with pytest.raises(KeyError, match='missing ONNX tensor "model.layers.1.attn.o_proj.Add.bias"'):
        ox.weights_from_graph(g, ext)
    with open(path, "rb") as f:
        data = f.read()
    with pytest.raises(ValueError):
        ox.parse_onnx_graph(data[: len(data) // 2])


def test_layer_count_probe(tmp_path):
    """Layers are counted by input_layernorm; the final norm sits at layer L."""
    w = synth.make_model_weights(PF_CONFIG, seed=32, num_layers=3, num_experts=4, vocab_size=64)
    p = tmp_path / "m.onnx"
    write_model(w, p, num_layers=3)
    got = ox.load_onnx_weights(str(p))
    assert max(int(k.split(".")[1]) for k in got if k.startswith("layers.")) == 2


def _f2h_node_scalar(v):
    """native/backend.ts:239-263, one value, as written there."""
    u = int(np.float32(v).view(np.uint32))
    sign, exp, mant = (u >> 16) & 0x8000, (u >> 23) & 0xFF, u & 0x7FFFFF
    if exp == 0xFF:
        return sign | 0x7C00 | (0x200 if mant else 0)
    if exp == 0:
        return sign
    e = exp - 127 + 15
    if e >= 0x1F:
        return sign | 0x7C00
    if e <= 0:
        return sign
    m, r, sticky = mant >> 13, (mant >> 12) & 1, (mant & 0xFFF) != 0
    h = sign | (e << 10) | m
    if r and (sticky or (m & 1)):
        h += 1
    return h & 0xFFFF


def test_f32_to_fp16_node_transform():
    rng = np.random.default_rng(3)
    specials = np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf, np.nan,
                         6.1e-5, 6.0e-5, 3e-8, 1e-45, -2.5, 2049.0, 2051.0, 1.0009765625, 1.00048828125],
                        np.float32)
    xs = np.concatenate([specials, rng.normal(0, 3, 20000).astype(np.float32),
                         rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    got = ox.f32_to_fp16_node(xs)
    want = np.array([_f2h_node_scalar(v) for v in xs], np.uint16)
    assert np.array_equal(got, want)
    # on normal fp16 results it is IEEE round-to-nearest-even
    normal = (np.abs(xs) >= 2.0 ** -14) & (np.abs(xs) <= 65504) & np.isfinite(xs)
    assert np.array_equal(got[normal], xs[normal].astype(np.float16).view(np.uint16))
