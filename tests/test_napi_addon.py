"""The Node-API module (textsift_amd/lib/textsift-hip.node, csrc/hip_napi.cc)
driven from Node by tests/napi/addon.js, the way textsift's NodeBackend drives
its native modules (src/native/backend.ts:34-131; napi.zig:546-864).

CPU: the module loads in Node 12, exports every verb, lists the reference's
kernel names, turns a missing GPU and bad arguments into JS Errors (never an
abort: the condition under which src/index.ts:69-103 falls back to WASM), and
its Viterbi decode (host only) equals the library's through ctypes and the
vectorised restatement of viterbi.ts. GPU: a whole forward through hipForward
equals the ctypes forward bit for bit, and a reference conformance fixture runs
through hipDispatchOneShot and through an encoder."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from textsift_amd import _native, build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, "tests", "napi", "addon.js")
NODE = shutil.which("node")

REFERENCE_KERNELS = ["rms_norm", "zero_f32", "cast_fp16_to_f32", "cast_f32_to_fp16_scaled", "add_fp16",
                     "add_rmsnorm_fp16_to_f32", "embed_lookup_int4", "matmul_int4_fp16_f16", "matmul_int4_f32_f32",
                     "rope_apply", "banded_attention", "router_topk", "qmoe_gate_up", "swiglu_clamp",
                     "qmoe_down_scatter"]

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


@pytest.fixture(scope="module")
def addon():
    if not os.path.exists(build.ADDON):
        _native.lib()
        if build.build_addon() is None:
            pytest.skip("Node headers not installed: the module was not built")
    return build.ADDON


def node(*args, timeout=120):
    r = subprocess.run([NODE, SCRIPT, *args], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr[-3000:]
    return r.stdout


def test_surface_and_errors(addon):
    out = json.loads(node("surface").strip().splitlines()[-1])
    assert out["missing"] == []
    assert out["version"].startswith("textsift-amd")
    assert set(REFERENCE_KERNELS) <= set(out["kernels"])
    assert out["bad_argument_errors"] == []
    be = out["backend"]
    if "threw" in be:  # no GPU here: a JS Error with the library's message, not an abort
        assert be["threw"] and "createBackend failed" in be["message"]
    else:
        assert be["created"]


def _tables_free_viterbi_inputs(seed, B, S):
    rng = np.random.default_rng(seed)
    logits = rng.normal(0, 2, (B, S, 33)).astype(np.float32)
    lens = rng.integers(1, S + 1, B).astype(np.uint32)
    biases = rng.normal(0, 0.5, 6).astype(np.float32)
    return logits, lens, biases


def test_viterbi_through_node_equals_library(addon, tmp_path):
    from test_spans import _tables, _viterbi_vectorized
    B, S = 5, 97
    logits, lens, biases = _tables_free_viterbi_inputs(3, B, S)
    logits.tofile(tmp_path / "logits.bin")
    (tmp_path / "meta.json").write_text(json.dumps({"batch": B, "seq_stride": S, "seq_lens": lens.tolist(),
                                                    "biases": biases.tolist(), "threads": 2}))
    node("viterbi", str(tmp_path))
    got = np.fromfile(tmp_path / "tags.bin", np.uint8).reshape(B, S)
    want = _native.viterbi_decode(logits, biases, lens.tolist())
    for b in range(B):
        n = int(lens[b])
        assert np.array_equal(got[b, :n], want[b, :n])
        trans, start = _tables(biases)
        assert np.array_equal(got[b, :n], _viterbi_vectorized(logits[b, :n], trans, start))


@pytest.mark.gpu
def test_forward_through_node_equals_ctypes(addon, tmp_path):
    from textsift_amd import synth
    from textsift_amd.backend import HipBackend
    from textsift_amd.config import PF_CONFIG
    L, E, V, B, T = 2, 16, 4096, 2, 300
    w = synth.make_model_weights(PF_CONFIG, seed=31, num_layers=L, num_experts=E, vocab_size=V)
    ids = synth.token_ids(32, B * T, V)
    man = {"config": {"layers": L, "experts": E, "vocab": V}, "batch": B, "seq_len": T, "weights": []}
    for i, (name, arr) in enumerate(w.items()):
        f = f"w{i}.bin"
        np.ascontiguousarray(arr).tofile(tmp_path / f)
        man["weights"].append({"name": name, "file": f})
    (tmp_path / "manifest.json").write_text(json.dumps(man))
    ids.tofile(tmp_path / "ids.bin")
    print(node("forward", str(tmp_path)))
    got = np.fromfile(tmp_path / "logits.bin", np.float32).reshape(B, T, 33)
    be = HipBackend(w)
    be.warmup()
    try:
        want = be.forward_batch(ids.reshape(B, T))
    finally:
        be.dispose()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_reference_fixture_through_node(addon, tmp_path, fixture):
    """matmul_int4_fp16_f16's conformance fixture, through hipDispatchOneShot
    and through an encoder: within 1 fp16 ulp of the WGSL output (the
    reference's own bar, tests/native/vulkan/conformance-all.js:31-44)."""
    from parity_util import fp16_ulp_diff
    fx = fixture("matmul_int4_fp16_f16")
    out = tmp_path / "out.bin"
    node("fixture", fx.dir, str(out))
    both = np.fromfile(out, np.uint16)
    n = both.size // 2
    exp = fx.expected(np.uint16)
    for half in (both[:n], both[n:]):
        assert fp16_ulp_diff(half, exp).max() <= 1.0
