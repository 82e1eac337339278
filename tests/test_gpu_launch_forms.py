"""GPU parity of the kernel forms the 16 x 2048 forward launches that the
smaller tests would not reach: the router GEMM's top-4 epilogue on its
64- and 128-row tiles, the fp16 grouped expert GEMMs (SwiGLU and down, scale-folded
weights) on each of their three tiles, the reference fixtures of the
qmoe_gate_up / qmoe_down_scatter / zero_f32 kernels, and the forward's
row-limit check. All calls go through the C ABI by kernel name."""
import dataclasses

import numpy as np
import pytest

import oracle
from parity_util import f16, rel_err_max, rel_err_norm
from textsift_amd import _native, synth
from textsift_amd.config import PF_CONFIG

pytestmark = pytest.mark.gpu


def u32s(*vals):
    return np.array(vals, np.uint32).tobytes()


@pytest.fixture(scope="module")
def be():
    b = _native.Backend(0)
    yield b
    b.close()


def run(be, name, inputs, outs, pushb):
    """Dispatches `name` with the input arrays followed by output buffers of
    the given byte sizes (or initial arrays); returns the outputs as bytes."""
    bufs = [be.buffer(np.ascontiguousarray(a)) for a in inputs]
    obufs = [be.buffer(np.ascontiguousarray(o)) if isinstance(o, np.ndarray) else be.buffer(nbytes=o) for o in outs]
    be.dispatch(name, bufs + obufs, pushb)
    res = [o.read(np.uint8) for o in obufs]
    for b in bufs + obufs:
        b.release()
    return res


# ---------------------------------------------------------------- router GEMM + top-4 epilogue

@pytest.mark.parametrize("tile,T", [(128, 1000), (128, 129), (64, 1000), (64, 37), (16, 300), (16, 5)])
@pytest.mark.parametrize("kind", ["random", "ties", "nan"])
def test_router_topk_epilogue_bit_exact(be, kind, tile, T):
    """The router GEMM's fused top-4 + softmax (zig/wasm_exports.zig:367-426,
    919-958) on its row tiles: 64 rows (four threads per row, insertion + rank
    merge; the forward's form from 16384 rows on), 128 rows (two threads per
    row) and 16 rows (sorting networks). Expert ids and weights must equal the
    oracle's insertion top-k and softmax of the logits the same launch wrote.
    "ties": every nibble at its zero-point, so each logit is its fp16 bias,
    rounded to integers (many exact ties within and across the segments the
    epilogue merges); "nan": two NaN biases (the sequential replay path)."""
    N, K = 128, 640
    w = synth.qweight(900 + T, N, K, zp=8)
    x = synth.to_fp16_bits(synth.normal(901 + T, T * K)).reshape(T, K)
    if kind != "random":
        w["int4"][:] = 0x88
        bias = np.round(synth.normal(902, N, 0.0, 1.5)).astype(np.float16)
        if kind == "nan":
            bias[[5, 70]] = np.nan
        w["bias"] = bias.view(np.uint16)
    lg, ix, wt = run(be, "matmul_int4_w4_topk", [x, w["int4"], w["scales"], w["zp"], w["bias"]],
                     [T * N * 4, T * 16, T * 16], u32s(T, N, K, tile))
    logits = lg.view(np.float32).reshape(T, N)
    idx = ix.view(np.int32).reshape(T, 4)
    rw = wt.view(np.float32).reshape(T, 4)
    idx_ref, val_ref = oracle.topk(logits, T, N, 4)
    w_ref = oracle.softmax(val_ref, T, 4)
    if kind == "ties":
        assert len(np.unique(logits[0])) < 16
    assert np.array_equal(idx, idx_ref)
    assert np.allclose(rw, w_ref, rtol=0.0, atol=2e-7, equal_nan=True)
    if kind == "random":
        # the logits themselves: the MatMulNBits oracle (f32 out) within the fp16 bar
        ref = oracle.matmul(x, w["int4"], w["scales"], w["zp"], w["bias"], N, K, x_f32=False, out_f32=True)
        assert rel_err_norm(logits, ref) < 2e-3


# ---------------------------------------------------------------- MoE layer in the fp16 numerics

@pytest.mark.parametrize("T,E,tile,dim", [(2048, 128, 64, 640),
                                          (8192, 128, 128, 640),   # the 16 x 2048 forward's tile
                                          (8192, 128, 128, 384),   # down's N = 256 + 128: the half column tile
                                          (37, 16, 16, 640)])      # the all-K 16-token tile
def test_moe_layer_fp16_vs_oracle(be, T, E, tile, dim):
    """moe_ffn in the forward's fp16 numerics: the gemm_w4 grouped SwiGLU
    and down kernels on scale-folded weights (the launches the forward makes),
    with the forward's tile choice, against the oracle's expert-major dispatch
    (browser/inference/expert.ts:104-212, zig/wasm_exports.zig:560-1055) on
    the GPU's routing. Config 3: Zipf(1.1)-skewed router. dim = 384 (hidden and
    intermediate size) runs the down GEMM's last column tile, 128 of its 256
    rows, as the half tile (two fragments on each of the four waves)."""
    cfg = dataclasses.replace(PF_CONFIG, hidden_size=dim, intermediate_size=dim)
    D, F, K = cfg.hidden_size, cfg.intermediate_size, cfg.num_experts_per_tok
    x = synth.to_fp16_bits(synth.normal(710 + T, T * D)).reshape(T, D)
    rw_, rb = synth.zipf_router(711, D, E)
    gu = synth.qweight(712, 2 * F, D, lead=(E,))
    dn = synth.qweight(713, D, F, lead=(E,))
    ins = [x, rw_, np.zeros(1, np.uint8), np.zeros(1, np.uint8), rb, gu["int4"], gu["scales"], gu["zp"], gu["bias"],
           dn["int4"], dn["scales"], dn["zp"], dn["bias"]]
    out, ix, wt = run(be, "moe_ffn", ins, [T * D * 2, T * K * 4, T * K * 4], u32s(T, D, E, K, F, 0, 0, 1))
    y = out.view(np.uint16).reshape(T, D)
    ridx = ix.view(np.int32).reshape(T, K)
    rwt = wt.view(np.float32).reshape(T, K)
    counts = np.bincount(ridx.ravel(), minlength=E)
    assert (T * K // E >= 256) == (tile == 128)
    w = {}
    for kk, vv in gu.items():
        w[f"layers.0.experts.gate_up.{kk}"] = vv
    for kk, vv in dn.items():
        w[f"layers.0.experts.down.{kk}"] = vv
    for name in ("attn.q_proj", "attn.k_proj", "attn.v_proj", "attn.o_proj", "router"):
        for kk, vv in synth.qweight(714, 64, 64).items():
            w[f"layers.0.{name}.{kk}"] = vv
    w["layers.0.input_layernorm"] = w["layers.0.post_attention_layernorm"] = np.zeros(D, np.uint16)
    w["layers.0.attn.sinks"] = np.zeros(14, np.float32)
    ref = oracle.expert_dispatch(cfg, w, 0, oracle.fp16_to_f32(x), ridx, rwt * np.float32(0.25), n_slices=8)
    err = rel_err_norm(f16(y), f16(ref))
    same = float(np.mean(y == ref))
    print(f"moe fp16 T={T} E={E} tile={tile} dim={dim}: rel-err {err:.3e}, identical {same:.4f}; "
          f"load max {counts.max()} min {counts.min()} (experts used {int((counts > 0).sum())})")
    assert err < 2e-3
    # the folded fp16 weights and the fp16 SwiGLU output each add one fp16
    # rounding; most outputs still round to the oracle's value
    assert same > 0.5
    if E == 128 and T == 2048:
        # the Zipf bias skews the load: the first experts take far more than the last
        assert counts[:8].sum() > 4 * counts[-8:].sum()


@pytest.mark.parametrize("T", [2048, 700])
def test_moe_layer_fused_router_chain(be, T):
    """BASELINE config 3 through the chain the forward runs (moe_ffn_w4 with
    the router weight transposed once by transpose_f16): the fp16-weight
    router GEMM whose epilogue takes the top-4 and, above 1024 tokens,
    counts each 64-row tile's picks per expert, the routing plan from those
    counts (one kernel; below 1024 tokens the single-workgroup plan), the
    grouped SwiGLU and down GEMMs and the combine. The routing equals the
    oracle's top-4 (zig/wasm_exports.zig:367-426) on float64 logits of the
    same fp16 inputs except where the 4th and 5th logits tie to within the
    f32 accumulation error; the output is the oracle's expert-major dispatch
    (browser/inference/expert.ts:104-212) of the GPU's routing to rel-err
    < 2e-3; the routing weights are the softmax of the selected logits."""
    cfg = PF_CONFIG
    D, F, K, E = cfg.hidden_size, cfg.intermediate_size, cfg.num_experts_per_tok, cfg.num_experts
    x = synth.to_fp16_bits(synth.normal(720 + T, T * D)).reshape(T, D)
    rw_, rb = synth.zipf_router(721, D, E)
    gu = synth.qweight(722, 2 * F, D, lead=(E,))
    dn = synth.qweight(723, D, F, lead=(E,))
    rwt = run(be, "transpose_f16", [rw_], [D * E * 2], u32s(D, E))[0].view(np.uint16).reshape(E, D)
    assert np.array_equal(rwt, rw_.T)

    def prep(qw, rows, kk):
        w4, sz = run(be, "w4_prepare", [qw["int4"], qw["scales"], qw["zp"]], [E * rows * kk // 2,
                                                                              E * rows * (kk // 32) * 4],
                     u32s(E * rows, kk, 1, 0))
        return [w4, sz, qw["bias"]]
    ins = [x, rwt, rb] + prep(gu, 2 * F, D) + prep(dn, D, F)
    out, ix, wt = run(be, "moe_ffn_w4", ins, [T * D * 2, T * K * 4, T * K * 4], u32s(T, D, E, K, F, 0, 0, 1))
    y = out.view(np.uint16).reshape(T, D)
    ridx = ix.view(np.int32).reshape(T, K)
    rwts = wt.view(np.float32).reshape(T, K)
    # routing vs float64 logits of the same fp16 inputs
    lg = f16(x) @ f16(rw_) + f16(rb)
    srt = -np.sort(-lg, axis=1)
    tie = (srt[:, 3] - srt[:, 4]) < 1e-4 * (np.abs(srt[:, 3]) + 1.0)
    want = np.argsort(-lg, axis=1, kind="stable")[:, :K]
    same = np.all(np.sort(ridx, 1) == np.sort(want, 1), axis=1)
    print(f"fused router chain T={T}: routing rows equal {same.mean():.5f}, near-tied rows {int(tie.sum())}")
    assert np.all(same | tie)
    sel = np.take_along_axis(lg, ridx.astype(np.int64), 1)
    sm = np.exp(sel - sel.max(1, keepdims=True))
    sm /= sm.sum(1, keepdims=True)
    assert np.allclose(rwts, sm, rtol=0, atol=1e-5)
    assert np.all(np.diff(np.take_along_axis(lg, ridx.astype(np.int64), 1)[~tie], axis=1) <= 1e-4)  # sorted
    w = {}
    for kk, vv in gu.items():
        w[f"layers.0.experts.gate_up.{kk}"] = vv
    for kk, vv in dn.items():
        w[f"layers.0.experts.down.{kk}"] = vv
    for name in ("attn.q_proj", "attn.k_proj", "attn.v_proj", "attn.o_proj", "router"):
        for kk, vv in synth.qweight(724, 64, 64).items():
            w[f"layers.0.{name}.{kk}"] = vv
    w["layers.0.input_layernorm"] = w["layers.0.post_attention_layernorm"] = np.zeros(D, np.uint16)
    w["layers.0.attn.sinks"] = np.zeros(14, np.float32)
    ref = oracle.expert_dispatch(cfg, w, 0, oracle.fp16_to_f32(x), ridx, rwts * np.float32(0.25), n_slices=8)
    err = rel_err_norm(f16(y), f16(ref))
    print(f"fused router chain T={T}: MoE output rel-err {err:.3e}")
    assert err < 2e-3


# ---------------------------------------------------------------- reference fixtures not run elsewhere

def test_qmoe_gate_up_fixture(be, fixture):
    """qmoe_gate_up (native/shaders/qmoe_gate_up.wgsl) on its conformance
    fixture, reference tolerance for f32 outputs: relative drift <= 1 %
    (tests/native/vulkan/conformance-all.js:146-168); ours is f32-grade."""
    fx = fixture("qmoe_gate_up")
    ins = [fx.input("x", np.float32), fx.input("routing_idx", np.int32), fx.input("w_int4"),
           fx.input("w_scales", np.uint16), fx.input("w_zp"), fx.input("bias", np.uint16)]
    (out,) = run(be, "qmoe_gate_up", ins, [fx.meta["output"]["byteLength"]], fx.raw("uniform.bin").tobytes())
    got, exp = out.view(np.float32), fx.expected(np.float32)
    rel = np.abs(got - exp) / np.maximum(np.abs(exp), 1e-6)
    print(f"qmoe_gate_up: max rel drift {rel.max():.2e}")
    assert rel.max() <= 1e-2
    assert rel_err_max(got, exp) < 1e-5


def test_qmoe_down_scatter_fixture(be, fixture):
    """qmoe_down_scatter (qmoe_down_scatter.wgsl, atomic f32 accumulate onto
    the output's initial contents) on its conformance fixture."""
    fx = fixture("qmoe_down_scatter")
    ins = [fx.input("glu", np.float32), fx.input("routing_idx", np.int32), fx.input("routing_scores", np.float32),
           fx.input("w_int4"), fx.input("w_scales", np.uint16), fx.input("w_zp"), fx.input("bias", np.uint16)]
    init = fx.raw("_output_initial.bin", np.float32)
    (out,) = run(be, "qmoe_down_scatter", ins, [init], fx.raw("uniform.bin").tobytes())
    got, exp = out.view(np.float32), fx.expected(np.float32)
    rel = np.abs(got - exp) / np.maximum(np.abs(exp), 1e-6)
    print(f"qmoe_down_scatter: max rel drift {rel.max():.2e}")
    assert rel.max() <= 1e-2
    assert rel_err_max(got, exp) < 1e-5


def test_zero_f32_fixture(be, fixture):
    """zero_f32 on its fixture: u32 output, byte-equal (conformance-all.js:171-180)."""
    fx = fixture("zero_f32")
    init = fx.raw("_output_initial.bin", np.uint8)
    (out,) = run(be, "zero_f32", [], [init], fx.raw("uniform.bin").tobytes())
    exp = fx.expected(np.uint8)
    assert np.array_equal(out[:exp.size], exp)


# ---------------------------------------------------------------- row limits

def test_forward_row_limit_is_checked_before_any_work(be):
    """A batch whose routed expert plane ([rows * topk][dff]) would pass the
    kernels' 32-bit element offsets is refused with an error before scratch
    is allocated or a kernel launched (the model has no weights uploaded, so
    reaching any later step would fail differently)."""
    import dataclasses
    cfg = dataclasses.replace(PF_CONFIG, hidden_size=128, num_heads=2, num_kv_heads=1, head_dim=64,
                              intermediate_size=1 << 20, num_experts=8, num_experts_per_tok=8, num_layers=1,
                              vocab_size=64)
    m = _native.Model(be, cfg)
    ids = be.buffer(np.zeros(512, np.int32))
    logits = be.buffer(nbytes=512 * cfg.num_classes * 4)
    try:
        with pytest.raises(RuntimeError, match="32-bit offsets"):
            m.forward_device(ids, None, 1, 512, logits)
        # a batch within the limit gets as far as the finalize check
        with pytest.raises(RuntimeError, match="finalize"):
            m.forward_device(ids, None, 1, 255, logits)
    finally:
        ids.release()
        logits.release()
        m.close()
