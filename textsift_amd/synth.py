"""Seeded synthetic inputs and random-init weights in MatMulNBits layout.

There is no network and no model checkpoint here, so every workload is
generated from fixed 64-bit seeds. Randomness is counter based (SplitMix64
of seed and element index) so any tensor can be regenerated independently,
in vectorised numpy, on any host.

Weight names and byte layouts are the ones NodeBackend uploads
(packages/textsift/src/native/backend.ts:140-236):

  embed.int4 [V, D/2] u8        embed.scales [V, D/32] f16   embed.zp [V, ceil(D/64)] u8
  layers.L.input_layernorm [D] f16, layers.L.post_attention_layernorm [D] f16
  layers.L.attn.{q,k,v,o}_proj.{int4,scales,zp,bias}
  layers.L.attn.sinks [Hq] f32
  layers.L.router.{int4,scales,zp,bias}          (router scales/bias already fp16)
  layers.L.experts.{gate_up,down}.{int4,scales,zp,bias}  ([E, N, ...], zp 0x88)
  final_norm [D] f16
  score.{int4,scales,zp,bias}                    (bias all zero, backend.ts:190)

fp16 tensors are carried as uint16 bit patterns. Generated fp16 values
flush subnormals to +-0: the reference's fp16 widen is not IEEE for
subnormals (zig/math.zig:45-52), GPU hardware is.
"""
from __future__ import annotations

import numpy as np

from .config import PF_CONFIG, QBLOCK, ModelConfig

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def u64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n pseudo-random uint64 for (seed, index) pairs."""
    idx = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        base = _splitmix64(np.array([seed & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64))[0]
        return _splitmix64(idx * np.uint64(0xD1B54A32D192ED03) + base)


def random_bytes(seed: int, n: int) -> np.ndarray:
    words = u64(seed, (n + 7) // 8)
    return words.view(np.uint8)[:n].copy()


def uniform(seed: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """float64 uniform in [lo, hi) from the top 53 bits."""
    v = (u64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return lo + (hi - lo) * v


def normal(seed: int, n: int, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    """Box-Muller normals (float64)."""
    m = (n + 1) // 2
    u1 = uniform(seed, m)
    u2 = uniform(seed ^ 0x5DEECE66D, m)
    r = np.sqrt(-2.0 * np.log1p(-u1))
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
    return mu + sigma * z


def to_fp16_bits(values: np.ndarray) -> np.ndarray:
    """IEEE RNE to fp16 bit patterns with subnormals flushed to +-0."""
    h = np.asarray(values, dtype=np.float32).astype(np.float16)
    tiny = np.abs(h.astype(np.float32)) < np.float32(2.0 ** -14)
    h = np.where(tiny, np.copysign(np.float16(0), h), h)
    return h.view(np.uint16)


def fp16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def zp_bytes(n_rows: int, k: int, zp: int = 8) -> np.ndarray:
    """Packed uint4 zero-points [n_rows, ceil(k/32/2)] all equal to zp."""
    nb = k // QBLOCK
    return np.full((n_rows, (nb + 1) // 2), (zp & 0xF) | ((zp & 0xF) << 4), dtype=np.uint8)


def qweight(seed: int, n: int, k: int, scale_lo: float = 0.005, scale_hi: float = 0.02,
            zp: int | None = 8, bias_sigma: float | None = 0.02, lead: tuple = ()) -> dict:
    """One MatMulNBits weight: uniform nibbles, fp16 scales ~U(lo,hi),
    packed zero-points (zp=None -> uniform random nibbles), fp16 bias."""
    if k % QBLOCK:
        raise ValueError(f"K={k} must be a multiple of {QBLOCK}")
    rows = int(np.prod(lead, dtype=np.int64)) * n if lead else n
    nb = k // QBLOCK
    out = {
        "int4": random_bytes(seed, rows * k // 2).reshape(*lead, n, k // 2),
        "scales": to_fp16_bits(uniform(seed + 1, rows * nb, scale_lo, scale_hi)).reshape(*lead, n, nb),
    }
    if zp is None:
        out["zp"] = random_bytes(seed + 2, rows * ((nb + 1) // 2)).reshape(*lead, n, (nb + 1) // 2)
    else:
        out["zp"] = zp_bytes(rows, k, zp).reshape(*lead, n, (nb + 1) // 2)
    if bias_sigma is None:
        out["bias"] = np.zeros((*lead, n), dtype=np.uint16)
    else:
        out["bias"] = to_fp16_bits(normal(seed + 3, rows, 0.0, bias_sigma)).reshape(*lead, n)
    return out


def make_model_weights(cfg: ModelConfig = PF_CONFIG, seed: int = 20260101, *, num_layers: int | None = None,
                       num_experts: int | None = None, vocab_size: int | None = None,
                       attn_scale=(0.002, 0.006)) -> dict:
    """Random-init weights of the privacy-filter architecture.

    Scales are U(0.005, 0.02) except Q/K, whose scales
    are smaller (attn_scale) so that with the model's unscaled Q.K
    (browser/inference/attention.ts:139-145) attention logits stay O(1-5)
    instead of saturating the softmax.
    """
    L = cfg.num_layers if num_layers is None else num_layers
    E = cfg.num_experts if num_experts is None else num_experts
    V = cfg.vocab_size if vocab_size is None else vocab_size
    D, Hq, Hkv, hd, dff = cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size
    w: dict = {}
    s = seed * 1000

    def put(prefix: str, qw: dict):
        for k, v in qw.items():
            w[f"{prefix}.{k}"] = v

    put("embed", qweight(s + 1, V, D, bias_sigma=None))
    del w["embed.bias"]
    for l in range(L):
        b = s + 100 * (l + 1)
        w[f"layers.{l}.input_layernorm"] = to_fp16_bits(normal(b + 1, D, 1.0, 0.1))
        w[f"layers.{l}.post_attention_layernorm"] = to_fp16_bits(normal(b + 2, D, 1.0, 0.1))
        put(f"layers.{l}.attn.q_proj", qweight(b + 10, Hq * hd, D, *attn_scale))
        put(f"layers.{l}.attn.k_proj", qweight(b + 20, Hkv * hd, D, *attn_scale))
        put(f"layers.{l}.attn.v_proj", qweight(b + 30, Hkv * hd, D))
        put(f"layers.{l}.attn.o_proj", qweight(b + 40, D, Hq * hd))
        w[f"layers.{l}.attn.sinks"] = normal(b + 50, Hq, 0.0, 1.0).astype(np.float32)
        put(f"layers.{l}.router", qweight(b + 60, E, D))
        put(f"layers.{l}.experts.gate_up", qweight(b + 70, 2 * dff, D, lead=(E,)))
        put(f"layers.{l}.experts.down", qweight(b + 80, D, dff, lead=(E,)))
    w["final_norm"] = to_fp16_bits(normal(s + 7, D, 1.0, 0.1))
    put("score", qweight(s + 9, cfg.num_classes, D, bias_sigma=None))
    return w


def zipf_router(seed: int, d: int, e: int, s: float = 1.1, strength: float = 0.32):
    """BASELINE config 3's router: fp16 W [d][e] ~ N(0, 0.02) and an fp16
    bias of -s * strength * ln(rank) (rank = expert id + 1), which skews the
    realised top-k load towards Zipf(s). strength 0.32 is calibrated for
    d = 640, e = 128, top-4 over 2048 N(0, 1) rows: a log-log fit over the 32
    most-loaded experts gives s = 1.10, and the 8 most-loaded take 58 % of
    the assignments (Zipf(1.1) over 128 ranks: 57 %).
    Returns (W bits [d][e], bias bits [e])."""
    w = to_fp16_bits(normal(seed, d * e, 0, 0.02)).reshape(d, e)
    bias = to_fp16_bits(s * -np.log(np.arange(1, e + 1)) * strength)
    return w, bias


def token_ids(seed: int, n: int, vocab: int = PF_CONFIG.vocab_size) -> np.ndarray:
    """Token ids uniform over [0, vocab) (BASELINE configs 2 and 5)."""
    return (u64(seed, n) % np.uint64(vocab)).astype(np.int32)
