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


def centred_nibbles(b: np.ndarray) -> np.ndarray:
    """Maps each nibble value 0 to 8 in place: uniform nibbles 0..15 become
    1..15 with 8 twice as likely, so q - 8 is symmetric about 0 (mean 0,
    E[(q-8)^2] = 17.5) instead of having mean -0.5."""
    lo = b & 0x0F
    hi = b & 0xF0
    lo = np.where(lo == 0, 8, lo).astype(np.uint8)
    hi = np.where(hi == 0, 0x80, hi).astype(np.uint8)
    return (lo | hi).astype(np.uint8)


def qweight(seed: int, n: int, k: int, scale_lo: float = 0.005, scale_hi: float = 0.02,
            zp: int | None = 8, bias_sigma: float | None = 0.02, lead: tuple = (),
            nibbles: str = "uniform") -> dict:
    """One MatMulNBits weight: nibbles uniform over 0..15 (nibbles="uniform")
    or centred on 8 (nibbles="centred", see centred_nibbles), fp16 scales
    ~U(lo,hi), packed zero-points (zp=None -> uniform random nibbles), fp16
    bias."""
    if k % QBLOCK:
        raise ValueError(f"K={k} must be a multiple of {QBLOCK}")
    if nibbles not in ("uniform", "centred"):
        raise ValueError(f"nibbles={nibbles!r}")
    rows = int(np.prod(lead, dtype=np.int64)) * n if lead else n
    nb = k // QBLOCK
    q = random_bytes(seed, rows * k // 2)
    if nibbles == "centred":
        q = centred_nibbles(q)
    out = {
        "int4": q.reshape(*lead, n, k // 2),
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


# Router skew of the "spread" recipe: expert e's router bias is
# -ROUTER_SKEW * sigma * ln(rank_e), sigma = the std of the router logits
# (sqrt(D) * rms(weight)) and rank_e a per-layer random permutation of
# 1..E. Calibrated so that each layer of the full model's realised top-4
# load sits where openai/privacy-filter's measured routing does
# (docs/stage3-gate-measurement.md:35-55: no expert above 10 %, the top 20 %
# of experts take 43-58 % of the picks, at most 2 experts under 0.1 %).
ROUTER_SKEW = 0.28

# Conditioning of the "spread" recipe. With zero-mean weights and every
# scale ~U(0.005, 0.02), each block adds vectors 20-25x the size of the
# embedding to the residual stream and the network is chaotic: a 1e-3
# relative perturbation of the norm outputs grows to 5.7e-2 on the logits
# after 2 layers, so no two implementations that round differently (fp16 vs
# f32 GEMM inputs) could agree. Trained residual networks keep each block's
# contribution a fraction of the stream. Here the embedding scales are 16x
# larger, the attention output projection's 16x smaller and the experts'
# down projection's 32x smaller, so attention adds about 7 % and the MoE
# about 5 % of the stream per layer and a 1e-4 perturbation stays at the
# 1e-4 level through 8 layers. The MoE share is the smaller one because a
# token whose 4th and 5th router logits nearly tie may take either expert
# (both are correct to the inputs' precision); the MoE output's size sets
# how far such a token's logits move (measured on the GPU at 16 x 2048:
# logit rel-err vs the CPU restatement of the WASM path 2.0e-3 with the
# down projection at 1/16 and the router scales at 1x, 0.8e-3 as chosen
# here).
EMBED_SCALE = (0.08, 0.32)
OUT_PROJ_SCALE = (0.0003125, 0.00125)
OUT_PROJ_BIAS_SIGMA = 0.00125
EXPERT_DOWN_SCALE = (0.00015625, 0.000625)
EXPERT_DOWN_BIAS_SIGMA = 0.000625
# Router weight scales (8x the others): router logits with a std of ~12 put
# most of the top-4 softmax weight on the first experts, so a near-tied
# token's MoE output moves little whichever 4th expert it takes.
ROUTER_SCALE = (0.04, 0.16)

# Planted classes of the "spread" recipe. A random classifier over random
# features is never confident: the top two of 33 logits are within one fp16
# ulp of each other for ~0.5 % of tokens, so any two correct implementations
# that round differently disagree on that many argmaxes. A trained token
# classifier is confident. Token id v carries class v mod 33 (a BIOES tag):
# its embedding row is the centred nibbles plus PLANT * u_c (u_c a random
# +-1 direction per class, nibbles clipped to 1..15), and classifier row c is
# the centred nibbles plus PLANT * u_c. The class signal survives the 8
# layers with a top-1/top-2 margin of several standard deviations, and a
# legal BIOES sequence of tags (tagged_token_ids) decodes to itself.
PLANT = 3


def _rms_scale(lo: float, hi: float) -> float:
    """sqrt(E[s^2]) of s ~ U(lo, hi)."""
    return float(np.sqrt((hi ** 3 - lo ** 3) / (3.0 * (hi - lo))))


def make_model_weights(cfg: ModelConfig = PF_CONFIG, seed: int = 20260101, *, num_layers: int | None = None,
                       num_experts: int | None = None, vocab_size: int | None = None,
                       attn_scale=(0.002, 0.006), recipe: str = "spread") -> dict:
    """Random-init weights of the privacy-filter architecture.

    Scales are U(0.005, 0.02) except Q/K, whose scales
    are smaller (attn_scale) so that with the model's unscaled Q.K
    (browser/inference/attention.ts:139-145) attention logits stay O(1-5)
    instead of saturating the softmax.

    recipe="spread" (the default): nibbles centred on the zero-point 8
    (centred_nibbles), a per-layer router bias of -ROUTER_SKEW * sigma *
    ln(rank), the conditioning of EMBED_SCALE / OUT_PROJ_SCALE /
    EXPERT_DOWN_SCALE / ROUTER_SCALE, and planted classes (PLANT). Every
    weight then has mean 0, as trained weights do, tokens stay distinct
    through the 8 layers, every expert is routed to, the classifier's argmax
    spreads over all classes, and rounding differences stay small.

    recipe="uniform": nibbles uniform over 0..15 and router bias ~N(0, 0.02),
    the recipe of BASELINE config 1 applied to every weight. q - 8 then has
    mean -0.5, so every weight row carries a common -0.5 * scale offset; each
    GEMM maps it onto the sum of its input, the residual stream converges to
    one direction shared by all tokens (cosine 0.98 to its mean after layer
    0, |h| ~ 2e4 by layer 7), routing collapses onto 4-8 experts from layer 1
    and every token takes the same class. Kept to compare against earlier
    measurements only.
    """
    if recipe not in ("spread", "uniform"):
        raise ValueError(f"recipe={recipe!r}")
    L = cfg.num_layers if num_layers is None else num_layers
    E = cfg.num_experts if num_experts is None else num_experts
    V = cfg.vocab_size if vocab_size is None else vocab_size
    D, Hq, Hkv, hd, dff = cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size
    nib = "centred" if recipe == "spread" else "uniform"
    w: dict = {}
    s = seed * 1000

    def put(prefix: str, qw: dict):
        for k, v in qw.items():
            w[f"{prefix}.{k}"] = v

    spread = recipe == "spread"
    put("embed", qweight(s + 1, V, D, *(EMBED_SCALE if spread else (0.005, 0.02)), bias_sigma=None, nibbles=nib))
    del w["embed.bias"]
    if spread:
        u = class_directions(s + 5, cfg.num_classes, D)
        w["embed.int4"] = _plant(w["embed.int4"], u[np.arange(V) % cfg.num_classes])
    for l in range(L):
        b = s + 100 * (l + 1)
        w[f"layers.{l}.input_layernorm"] = to_fp16_bits(normal(b + 1, D, 1.0, 0.1))
        w[f"layers.{l}.post_attention_layernorm"] = to_fp16_bits(normal(b + 2, D, 1.0, 0.1))
        put(f"layers.{l}.attn.q_proj", qweight(b + 10, Hq * hd, D, *attn_scale, nibbles=nib))
        put(f"layers.{l}.attn.k_proj", qweight(b + 20, Hkv * hd, D, *attn_scale, nibbles=nib))
        put(f"layers.{l}.attn.v_proj", qweight(b + 30, Hkv * hd, D, nibbles=nib))
        out_kw = dict(scale_lo=OUT_PROJ_SCALE[0], scale_hi=OUT_PROJ_SCALE[1],
                      bias_sigma=OUT_PROJ_BIAS_SIGMA) if spread else {}
        put(f"layers.{l}.attn.o_proj", qweight(b + 40, D, Hq * hd, nibbles=nib, **out_kw))
        w[f"layers.{l}.attn.sinks"] = normal(b + 50, Hq, 0.0, 1.0).astype(np.float32)
        put(f"layers.{l}.router", qweight(b + 60, E, D, *(ROUTER_SCALE if spread else (0.005, 0.02)), nibbles=nib))
        if spread:
            sigma = np.sqrt(D * 17.5) * _rms_scale(*ROUTER_SCALE)
            rank = np.empty(E)
            rank[np.argsort(u64(b + 61, E), kind="stable")] = np.arange(1, E + 1)
            w[f"layers.{l}.router.bias"] = to_fp16_bits(-ROUTER_SKEW * sigma * np.log(rank))
        put(f"layers.{l}.experts.gate_up", qweight(b + 70, 2 * dff, D, lead=(E,), nibbles=nib))
        down_kw = dict(scale_lo=EXPERT_DOWN_SCALE[0], scale_hi=EXPERT_DOWN_SCALE[1],
                       bias_sigma=EXPERT_DOWN_BIAS_SIGMA) if spread else {}
        put(f"layers.{l}.experts.down", qweight(b + 80, D, dff, lead=(E,), nibbles=nib, **down_kw))
    w["final_norm"] = to_fp16_bits(normal(s + 7, D, 1.0, 0.1))
    put("score", qweight(s + 9, cfg.num_classes, D, bias_sigma=None, nibbles=nib))
    if spread:
        w["score.int4"] = _plant(w["score.int4"], u)
    return w


def class_directions(seed: int, n_classes: int, d: int) -> np.ndarray:
    """One random +-1 direction per class: int8 [n_classes, d]."""
    return np.where(u64(seed, n_classes * d) & np.uint64(1), 1, -1).astype(np.int8).reshape(n_classes, d)


def _plant(packed: np.ndarray, dirs: np.ndarray) -> np.ndarray:
    """Adds PLANT * dirs (int8 [rows, K]) to the nibbles of a packed uint4
    [rows, K/2] weight (low nibble = even k), clipped to 1..15."""
    lo = (packed & 0x0F).astype(np.int16) + PLANT * dirs[:, 0::2]
    hi = (packed >> 4).astype(np.int16) + PLANT * dirs[:, 1::2]
    lo = np.clip(lo, 1, 15).astype(np.uint8)
    hi = np.clip(hi, 1, 15).astype(np.uint8)
    return (lo | (hi << 4)).astype(np.uint8)


def routing_load(idx: np.ndarray, num_experts: int) -> dict:
    """Statistics of a realised top-k load (idx [T, k] expert ids): experts
    touched, the largest expert's share, the share of the top 20 % of
    experts, and the number of experts under 0.1 % of the picks -- the
    figures docs/stage3-gate-measurement.md:35-55 reports per layer."""
    cnt = np.sort(np.bincount(np.asarray(idx).ravel(), minlength=num_experts))[::-1]
    tot = max(int(cnt.sum()), 1)
    top = max(1, int(round(0.2 * num_experts)))
    return {"touched": int(np.count_nonzero(cnt)), "max_share": float(cnt[0] / tot),
            "top20_share": float(cnt[:top].sum() / tot), "under_0p1pct": int(np.sum(cnt < 0.001 * tot))}


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


def tag_sequence(seed: int, n: int, n_labels: int = 8) -> np.ndarray:
    """A legal BIOES tag sequence (viterbi.ts:159-219 transitions) of n tags
    in which every tag of the 33 is equally frequent: segments O, S-l and
    B-l I-l E-l with equal counts (a 3-token run per label for each S-l, one
    O per label's worth of tags), in random order, labels uniform. Tag ids
    are browser/inference/viterbi.ts's: 0 = O, 1 + 4 l + {0,1,2,3} = B, I,
    E, S of label l."""
    n_classes = 1 + 4 * n_labels
    # one "unit" = for one label: B I E and S (4 tags) -- n_labels units per O
    n_units = -(-n * n_labels // n_classes) + n_labels
    r = u64(seed, 3 * n_units + n)
    labels = (r[:n_units] % np.uint64(n_labels)).astype(np.int64)
    order = np.argsort(r[n_units:3 * n_units], kind="stable")  # 2 segments per unit, shuffled
    segs = []
    for j in order:
        lab = labels[j // 2]
        segs.append([1 + 4 * lab, 2 + 4 * lab, 3 + 4 * lab] if j % 2 == 0 else [4 + 4 * lab])
    out = []
    k = 0
    for i, seg in enumerate(segs):
        if i % (2 * n_labels) == 0:
            out.append(0)  # O once per 2 * n_labels segments (n_labels units)
        out.extend(seg)
        if len(out) >= n:
            break
    return np.array(out[:n], np.int32)


def tagged_token_ids(seed: int, n: int, vocab: int = PF_CONFIG.vocab_size, n_classes: int = 33) -> np.ndarray:
    """Token ids whose planted classes (v mod n_classes) follow tag_sequence:
    each id uniform within its class, so with the tags equally frequent every
    id of the vocabulary is (up to the classes' sizes differing by one) equally
    likely, as in BASELINE config 5's uniform ids; the model's classifier then
    sees legal BIOES runs, spans of 1-3 tokens."""
    tags = tag_sequence(seed, n, (n_classes - 1) // 4).astype(np.int64)
    per_class = (vocab - 1 - tags) // n_classes + 1
    j = (u64(seed + 1, n) % per_class.astype(np.uint64)).astype(np.int64)
    return (tags + n_classes * j).astype(np.int32)
