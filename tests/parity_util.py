"""Comparison helpers shared by the parity tests."""
import numpy as np


def f16(bits):
    """IEEE fp16 bits -> float64 (numpy's IEEE widen)."""
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def fp16_ulp_diff(actual_bits, expected_bits):
    """Per-element |a-e| in units of the expected value's fp16 ulp, with the
    ulp floored at the smallest normal's (tests/native/vulkan/conformance-all.js:125-131)."""
    a, e = f16(actual_bits), f16(expected_bits)
    mag = np.maximum(np.abs(e), 2.0 ** -14)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 10)
    return np.abs(a - e) / ulp


def rel_err_norm(actual, expected):
    """Normwise relative error ||a-e||_2 / ||e||_2."""
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    den = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (den if den > 0 else 1.0))


def rel_err_max(actual, expected):
    """max|a-e| / max|e|."""
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    den = np.max(np.abs(e))
    return float(np.max(np.abs(a - e)) / (den if den > 0 else 1.0))


def dequant_rows(int4, scales, zp, n_rows, k):
    """Closed-form MatMulNBits dequant in float64: (q - zp) * scale,
    low nibble first, zp nibble per 32-block (even block = low nibble)."""
    b = np.asarray(int4, np.uint8).reshape(n_rows, k // 2)
    q = np.empty((n_rows, k), np.int32)
    q[:, 0::2] = b & 0xF
    q[:, 1::2] = b >> 4
    nb = k // 32
    if zp is None:
        z = np.zeros((n_rows, nb), np.int32)
    else:
        zb = np.asarray(zp, np.uint8).reshape(n_rows, -1)
        z = np.empty((n_rows, zb.shape[1] * 2), np.int32)
        z[:, 0::2] = zb & 0xF
        z[:, 1::2] = zb >> 4
        z = z[:, :nb]
    s = f16(np.asarray(scales, np.uint16).reshape(n_rows, nb))
    return (q - np.repeat(z, 32, axis=1)).astype(np.float64) * np.repeat(s, 32, axis=1)


def fp16_ieee(x):
    """float -> fp16 bits with IEEE RNE, subnormals kept (for expected values)."""
    return np.asarray(x, np.float64).astype(np.float16).view(np.uint16)


class WordTokenizer:
    """Test tokenizer with the reference Tokenizer's encode() contract
    (browser/model/tokenizer.ts:240-305): word pieces carrying their leading
    space, as ByteLevel BPE does; token_to_char_offset has n + 1 entries (the
    last is the end of the last token). Ids are a stable hash of the piece
    modulo `vocab`."""

    def __init__(self, vocab=200064):
        import re
        self._re = re.compile(r"\s?\w+|\s?[^\w\s]+|\s+")
        self._vocab = vocab

    def encode(self, text):
        import types
        import zlib
        ms = list(self._re.finditer(text))
        return types.SimpleNamespace(
            token_ids=np.array([zlib.crc32(m.group().encode()) % self._vocab for m in ms], np.int32),
            attention_mask=np.ones(len(ms), np.uint8),
            token_to_char_offset=[m.start() for m in ms] + [ms[-1].end() if ms else 0],
            words=[m.group() for m in ms])

    def labels(self):
        from textsift_amd.spans import ALL_SPAN_LABELS
        return ALL_SPAN_LABELS


def random_words(n, seed):
    rng = np.random.default_rng(seed)
    vocab = ["alpha", "beta", "Gamma", "delta", "Eps", "zeta", "eta", ",", "theta", "Iota", "kappa", "Lambda",
             "mu@nu.io", "(617)", "555-0199", "42"]
    return " ".join(vocab[i] for i in rng.integers(0, len(vocab), n))


# A Viterbi operating point for the synthetic model, in the calibration
# artifact's JSON format (browser/model/calibration.ts:6-21). Staying in the
# background and continuing an entity are favoured, starting one is
# penalised, so decoded spans are runs of several tokens separated by
# background, as a tuned artifact's are; with the zero calibration nearly
# every token of a random-weight model is a single-token span.
SYNTH_OPERATING_POINT = {"operating_points": {"default": {"biases": {
    "transition_bias_background_stay": 2.0,
    "transition_bias_background_to_start": -1.0,
    "transition_bias_inside_to_continue": 1.0,
    "transition_bias_inside_to_end": 0.0,
    "transition_bias_end_to_background": 0.0,
    "transition_bias_end_to_start": -1.0}}}}


def transition_scores(cal):
    """[to, from] transition scores of the BIOES lattice under `cal`
    (viterbi.ts:159-219): legal moves get their calibration bias, illegal
    ones -inf; start scores 0 for O, B-*, S-*."""
    C, nl = 33, 8
    t = np.full((C, C), -np.inf)
    b = cal.biases().astype(np.float64)
    bg_stay, bg_start, in_cont, in_end, end_bg, end_start = b
    t[0, 0] = bg_stay
    tag = lambda l, k: 1 + 4 * l + k
    for l in range(nl):
        B, I, E, S = (tag(l, k) for k in range(4))
        t[B, 0] = t[S, 0] = bg_start
        t[I, B] = t[I, I] = in_cont
        t[E, B] = t[E, I] = in_end
        t[0, E] = t[0, S] = end_bg
        for l2 in range(nl):
            for src in (E, S):
                t[tag(l2, 0), src] = t[tag(l2, 3), src] = end_start
    start = np.full(C, -np.inf)
    start[0] = 0.0
    for l in range(nl):
        start[tag(l, 0)] = start[tag(l, 3)] = 0.0
    return t, start


def path_score(logits, path, cal):
    """Score of a tag path under the lattice: emissions plus transitions."""
    t, start = transition_scores(cal)
    p = np.asarray(path, np.int64)
    lg = np.asarray(logits, np.float64)
    return float(lg[np.arange(p.size), p].sum() + start[p[0]] + t[p[1:], p[:-1]].sum())


def span_parity(got, ref, chunk, labels=None, calibration=None):
    """Spans of two logit grids [T, 33] (Viterbi under `calibration`, the
    zero calibration by default, then BIOES -> spans over `chunk`), compared.

    Returns (identical, report). When the tag paths differ, `report` holds
    the evidence that the difference is a near-tie the logit error explains.
    A path's score is the sum of its logits plus its transition scores, and
    the transition part is the same function of the path for both grids, so
    for the GPU path p (optimal for `got`) and the oracle's q (optimal for
    `ref`), 0 <= S_ref(q) - S_ref(p) <= sum over tokens where the paths
    differ of |d[t, p_t] - d[t, q_t]|, d = got - ref. A decoder or logit bug
    that is not a near-tie breaks that bound."""
    from textsift_amd.spans import ALL_SPAN_LABELS, ViterbiDecoder, bioes_to_spans, zero_calibration
    labels = labels or ALL_SPAN_LABELS
    cal = calibration or zero_calibration()
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    dec = ViterbiDecoder(cal)
    p, q = dec.decode(got).astype(np.int64), dec.decode(ref).astype(np.int64)
    key = lambda s: (s.label, s.start, s.end)
    sg = [key(s) for s in bioes_to_spans(p, chunk, labels)]
    sr = [key(s) for s in bioes_to_spans(q, chunk, labels)]
    diff = np.nonzero(p != q)[0]
    g64, r64 = got.astype(np.float64), ref.astype(np.float64)
    gap = path_score(r64, q, cal) - path_score(r64, p, cal) if diff.size else 0.0
    d = g64 - r64
    bound = float(np.abs(d[diff, p[diff]] - d[diff, q[diff]]).sum())
    # spans away from the differing tokens must agree exactly
    offs = chunk.token_to_char_offset
    bad_chars = [(chunk.char_offset + offs[i], chunk.char_offset + offs[i + 1]) for i in diff]
    touches = lambda s: any(s[1] < e and b < s[2] for b, e in bad_chars)
    rest_equal = [s for s in sg if not touches(s)] == [s for s in sr if not touches(s)]
    multi = sum(1 for s in sr if s[2] - s[1] > (offs[1] - offs[0] if len(offs) > 1 else 1))
    report = {"n_spans": len(sr), "multi_token_spans": multi, "diff_tokens": int(diff.size), "gap": gap,
              "bound": bound, "rest_equal": rest_equal}
    return sg == sr, report


def logit_spread(logits):
    """(classes used by the argmax, largest class share) of a [T, C] grid."""
    am = np.argmax(np.asarray(logits), 1)
    cnt = np.bincount(am)
    return int(np.count_nonzero(cnt)), float(cnt.max() / am.size)


def near_tie_only(report, T, max_frac=0.01):
    """True if a span difference is a near-tie of the kind span_parity
    describes, on at most max_frac of the tokens."""
    return (report["rest_equal"] and report["diff_tokens"] <= max_frac * T
            and report["gap"] <= report["bound"] * (1 + 1e-6) + 1e-3)
