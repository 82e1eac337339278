"""Host span pipeline (logits -> tags -> character spans), CPU only.

Pinned by:
  * the reference's PyTorch span fixtures (tests/conformance/pytorch/
    fixtures.json, copied to tests/golden/spans/): text, token offsets, the
    model's BIOES tags and the expected spans;
  * brute force over every tag sequence of tiny inputs (the Viterbi optimum
    and its legality under the BIOES transition rules);
  * an independent vectorized restatement (the fixture generator's
    viterbi_decode layout, generate-fixtures.py:150-172) on random inputs;
  * closed properties of chunking (every token emitted, chunk text equals
    the input slice) and of merging (a long input gives the spans of one
    pass over the whole input when every span lies inside one window).
"""
import itertools
import json
import os

import numpy as np
import pytest

from parity_util import WordTokenizer, random_words
from textsift_amd import spans as sp

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "spans", "pytorch_fixtures.json")
C = sp.NUM_BIOES_CLASSES
NEG = np.float32(-1e30)


def _tag_id(name):
    if name == "O":
        return 0
    prefix, _, label = name.partition("-")
    return sp.bioes_tag_of(sp.ALL_SPAN_LABELS.index(label), "BIES".index(prefix))


def _fixture_chunk(fx):
    offs = [o[0] for o in fx["offsets"]] + [fx["offsets"][-1][1]]
    n = len(fx["token_ids"])
    return sp.Chunk(np.asarray(fx["token_ids"], np.int32), np.ones(n, np.uint8), offs, fx["text"], 0, (0, n))


@pytest.fixture(scope="module")
def fixtures():
    with open(GOLDEN) as f:
        return json.load(f)


def test_bioes_to_spans_matches_reference_fixtures(fixtures):
    for fx in fixtures:
        tags = np.array([_tag_id(t) for t in fx["tags"]], np.uint8)
        got = [(s.label, s.start, s.end) for s in sp.bioes_to_spans(tags, _fixture_chunk(fx), sp.ALL_SPAN_LABELS)]
        want = [(s["label"], s["start"], s["end"]) for s in fx["spans"]]
        assert got == want, fx["text"]
        for s in sp.bioes_to_spans(tags, _fixture_chunk(fx), sp.ALL_SPAN_LABELS):
            assert s.text == fx["text"][s.start:s.end] and s.marker == f"[{s.label}]" and s.source == "model"


def test_viterbi_recovers_fixture_tags(fixtures):
    """One-hot emissions of a legal tag sequence decode to that sequence."""
    dec = sp.ViterbiDecoder(sp.zero_calibration())
    for fx in fixtures:
        want = np.array([_tag_id(t) for t in fx["tags"]], np.uint8)
        lg = np.full((want.size, C), -4.0, np.float32)
        lg[np.arange(want.size), want] = 4.0
        assert np.array_equal(dec.decode(lg), want), fx["text"]


def _tables(bias):
    """Transition/start tables from the BIOES rules as the fixture generator
    states them (generate-fixtures.py:104-145): trans[to, from]."""
    t = np.full((C, C), NEG, np.float32)
    t[0, 0] = bias[0]
    groups = [[sp.bioes_tag_of(l, b) for b in range(4)] for l in range(8)]
    for B, I, E, S in groups:
        t[B, 0] = t[S, 0] = bias[1]
        t[I, B] = bias[2]
        t[E, B] = bias[3]
        t[I, I] = bias[2]
        t[E, I] = bias[3]
        t[0, E] = t[0, S] = bias[4]
        for B2, _, _, S2 in groups:
            t[B2, E] = t[S2, E] = t[B2, S] = t[S2, S] = bias[5]
    start = np.full(C, NEG, np.float32)
    start[0] = 0
    for B, _, _, S in groups:
        start[B] = start[S] = 0
    return t, start


def _score(path, lg, trans, start):
    s = float(start[path[0]]) + float(lg[0, path[0]])
    for t in range(1, len(path)):
        s += float(trans[path[t], path[t - 1]]) + float(lg[t, path[t]])
    return s


def test_viterbi_is_the_brute_force_optimum():
    rng = np.random.default_rng(7)
    for T in (1, 2, 3):
        for trial in range(4):
            bias = rng.normal(0, 1, 6).astype(np.float32)
            lg = rng.normal(0, 2, (T, C)).astype(np.float32)
            trans, start = _tables(bias)
            cal = sp.ViterbiCalibration(*map(float, bias))
            got = sp.ViterbiDecoder(cal).decode(lg)
            best, best_path = -np.inf, None
            for path in itertools.product(range(C), repeat=T):
                s = _score(path, lg, trans, start)
                if s > best:
                    best, best_path = s, path
            assert best > -1e29  # a legal path exists
            assert abs(_score(got, lg, trans, start) - best) <= 1e-4 * max(1.0, abs(best)), (T, trial)
            assert tuple(got) == best_path, (T, trial)


def _viterbi_vectorized(lg, trans, start):
    T = lg.shape[0]
    alpha = start + lg[0]
    back = np.zeros((T, C), np.int64)
    for t in range(1, T):
        scores = alpha[None, :] + trans
        bf = scores.argmax(axis=1)
        alpha = scores[np.arange(C), bf] + lg[t]
        back[t] = bf
    tags = np.zeros(T, np.int64)
    tags[-1] = alpha.argmax()
    for t in range(T - 1, 0, -1):
        tags[t - 1] = back[t, tags[t]]
    return tags


def test_viterbi_matches_vectorized_restatement_and_batches():
    rng = np.random.default_rng(11)
    bias = rng.normal(0, 1, 6).astype(np.float32)
    trans, start = _tables(bias)
    dec = sp.ViterbiDecoder(sp.ViterbiCalibration(*map(float, bias)))
    lg = rng.normal(0, 3, (4, 257, C)).astype(np.float32)
    singles = [dec.decode(lg[b]) for b in range(4)]
    for b in range(4):
        assert np.array_equal(singles[b], _viterbi_vectorized(lg[b], trans, start))
    # batched, ragged lengths == per-sequence decode of each prefix
    lens = [257, 100, 1, 0]
    batch = dec.decode_batch(lg, lens)
    for b, n in enumerate(lens):
        assert np.array_equal(batch[b], dec.decode(lg[b], n) if n > 0 else np.zeros(0, np.uint8))


def test_viterbi_contract_errors():
    dec = sp.ViterbiDecoder(sp.zero_calibration())
    with pytest.raises(ValueError, match="expected 33 classes"):
        dec.decode(np.zeros((4, 32), np.float32))
    with pytest.raises(ValueError, match="exceeds"):
        dec.decode(np.zeros((4, C), np.float32), 5)
    assert dec.decode(np.zeros((4, C), np.float32), 0).size == 0
    with pytest.raises(ValueError, match="expected 8 labels"):
        sp.ViterbiDecoder(sp.zero_calibration(), ["a"] * 7)


def test_calibration_loader():
    good = {"operating_points": {"default": {"biases": {k: float(i) for i, k in enumerate(sp._BIAS_KEYS)}}}}
    cal = sp.load_calibration(good)
    assert list(cal.biases()) == [0, 1, 2, 3, 4, 5]
    bad = json.loads(json.dumps(good))
    del bad["operating_points"]["default"]["biases"]["transition_bias_end_to_start"]
    with pytest.raises(sp.PrivacyFilterError, match="missing required key") as e:
        sp.load_calibration(bad)
    assert e.value.code == "CALIBRATION_INVALID"
    bad = json.loads(json.dumps(good))
    bad["operating_points"]["default"]["biases"]["transition_bias_inside_to_end"] = "1"
    with pytest.raises(sp.PrivacyFilterError, match="must be a number; got string"):
        sp.load_calibration(bad)
    with pytest.raises(sp.PrivacyFilterError, match="expected object at operating_points, got array"):
        sp.load_calibration({"operating_points": []})


def test_malformed_runs_are_salvaged_like_the_reference():
    """spans.ts:44-101: I without B opens a run, E without B is a single-token
    span, a label change closes the open run, O closes an unterminated run."""
    text = "aa bb cc dd ee ff"
    offs = [0, 2, 5, 8, 11, 14, 17]
    chunk = sp.Chunk(np.zeros(6, np.int32), np.ones(6, np.uint8), offs, text, 100, (0, 6))
    P, E_ = sp.ALL_SPAN_LABELS.index("private_person"), sp.ALL_SPAN_LABELS.index("private_email")
    tags = np.array([sp.bioes_tag_of(P, 1), sp.bioes_tag_of(P, 1), sp.bioes_tag_of(E_, 2),
                     sp.bioes_tag_of(P, 0), 0, sp.bioes_tag_of(E_, 1)], np.uint8)
    got = [(s.label, s.start, s.end, s.text) for s in sp.bioes_to_spans(tags, chunk, sp.ALL_SPAN_LABELS)]
    assert got == [("private_person", 100, 105, "aa bb"), ("private_email", 106, 108, "cc"),
                   ("private_person", 109, 111, "dd"), ("private_email", 115, 117, "ff")]


def test_chunk_input_covers_the_text():
    tok = WordTokenizer()
    text = random_words(300, 3)
    full = tok.encode(text)
    chunks = sp.chunk_input(text, tok, 64, 16)
    assert len(chunks) > 4
    n = full.token_ids.size
    covered = np.zeros(n, bool)
    pos = 0
    for i, c in enumerate(chunks):
        assert c.text == text[c.char_offset:c.char_offset + len(c.text)]
        assert c.token_to_char_offset[0] == 0 and len(c.token_to_char_offset) == c.token_ids.size + 1
        lo, hi = c.emit_range
        assert lo == (0 if i == 0 else 8) and hi == (c.token_ids.size if i == len(chunks) - 1 else c.token_ids.size - 8)
        covered[pos:pos + c.token_ids.size] = True
        assert np.array_equal(c.token_ids, full.token_ids[pos:pos + c.token_ids.size])
        pos += 64 - 16
    assert covered.all()
    single = sp.chunk_input("just a few words", tok, 64)
    assert len(single) == 1 and single[0].emit_range == (0, single[0].token_ids.size)


class TagBackend:
    """CPU stand-in for HipBackend whose logits mark every capitalised word
    as a single-token person and every comma as a single-token secret."""

    def __init__(self, tok, text):
        self._words = {}
        self.calls = []
        self._tok = tok

    def _logits(self, ids, words):
        lg = np.full((len(ids), C), -5.0, np.float32)
        lg[:, 0] = 5.0
        for i, w in enumerate(words):
            w = w.strip()
            if w[:1].isupper():
                lg[i, sp.bioes_tag_of(sp.ALL_SPAN_LABELS.index("private_person"), 3)] = 9.0
            elif w == ",":
                lg[i, sp.bioes_tag_of(sp.ALL_SPAN_LABELS.index("secret"), 3)] = 9.0
        return lg

    def bind(self, text):
        enc = self._tok.encode(text)
        self._by_id_seq = (enc.token_ids, enc.words)

    def _words_for(self, ids):
        all_ids, words = self._by_id_seq
        for s in range(all_ids.size - ids.size + 1):
            if np.array_equal(all_ids[s:s + ids.size], ids):
                return words[s:s + ids.size]
        raise AssertionError("chunk not found")

    def forward(self, ids, mask):
        self.calls.append(("forward", ids.size))
        return self._logits(ids, self._words_for(ids))

    def forward_batch(self, ids, mask):
        self.calls.append(("forward_batch", ids.shape))
        return np.stack([self._logits(r, self._words_for(r)) for r in ids])


def test_detect_long_input_equals_one_pass():
    tok = WordTokenizer()
    text = random_words(700, 5)
    be = TagBackend(tok, text)
    be.bind(text)
    dec = sp.ViterbiDecoder(sp.zero_calibration())
    got = sp.detect(text, be, tok, dec, max_chunk_tokens=256)
    assert be.calls[0][0] == "forward_batch" and be.calls[0][1][0] >= 2
    one = sp.detect(text, be, tok, dec, max_chunk_tokens=10_000)
    key = lambda s: (s.start, s.end, s.label)
    assert [key(s) for s in got] == [key(s) for s in one]
    assert len(one) > 50
    assert all(text[s.start:s.end] == s.text for s in got)
    assert sp.detect(text, be, tok, dec, max_chunk_tokens=10_000, min_confidence=1.0) == one


def test_parity_util_lattice_matches_the_rules():
    """The lattice parity_util scores paths with (for the span near-tie bound)
    equals this file's tables, and the decoder's path is its optimum."""
    from parity_util import SYNTH_OPERATING_POINT, path_score, transition_scores
    rng = np.random.default_rng(5)
    for cal in (sp.zero_calibration(), sp.load_calibration(SYNTH_OPERATING_POINT),
                sp.ViterbiCalibration(*map(float, rng.normal(0, 1, 6)))):
        t, start = transition_scores(cal)
        t2, s2 = _tables(cal.biases())
        assert np.array_equal(np.where(np.isinf(t), NEG, t).astype(np.float32), t2)
        assert np.array_equal(np.where(np.isinf(start), NEG, start).astype(np.float32), s2)
        lg = rng.normal(0, 2, (64, C)).astype(np.float32)
        best = sp.ViterbiDecoder(cal).decode(lg)
        assert abs(path_score(lg, best, cal) - _score(best, lg, t2, s2)) < 1e-3
