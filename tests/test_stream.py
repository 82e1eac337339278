"""Streaming detection (CPU, with a context-free stand-in backend).

With logits that depend only on each token, the spans of a token sequence
do not depend on how it is windowed, so streaming must end with exactly the
spans of one pass over the whole input, emit each span once, and emit a span
during streaming only once it ends behind the safety edge. The batcher must
give every stream the same spans as running it alone, in one forward per
step (windows padded to the longest and masked).
"""
import numpy as np
import pytest

from parity_util import WordTokenizer, random_words
from textsift_amd import spans as sp
from textsift_amd import stream as st

VOCAB = 4096
C = sp.NUM_BIOES_CLASSES


class IdBackend:
    """Logits a function of the token id alone: capitalised pieces are a
    single-token person, commas a single-token secret, the rest background."""

    def __init__(self, tok):
        self.tag = {}
        for word in ["alpha", "beta", "Gamma", "delta", "Eps", "zeta", "eta", ",", "theta", "Iota", "kappa",
                     "Lambda", "mu", "@", "nu", ".", "io", "(", "617", ")", "555", "-", "0199", "42"]:
            for piece in (word, " " + word):
                i = int(tok.encode(piece).token_ids[0])
                if word[:1].isupper():
                    self.tag[i] = sp.bioes_tag_of(sp.ALL_SPAN_LABELS.index("private_person"), 3)
                elif word == ",":
                    self.tag[i] = sp.bioes_tag_of(sp.ALL_SPAN_LABELS.index("secret"), 3)
        self.calls = []

    def _logits(self, ids):
        lg = np.full((ids.size, C), -5.0, np.float32)
        lg[:, 0] = 5.0
        for t, i in enumerate(ids):
            if int(i) in self.tag:
                lg[t, self.tag[int(i)]] = 9.0
        return lg

    def forward(self, ids, mask):
        self.calls.append(("forward", ids.size))
        return self._logits(np.asarray(ids))

    def forward_batch(self, ids, mask):
        self.calls.append(("forward_batch", ids.shape))
        out = np.stack([self._logits(r) for r in ids])
        out[np.asarray(mask) == 0] = np.nan  # padding must never be read
        return out


def _pieces(text, seed):
    rng = np.random.default_rng(seed)
    out, i = [], 0
    while i < len(text):
        n = int(rng.integers(1, 200))
        out.append(text[i:i + n])
        i += n
    return out


@pytest.fixture(scope="module")
def env():
    tok = WordTokenizer(VOCAB)
    return tok, IdBackend(tok), sp.ViterbiDecoder(sp.zero_calibration())


def key(s):
    return (s.label, s.start, s.end)


def test_stream_equals_one_pass_and_emits_once(env):
    tok, be, dec = env
    text = random_words(1500, 9)
    ds = st.DetectStream(_pieces(text, 1), be, tok, dec, window_tokens=256, safety_margin_tokens=64)
    got = list(ds)
    one = sp.detect(text, be, tok, dec, max_chunk_tokens=100000)
    assert sorted(map(key, got)) == sorted(map(key, one)) and len(one) > 100
    assert len(set(map(key, got))) == len(got)
    assert ds.result.spans == got and ds.result.input == text and ds.result.contains_pii
    assert sum(ds.result.summary.values()) == len(got)


def test_spans_wait_for_the_safety_edge(env):
    tok, be, dec = env
    text = random_words(600, 10)
    b = st.StreamBatcher(be, tok, dec, window_tokens=128, safety_margin_tokens=32)
    sid = b.open()
    buf = ""
    for piece in _pieces(text, 2):
        buf += piece
        b.feed(sid, piece)
        for s in b.step().get(sid, []):
            assert s.end <= max(0, len(buf) - 32 * 4)
    b.finish(sid)


def test_batcher_matches_streams_run_alone(env):
    tok, be, dec = env
    texts = [random_words(n, 20 + n) for n in (300, 700, 50, 1000, 5)]
    alone = [list(st.DetectStream(_pieces(t, i), be, tok, dec, 512, 128)) for i, t in enumerate(texts)]
    b = st.StreamBatcher(be, tok, dec, 512, 128)
    sids = [b.open() for _ in texts]
    queues = [_pieces(t, i) for i, t in enumerate(texts)]
    got = {sid: [] for sid in sids}
    steps = 0
    while any(queues):
        for sid, q in zip(sids, queues):
            if q:
                b.feed(sid, q.pop(0))
        calls = b.forward_calls
        for sid, spans in b.step().items():
            got[sid] += spans
        assert b.forward_calls == calls + 1  # one forward for every stream's window
        steps += 1
    for sid in sids:
        got[sid] += b.finish(sid)
    for sid, ref in zip(sids, alone):
        assert list(map(key, got[sid])) == list(map(key, ref))


def test_enabled_categories_and_options(env):
    tok, be, dec = env
    text = random_words(400, 11)
    only = list(st.DetectStream(_pieces(text, 3), be, tok, dec, 256, 64, enabled_categories=["secret"]))
    assert only and all(s.label == "secret" for s in only)
    with pytest.raises(sp.PrivacyFilterError, match="must be < windowTokens"):
        st.StreamBatcher(be, tok, dec, 64, 64)
    with pytest.raises(sp.PrivacyFilterError, match="invalid windowTokens"):
        st.resolve_stream_options(0, 0)
    with pytest.raises(sp.PrivacyFilterError, match="invalid safetyMarginTokens"):
        st.resolve_stream_options(10, -1)
