"""Streaming-input detection on the HIP forward.

Restates the reference's `detect(AsyncIterable<string>)` driver
(packages/textsift/src/browser/inference/stream.ts:157-318, options
:700-752): on every incoming piece of text the trailing window of the
accumulated buffer (default 1024 tokens) goes through the model; spans that
end more than the safety margin (default 256 tokens, counted as 4
characters per token) behind the buffer's end are emitted, once each
(deduplicated by label, start, end); when the input ends, a chunked pass
over the whole buffer flushes the rest.

MI355X-specific addition: `StreamBatcher` serves many concurrent streams
and runs every pending trailing window of one step in a single batched
forward. Windows of different lengths are right-padded to the longest and
the padding is masked out; padded keys score -inf in attention and every
other stage is per token, so each window's logits equal those of its own
unpadded forward (checked bit-for-bit on the GPU by the tests).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Iterable, Iterator, Sequence

import numpy as np

from .spans import (ALL_SPAN_LABELS, Chunk, DetectedSpan, PrivacyFilterError, Tokenizer, ViterbiDecoder,
                    bioes_to_spans, chunk_input)

DEFAULT_WINDOW_TOKENS = 1024
DEFAULT_SAFETY_MARGIN_TOKENS = 256


def resolve_stream_options(window_tokens: int = DEFAULT_WINDOW_TOKENS,
                           safety_margin_tokens: int = DEFAULT_SAFETY_MARGIN_TOKENS) -> tuple[int, int]:
    """stream.ts:713-751."""
    if not (window_tokens > 0 and np.isfinite(window_tokens)):
        raise PrivacyFilterError(f"detect(stream): invalid windowTokens={window_tokens}; must be > 0", "INTERNAL")
    if not (safety_margin_tokens >= 0 and np.isfinite(safety_margin_tokens)):
        raise PrivacyFilterError(
            f"detect(stream): invalid safetyMarginTokens={safety_margin_tokens}; must be ≥ 0", "INTERNAL")
    if safety_margin_tokens >= window_tokens:
        raise PrivacyFilterError(f"detect(stream): safetyMarginTokens ({safety_margin_tokens}) must be < "
                                 f"windowTokens ({window_tokens})", "INTERNAL")
    return int(window_tokens), int(safety_margin_tokens)


def build_summary(spans: Sequence[DetectedSpan]) -> dict:
    out: dict = {}
    for s in spans:
        out[s.label] = out.get(s.label, 0) + 1
    return out


@dataclass
class DetectResult:
    input: str
    spans: list
    summary: dict
    contains_pii: bool


@dataclass
class _Window:
    chunk: Chunk
    safety_edge: int


@dataclass
class _StreamState:
    window_tokens: int
    margin_tokens: int
    enabled: frozenset | None
    buffer: str = ""
    emitted: set = field(default_factory=set)
    spans: list = field(default_factory=list)

    def should_emit(self, span: DetectedSpan) -> bool:
        if self.enabled is not None and span.source != "rule" and span.label not in self.enabled:
            return False
        key = (span.label, span.start, span.end)
        if key in self.emitted:
            return False
        self.emitted.add(key)
        return True


def _trailing_window(st: _StreamState, tokenizer: Tokenizer) -> _Window | None:
    """runWindow's tokenisation and window choice (stream.ts:221-254)."""
    if not st.buffer:
        return None
    enc = tokenizer.encode(st.buffer)
    ids = np.asarray(enc.token_ids, np.int32)
    total = ids.size
    if total == 0:
        return None
    start = max(0, total - st.window_tokens)
    n = total - start
    offs = list(enc.token_to_char_offset)
    first = offs[start] if start < len(offs) else 0
    local = [(offs[start + i] if start + i < len(offs) else len(st.buffer)) - first for i in range(n + 1)]
    chunk = Chunk(ids[start:], np.asarray(enc.attention_mask, np.uint8)[start:], local, st.buffer[first:], first,
                  (0, n))
    edge = max(0, len(st.buffer) - st.margin_tokens * 4)
    return _Window(chunk, edge)


def _emit_window(st: _StreamState, win: _Window, tags, labels) -> list:
    out = []
    for span in bioes_to_spans(tags, win.chunk, labels):
        if span.end > win.safety_edge:
            continue
        if st.should_emit(span):
            st.spans.append(span)
            out.append(span)
    return out


def _forward_windows(backend, chunks: Sequence[Chunk]) -> list:
    """Logits [n_i, C] of each chunk; all of them in one batched forward when
    the backend has one (right-padded to the longest, padding masked)."""
    # padded windows are exact in the fp16 numerics (masked keys add exact
    # zeros to the softmax); the split numerics pick the WASM path's exp per
    # key position within the window, which padding would shift
    split = getattr(backend, "precision", None) == 1
    if len(chunks) == 1 or split or not hasattr(backend, "forward_batch"):
        return [_as_matrix(backend.forward(c.token_ids, c.attention_mask), c.token_ids.size) for c in chunks]
    T = max(c.token_ids.size for c in chunks)
    ids = np.zeros((len(chunks), T), np.int32)
    mask = np.zeros((len(chunks), T), np.uint8)
    for i, c in enumerate(chunks):
        n = c.token_ids.size
        ids[i, :n] = c.token_ids
        mask[i, :n] = c.attention_mask
    lg = backend.forward_batch(ids, mask)
    return [np.asarray(lg[i, :c.token_ids.size]) for i, c in enumerate(chunks)]


def _as_matrix(logits, n):
    if hasattr(logits, "as_matrix"):
        return logits.as_matrix()
    return np.asarray(logits).reshape(n, -1)


class DetectStream:
    """`detect(stream)` for one stream: iterate to receive spans as they
    become stable; `result` holds the DetectResult once the input ended."""

    def __init__(self, pieces: Iterable[str], backend, tokenizer: Tokenizer, decoder: ViterbiDecoder,
                 window_tokens: int = DEFAULT_WINDOW_TOKENS, safety_margin_tokens: int = DEFAULT_SAFETY_MARGIN_TOKENS,
                 enabled_categories: Sequence[str] | None = None):
        w, m = resolve_stream_options(window_tokens, safety_margin_tokens)
        self._batcher = StreamBatcher(backend, tokenizer, decoder, w, m, enabled_categories)
        self._pieces = pieces
        self.result: DetectResult | None = None

    def __iter__(self) -> Iterator[DetectedSpan]:
        b = self._batcher
        sid = b.open()
        for piece in self._pieces:
            if not piece:
                continue
            b.feed(sid, piece)
            yield from b.step().get(sid, [])
        yield from b.finish(sid)
        self.result = b.result(sid)


class StreamBatcher:
    """Many concurrent streams, one forward per step for all their windows."""

    def __init__(self, backend, tokenizer: Tokenizer, decoder: ViterbiDecoder,
                 window_tokens: int = DEFAULT_WINDOW_TOKENS, safety_margin_tokens: int = DEFAULT_SAFETY_MARGIN_TOKENS,
                 enabled_categories: Sequence[str] | None = None):
        self.window_tokens, self.margin_tokens = resolve_stream_options(window_tokens, safety_margin_tokens)
        self.backend, self.tokenizer, self.decoder = backend, tokenizer, decoder
        self.labels = list(tokenizer.labels())
        en = None if enabled_categories is None or len(enabled_categories) == len(ALL_SPAN_LABELS) else frozenset(
            enabled_categories)
        self._enabled = en
        self._streams: dict = {}
        self._pending: set = set()
        self._next = 0
        self.forward_calls = 0

    def open(self) -> int:
        sid = self._next
        self._next += 1
        self._streams[sid] = _StreamState(self.window_tokens, self.margin_tokens, self._enabled)
        return sid

    def feed(self, sid: int, text: str):
        """Append a piece of text; its window runs at the next step()."""
        if text:
            self._streams[sid].buffer += text
            self._pending.add(sid)

    def step(self) -> dict:
        """Runs the trailing window of every stream fed since the last step
        in one forward; returns {stream id: newly stable spans}."""
        sids = sorted(self._pending)
        self._pending.clear()
        wins = [(sid, _trailing_window(self._streams[sid], self.tokenizer)) for sid in sids]
        wins = [(sid, w) for sid, w in wins if w is not None]
        if not wins:
            return {}
        logits = _forward_windows(self.backend, [w.chunk for _, w in wins])
        self.forward_calls += 1
        tags = self.decoder.decode_batch(_stack(logits), [w.chunk.token_ids.size for _, w in wins])
        return {sid: _emit_window(self._streams[sid], w, t, self.labels) for (sid, w), t in zip(wins, tags)}

    def finish(self, sid: int) -> list:
        """Input ended: the chunked pass over the whole buffer (stream.ts:277-305)."""
        st = self._streams[sid]
        self._pending.discard(sid)
        out = []
        if st.buffer:
            chunks = chunk_input(st.buffer, self.tokenizer, max(self.window_tokens, 2048))
            chunks = [c for c in chunks if c.token_ids.size > 0]
            if chunks:
                logits = _forward_windows(self.backend, chunks)
                self.forward_calls += 1
                tags = self.decoder.decode_batch(_stack(logits), [c.token_ids.size for c in chunks])
                for c, t in zip(chunks, tags):
                    for span in bioes_to_spans(t, c, self.labels):
                        if st.should_emit(span):
                            st.spans.append(span)
                            out.append(span)
        return out

    def result(self, sid: int) -> DetectResult:
        st = self._streams[sid]
        return DetectResult(st.buffer, list(st.spans), build_summary(st.spans), len(st.spans) > 0)

    def close(self, sid: int):
        self._streams.pop(sid, None)
        self._pending.discard(sid)


def _stack(logits: list) -> np.ndarray:
    T = max(l.shape[0] for l in logits)
    out = np.zeros((len(logits), T, logits[0].shape[1]), np.float32)
    for i, l in enumerate(logits):
        out[i, :l.shape[0]] = l
    return out
