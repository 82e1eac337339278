"""Logits -> character spans: the host side of detection on the HIP forward.

Mirrors the reference's pipeline after InferenceBackend.forward
(packages/textsift/src/browser/privacy-filter.ts:488-521, runDetection):

  chunk_input          browser/inference/chunking.ts:55-123   (chunkInput)
  HipBackend.forward / forward_batch                            (the GPU path)
  ViterbiDecoder       browser/inference/viterbi.ts:51-146     (decode; the
                       lattice runs natively, pfhip_viterbi_decode)
  bioes_to_spans       browser/inference/spans.ts:23-140       (bioesToSpans)
  merge_chunk_results  browser/inference/chunking.ts:134-152   (mergeChunkResults)
  load_calibration     browser/model/calibration.ts:45-84

Names, argument meaning and errors follow the reference. One deliberate
difference: `detect` hands every full-length chunk of a long input to the
backend in one forward_batch call (the chunks are independent sequences)
instead of one forward per chunk; the per-chunk logits, tags and spans are
the same. Character offsets index Python strings (code points); the
reference indexes JS strings (UTF-16 code units). They agree on text
without characters outside the Basic Multilingual Plane.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol, Sequence

import numpy as np

from . import _native

# browser/types.ts:24-45
ALL_SPAN_LABELS: tuple[str, ...] = (
    "account_number",
    "private_address",
    "private_email",
    "private_person",
    "private_phone",
    "private_url",
    "private_date",
    "secret",
)

# browser/inference/viterbi.ts:29-38
BIOES_BACKGROUND = 0
FIRST_SPAN_CLASS = 1
NUM_BOUNDARY_TAGS = 4
NUM_BIOES_CLASSES = 33
NUM_SPAN_LABELS = 8

DEFAULT_OVERLAP_TOKENS = 128     # chunking.ts:154
DEFAULT_MAX_CHUNK_TOKENS = 2048  # privacy-filter.ts:559


class PrivacyFilterError(Exception):
    """browser/types.ts PrivacyFilterError: a message plus a machine-readable code."""

    def __init__(self, message: str, code: str):
        super().__init__(message)
        self.code = code


# ---------------------------------------------------------------- calibration

@dataclass(frozen=True)
class ViterbiCalibration:
    background_stay: float
    background_to_start: float
    inside_to_continue: float
    inside_to_end: float
    end_to_background: float
    end_to_start: float

    def biases(self) -> np.ndarray:
        return np.array([self.background_stay, self.background_to_start, self.inside_to_continue,
                         self.inside_to_end, self.end_to_background, self.end_to_start], np.float32)


_BIAS_KEYS = (
    "transition_bias_background_stay",
    "transition_bias_background_to_start",
    "transition_bias_inside_to_continue",
    "transition_bias_inside_to_end",
    "transition_bias_end_to_background",
    "transition_bias_end_to_start",
)


def _describe(v) -> str:
    if v is None:
        return "null"
    if isinstance(v, list):
        return "array"
    if isinstance(v, bool):
        return "boolean"
    if isinstance(v, (int, float)):
        return "number"
    if isinstance(v, str):
        return "string"
    return "object" if isinstance(v, dict) else type(v).__name__


def _as_object(v, where: str) -> dict:
    if not isinstance(v, dict):
        raise PrivacyFilterError(f"calibration artifact: expected object at {where}, got {_describe(v)}",
                                 "CALIBRATION_INVALID")
    return v


def load_calibration(obj) -> ViterbiCalibration:
    """Parses the calibration JSON (already decoded) — calibration.ts:45-73."""
    env = _as_object(obj, "calibration JSON")
    ops = _as_object(env.get("operating_points"), "operating_points")
    default = _as_object(ops.get("default"), "operating_points.default")
    biases = _as_object(default.get("biases"), "operating_points.default.biases")
    for k in _BIAS_KEYS:
        if k not in biases:
            raise PrivacyFilterError(f"calibration artifact missing required key: {k}", "CALIBRATION_INVALID")
        v = biases[k]
        if isinstance(v, bool) or not isinstance(v, (int, float)):
            raise PrivacyFilterError(f"calibration artifact value for {k} must be a number; got {_describe(v)}",
                                     "CALIBRATION_INVALID")
    return ViterbiCalibration(*(float(biases[k]) for k in _BIAS_KEYS))


def zero_calibration() -> ViterbiCalibration:
    """calibration.ts:76-85."""
    return ViterbiCalibration(0.0, 0.0, 0.0, 0.0, 0.0, 0.0)


# ---------------------------------------------------------------- Viterbi

def bioes_tag_of(label_index: int, boundary: int) -> int:
    """viterbi.ts:47-49; boundary 0..3 = B, I, E, S."""
    return FIRST_SPAN_CLASS + label_index * NUM_BOUNDARY_TAGS + boundary


def describe_tag(tag: int) -> tuple[str, int]:
    """(prefix, label index) of a tag id; label index -1 for O (viterbi.ts:221-231)."""
    if tag == BIOES_BACKGROUND:
        return "O", -1
    off = tag - FIRST_SPAN_CLASS
    return "BIES"[off % NUM_BOUNDARY_TAGS], off // NUM_BOUNDARY_TAGS


class ViterbiDecoder:
    """viterbi.ts:51-146. The lattice is evaluated natively."""

    def __init__(self, calibration: ViterbiCalibration, label_set: Sequence[str] = ALL_SPAN_LABELS):
        if len(label_set) != NUM_SPAN_LABELS:
            raise ValueError(f"ViterbiDecoder: expected {NUM_SPAN_LABELS} labels, got {len(label_set)}")
        self._labels = tuple(label_set)
        self._biases = calibration.biases()

    def get_label_set(self) -> tuple[str, ...]:
        return self._labels

    def decode(self, logits, sequence_length: int | None = None) -> np.ndarray:
        """Tags (u8 [T]) of one sequence. `logits`: a Logits (data,
        sequence_length, num_classes) or an f32 [T, C] array."""
        data, T_full, C = _logit_grid(logits)
        if C != NUM_BIOES_CLASSES:
            raise ValueError(f"ViterbiDecoder: expected {NUM_BIOES_CLASSES} classes, got {C}")
        T = T_full if sequence_length is None else int(sequence_length)
        if T <= 0:
            return np.zeros(0, np.uint8)
        if T > T_full:
            raise ValueError(f"ViterbiDecoder: sequenceLength {T} exceeds logits.sequenceLength {T_full}")
        return _native.viterbi_decode(data.reshape(T_full, C), self._biases, [T])[:T]

    def decode_batch(self, logits: np.ndarray, sequence_lengths=None) -> list[np.ndarray]:
        """decode() of every sequence of f32 [B, T, C] logits, on host threads."""
        lg = np.asarray(logits, np.float32)
        if lg.ndim != 3 or lg.shape[2] != NUM_BIOES_CLASSES:
            raise ValueError(f"ViterbiDecoder: expected [B, T, {NUM_BIOES_CLASSES}] logits")
        B, T, _ = lg.shape
        lens = [T] * B if sequence_lengths is None else [int(n) for n in sequence_lengths]
        for n in lens:
            if n > T:
                raise ValueError(f"ViterbiDecoder: sequenceLength {n} exceeds logits.sequenceLength {T}")
        tags = _native.viterbi_decode(lg, self._biases, [max(n, 0) for n in lens])
        return [tags[b, :max(lens[b], 0)] for b in range(B)]


def _logit_grid(logits):
    if hasattr(logits, "sequence_length"):
        return np.asarray(logits.data, np.float32), int(logits.sequence_length), int(logits.num_classes)
    a = np.asarray(logits, np.float32)
    if a.ndim != 2:
        raise ValueError("ViterbiDecoder: logits must be [T, C]")
    return a, a.shape[0], a.shape[1]


# ---------------------------------------------------------------- chunks and spans

@dataclass
class Chunk:
    """chunking.ts:30-53."""
    token_ids: np.ndarray                 # int32 [n]
    attention_mask: np.ndarray            # uint8 [n]
    token_to_char_offset: list[int]       # n + 1 entries (sentinel last), relative to `text`
    text: str
    char_offset: int
    emit_range: tuple[int, int]


@dataclass
class DetectedSpan:
    """browser/types.ts DetectedSpan (model spans)."""
    label: str
    start: int
    end: int
    text: str
    source: str = "model"
    marker: str = ""
    confidence: float = 1.0

    def __post_init__(self):
        if not self.marker:
            self.marker = f"[{self.label}]"


class EncodeResult(Protocol):
    token_ids: np.ndarray
    attention_mask: np.ndarray
    token_to_char_offset: Sequence[int]


class Tokenizer(Protocol):
    def encode(self, text: str) -> EncodeResult: ...

    def labels(self) -> Sequence[str]: ...


_WS = frozenset((0x20, 0x09, 0x0A, 0x0B, 0x0C, 0x0D, 0xA0))  # spans.ts:143-154


def bioes_to_spans(tags, chunk: Chunk, labels: Sequence[str]) -> list[DetectedSpan]:
    """spans.ts:23-140: runs of B/I/E and single S tags -> character spans,
    salvaging malformed runs the way the reference does, trimmed of
    whitespace at both ends."""
    if len(labels) != NUM_SPAN_LABELS:
        raise ValueError(f"bioesToSpans: tokenizer reports {len(labels)} labels, expected {NUM_SPAN_LABELS}")
    spans: list[DetectedSpan] = []
    offs = chunk.token_to_char_offset
    text = chunk.text

    def emit(s_tok: int, e_tok: int, lbl: int):
        if not 0 <= s_tok < len(offs):
            return
        raw_end = offs[e_tok + 1] if 0 <= e_tok + 1 < len(offs) else (offs[e_tok] if 0 <= e_tok < len(offs) else None)
        if raw_end is None:
            return
        if not 0 <= lbl < len(labels):
            return
        s, e = offs[s_tok], raw_end
        while s < e and s < len(text) and ord(text[s]) in _WS:
            s += 1
        while e > s and e <= len(text) and ord(text[e - 1]) in _WS:
            e -= 1
        if e <= s:
            return
        spans.append(DetectedSpan(label=labels[lbl], start=chunk.char_offset + s, end=chunk.char_offset + e,
                                  text=text[s:e]))

    open_run: tuple[int, int] | None = None  # (label, start token)
    T = len(tags)
    for t in range(T):
        prefix, lbl = describe_tag(int(tags[t]))
        if prefix == "O":
            if open_run is not None:
                emit(open_run[1], t - 1, open_run[0])
                open_run = None
        elif prefix == "S":
            if open_run is not None:
                emit(open_run[1], t - 1, open_run[0])
                open_run = None
            emit(t, t, lbl)
        elif prefix == "E":
            if open_run is not None and open_run[0] == lbl:
                emit(open_run[1], t, lbl)
                open_run = None
            else:
                if open_run is not None:
                    emit(open_run[1], t - 1, open_run[0])
                    open_run = None
                emit(t, t, lbl)
        elif prefix == "I":
            if open_run is None or open_run[0] != lbl:
                if open_run is not None:
                    emit(open_run[1], t - 1, open_run[0])
                open_run = (lbl, t)
        else:  # B
            if open_run is not None:
                emit(open_run[1], t - 1, open_run[0])
            open_run = (lbl, t)
    if open_run is not None:
        emit(open_run[1], T - 1, open_run[0])
    return spans


def chunk_input(text: str, tokenizer: Tokenizer, max_chunk_tokens: int,
                overlap_tokens: int = DEFAULT_OVERLAP_TOKENS) -> list[Chunk]:
    """chunking.ts:55-123: overlapping windows of max_chunk_tokens tokens."""
    full = tokenizer.encode(text)
    ids = np.asarray(full.token_ids, np.int32)
    mask = np.asarray(full.attention_mask, np.uint8)
    offs = list(full.token_to_char_offset)
    n = ids.size
    if n <= max_chunk_tokens:
        return [Chunk(ids, mask, offs, text, 0, (0, n))]
    step = max_chunk_tokens - overlap_tokens
    if step <= 0:
        raise ValueError("chunk_input: maxChunkTokens must exceed overlapTokens")
    chunks: list[Chunk] = []
    start = 0
    while start < n:
        end = min(start + max_chunk_tokens, n)
        abs_start = offs[start]
        abs_end = offs[end] if end < len(offs) else offs[end - 1] + (len(text) - offs[end - 1])
        rel = [(offs[i] if i < len(offs) else abs_end) - abs_start for i in range(start, end + 1)]
        first, last = start == 0, end >= n
        emit_from = 0 if first else overlap_tokens // 2
        emit_to = (end - start) if last else (end - start) - (overlap_tokens + 1) // 2
        chunks.append(Chunk(ids[start:end], mask[start:end], rel, text[abs_start:abs_end], abs_start,
                            (emit_from, emit_to)))
        if last:
            break
        start += step
    return chunks


def merge_chunk_results(per_chunk_spans: Sequence[Sequence[DetectedSpan]],
                        chunks: Sequence[Chunk]) -> list[DetectedSpan]:
    """chunking.ts:134-152: de-duplicate by (start, end, label), then a
    stable sort by start."""
    out: list[DetectedSpan] = []
    seen: set[tuple[int, int, str]] = set()
    for c in range(len(chunks)):
        for s in per_chunk_spans[c]:
            key = (s.start, s.end, s.label)
            if key in seen:
                continue
            seen.add(key)
            out.append(s)
    out.sort(key=lambda s: s.start)
    return out


def detect(text: str, backend, tokenizer: Tokenizer, decoder: ViterbiDecoder,
           max_chunk_tokens: int = DEFAULT_MAX_CHUNK_TOKENS, min_confidence: float = 0.0) -> list[DetectedSpan]:
    """runDetection (privacy-filter.ts:488-521) without the rule engine:
    chunk, forward, Viterbi, spans, merge, confidence filter. Chunks of the
    full window length go to the backend together (forward_batch)."""
    chunks = chunk_input(text, tokenizer, max_chunk_tokens)
    labels = list(tokenizer.labels())
    tags: list[np.ndarray | None] = [None] * len(chunks)
    full = [i for i, c in enumerate(chunks) if c.token_ids.size == max_chunk_tokens and c.token_ids.size > 0]
    if len(full) > 1 and hasattr(backend, "forward_batch"):
        ids = np.stack([chunks[i].token_ids for i in full])
        mask = np.stack([chunks[i].attention_mask for i in full])
        logits = backend.forward_batch(ids, mask)
        for i, t in zip(full, decoder.decode_batch(logits)):
            tags[i] = t
    for i, c in enumerate(chunks):
        if tags[i] is None:
            if c.token_ids.size == 0:
                tags[i] = np.zeros(0, np.uint8)
                continue
            logits = backend.forward(c.token_ids, c.attention_mask)
            tags[i] = decoder.decode(logits, c.token_ids.size)
    per_chunk = [bioes_to_spans(tags[i], c, labels) for i, c in enumerate(chunks)]
    spans = merge_chunk_results(per_chunk, chunks)
    if min_confidence <= 0:
        return spans
    return [s for s in spans if s.confidence >= min_confidence]
