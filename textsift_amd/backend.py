"""HipBackend — the reference's InferenceBackend contract on the gfx950 library.

Mirrors packages/textsift/src/browser/backends/abstract.ts:29-56:

    interface InferenceBackend {
      readonly name; warmup(): Promise<void>;
      forward(tokenIds: Int32Array, attentionMask: Uint8Array): Promise<Logits>;
      dispose(): void }
    Logits = { data: Float32Array /* T*33 row-major */, sequenceLength, numClasses }

and NodeBackend's behaviour (native/backend.ts:361-759): warmup is idempotent
(the base PrivacyFilter calls it twice, :408), uploads every weight once by
its NodeBackend name, and throws if the device or library is unavailable so
the caller's WASM fallback can take over (src/index.ts:69-103). forward
checks the mask length like WasmBackend (wasm.ts:735-741) and returns the
fp16-rounded logits widened to f32, as the WASM path does (wasm.ts:776-796).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _native
from .config import PF_CONFIG, ModelConfig


@dataclass
class Logits:
    data: np.ndarray          # float32 [sequence_length * num_classes], row-major
    sequence_length: int
    num_classes: int

    def as_matrix(self) -> np.ndarray:
        return self.data.reshape(self.sequence_length, self.num_classes)


class HipBackend:
    name = "native-hip"

    def __init__(self, weights: dict, config: ModelConfig = PF_CONFIG, device: int = 0,
                 precision: int = _native.PRECISION_FP16):
        """weights: NodeBackend-named tensors (see textsift_amd.synth) as numpy
        arrays holding the ONNX byte layouts. precision: PRECISION_FP16 (fp16
        GEMM inputs, the reference GPU paths' numerics) or PRECISION_SPLIT
        (f32 GEMM inputs carried as hi/lo fp16, the WASM path's numerics)."""
        self._weights = weights
        self._cfg = config
        self._device = device
        self._precision = int(precision)
        self._backend: _native.Backend | None = None
        self._model: _native.Model | None = None
        self.num_layers = max(int(k.split(".")[1]) for k in weights if k.startswith("layers.")) + 1
        self.num_experts = int(weights["layers.0.router.int4"].shape[0])
        self.vocab_size = int(weights["embed.int4"].shape[0])

    # InferenceBackend.warmup
    def warmup(self) -> None:
        if self._model is not None:
            return  # idempotent (native/backend.ts:408)
        be = _native.Backend(self._device)
        try:
            m = _native.Model(be, self._cfg, self.num_layers, self.num_experts, self.vocab_size, self._precision)
            try:
                for name, arr in self._weights.items():
                    m.set_weight(name, arr)
                m.finalize()
            except Exception:
                m.close()
                raise
        except Exception:
            be.close()
            raise
        self._backend, self._model = be, m

    # InferenceBackend.forward
    def forward(self, token_ids, attention_mask) -> Logits:
        if self._model is None:
            raise RuntimeError("HipBackend.forward: call warmup() first")
        ids = np.ascontiguousarray(token_ids, np.int32).ravel()
        mask = np.ascontiguousarray(attention_mask, np.uint8).ravel()
        if mask.size != ids.size:
            raise ValueError(f"HipBackend.forward: attentionMask length {mask.size} does not match "
                             f"tokenIds length {ids.size}")
        T = ids.size
        data = self._model.forward(ids, mask, 1, T)
        return Logits(data, T, self._cfg.num_classes)

    def forward_batch(self, token_ids, attention_mask=None) -> np.ndarray:
        """B independent sequences [B, T] in one launch set -> logits [B, T, C]."""
        ids = np.ascontiguousarray(token_ids, np.int32)
        if ids.ndim != 2:
            raise ValueError("forward_batch expects token ids of shape [B, T]")
        B, T = ids.shape
        mask = None if attention_mask is None else np.ascontiguousarray(attention_mask, np.uint8)
        if mask is not None and mask.shape != ids.shape:
            raise ValueError("forward_batch: attention mask shape must match token ids")
        data = self._model.forward(ids.ravel(), None if mask is None else mask.ravel(), B, T)
        return data.reshape(B, T, self._cfg.num_classes)

    @property
    def precision(self) -> int:
        return self._precision

    @property
    def model(self) -> _native.Model:
        return self._model

    @property
    def device(self) -> _native.Backend:
        return self._backend

    # InferenceBackend.dispose — safe to call more than once
    def dispose(self) -> None:
        if self._model is not None:
            self._model.close()
            self._model = None
        if self._backend is not None:
            self._backend.close()
            self._backend = None
