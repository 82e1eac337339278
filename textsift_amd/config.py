"""Model constants of openai/privacy-filter as the reference bakes them in.

Mirrors ``PF_CONFIG`` (packages/textsift/src/browser/backends/wasm.ts:464-483)
and the NodeBackend copy (packages/textsift/src/native/backend.ts:392-404).
The vocabulary is the ONNX embed row count (200064), not the 200000
placeholder the reference's native benches use.
"""
from dataclasses import dataclass, field, asdict


@dataclass(frozen=True)
class RopeConfig:
    """YARN RoPE parameters (browser/inference/rope.ts:9-24)."""
    head_dim: int = 64
    theta: float = 150000.0
    factor: float = 32.0
    original_max_position_embeddings: int = 4096
    beta_fast: float = 32.0
    beta_slow: float = 1.0
    truncate: bool = False


@dataclass(frozen=True)
class ModelConfig:
    hidden_size: int = 640
    num_heads: int = 14
    num_kv_heads: int = 2
    head_dim: int = 64
    sliding_window: int = 128
    intermediate_size: int = 640
    num_experts: int = 128
    num_experts_per_tok: int = 4
    num_classes: int = 33
    vocab_size: int = 200064
    num_layers: int = 8
    rms_norm_eps: float = 1e-5
    rope: RopeConfig = field(default_factory=RopeConfig)

    def as_dict(self):
        return asdict(self)


PF_CONFIG = ModelConfig()

# Host-side chunking (browser/privacy-filter.ts:559, inference/chunking.ts:154)
CHUNK_TOKENS = 2048
CHUNK_OVERLAP = 128

# Quantization block along K for every MatMulNBits / GatherBlockQuantized
# tensor of the model (zig/wasm_exports.zig:575).
QBLOCK = 32
