"""Model configuration (python/aios/models/config.py:8-55) and the named
synthetic model shapes the attention backend is exercised with."""
from __future__ import annotations

from dataclasses import dataclass, replace


@dataclass(frozen=True)
class ModelConfig:
    num_layers: int
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    hidden_size: int
    vocab_size: int
    intermediate_size: int
    hidden_act: str = "silu"
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    max_position_embeddings: int = 32768
    tie_word_embeddings: bool = True
    model_type: str = "synthetic"

    def __post_init__(self) -> None:
        if self.num_qo_heads % self.num_kv_heads:
            raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
        if self.hidden_act != "silu":
            raise ValueError(f"Unsupported activation: {self.hidden_act}")

    def with_layers(self, n: int) -> "ModelConfig":
        return replace(self, num_layers=n)


# MiniMind-0.1B-shaped: 14 layers, hidden 768, 8 query / 2 KV heads of 96,
# SwiGLU 2048, vocab 6400 (the legacy MiniMind head_dim-96 shape).
MINIMIND_0P1B = ModelConfig(num_layers=14, num_qo_heads=8, num_kv_heads=2, head_dim=96,
                            hidden_size=768, vocab_size=6400, intermediate_size=2048,
                            rms_norm_eps=1e-5, rope_theta=1000000.0,
                            max_position_embeddings=32768, model_type="minimind")

# Deployed MiniMind-IME 0.1B shape (12 query / 4 KV heads of 64, vocab 16384).
MINIMIND_IME_0P1B = ModelConfig(num_layers=14, num_qo_heads=12, num_kv_heads=4, head_dim=64,
                                hidden_size=768, vocab_size=16384, intermediate_size=2048,
                                rms_norm_eps=1e-5, model_type="minimind")

# Qwen3-0.6B-shaped: 28 layers, hidden 1024, 16 query / 8 KV heads of 128.
QWEN3_0P6B = ModelConfig(num_layers=28, num_qo_heads=16, num_kv_heads=8, head_dim=128,
                         hidden_size=1024, vocab_size=151936, intermediate_size=3072,
                         model_type="qwen3")

# Qwen3-4B-shaped: 36 layers, hidden 2560, 32 query / 8 KV heads of 128.
QWEN3_4B = ModelConfig(num_layers=36, num_qo_heads=32, num_kv_heads=8, head_dim=128,
                       hidden_size=2560, vocab_size=151936, intermediate_size=9728,
                       model_type="qwen3")

MODELS = {
    "minimind-0.1b": MINIMIND_0P1B,
    "minimind-ime-0.1b": MINIMIND_IME_0P1B,
    "qwen3-0.6b": QWEN3_0P6B,
    "qwen3-4b": QWEN3_4B,
}
