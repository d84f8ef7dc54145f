"""Model configuration (python/aios/models/config.py:8-60) and the named
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
    # Block-AttnRes trunk (models/config.py:24-60): "standard" residuals or
    # "block_attnres" depth routing over attnres_num_blocks blocks.
    residual_type: str = "standard"
    attnres_num_blocks: int = 0
    attnres_alpha: float = 1.0
    # The tokenizer's pad id (config.json "pad_token_id"); the CandidateGroup
    # engine fills its refill ban table with it when the group config names none.
    pad_token_id: int | None = None

    def __post_init__(self) -> None:
        if self.num_qo_heads % self.num_kv_heads:
            raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
        if self.hidden_act != "silu":
            raise ValueError(f"Unsupported activation: {self.hidden_act}")
        if self.residual_type not in {"standard", "block_attnres"}:
            raise ValueError("residual_type must be 'standard' or 'block_attnres'")
        if self.residual_type == "block_attnres":
            if self.attnres_num_blocks < 1:
                raise ValueError("block_attnres requires attnres_num_blocks >= 1")
            if self.num_layers % self.attnres_num_blocks:
                raise ValueError("num_layers must be divisible by attnres_num_blocks")
            if float(self.attnres_alpha) != 1.0:
                raise ValueError("only fully migrated Block AttnRes models with "
                                 "attnres_alpha=1.0 are served")

    @property
    def layers_per_attnres_block(self) -> int:
        if self.residual_type != "block_attnres":
            raise ValueError("standard residual models do not have AttnRes blocks")
        return self.num_layers // self.attnres_num_blocks

    def with_layers(self, n: int) -> "ModelConfig":
        if self.residual_type == "block_attnres":
            # keep the layers per block: n must be a multiple of them
            per = self.layers_per_attnres_block
            return replace(self, num_layers=n, attnres_num_blocks=max(1, n // per))
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

# 0.214B Block-AttnRes-shaped: 32 layers in 8 AttnRes blocks of 4, hidden
# 768, 8 query / 2 KV heads of 96, SwiGLU 2048, vocab 6400 (the MiniMind
# head_dim-96 shape with the depth-routed trunk; 65 depth mixers).
MINIMIND_ATTNRES_0P214B = ModelConfig(num_layers=32, num_qo_heads=8, num_kv_heads=2, head_dim=96,
                                      hidden_size=768, vocab_size=6400, intermediate_size=2048,
                                      rms_norm_eps=1e-5, model_type="minimind",
                                      residual_type="block_attnres", attnres_num_blocks=8)

MODELS = {
    "minimind-0.1b": MINIMIND_0P1B,
    "minimind-ime-0.1b": MINIMIND_IME_0P1B,
    "qwen3-0.6b": QWEN3_0P6B,
    "qwen3-4b": QWEN3_4B,
    "minimind-attnres-0.214b": MINIMIND_ATTNRES_0P214B,
}
