"""Target model configurations (field names follow mlx-lm's qwen3 ModelArgs)."""
from __future__ import annotations

from dataclasses import dataclass, replace


@dataclass(frozen=True)
class Qwen3Config:
    hidden_size: int = 2560
    num_hidden_layers: int = 36
    intermediate_size: int = 9728
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    tie_word_embeddings: bool = True
    model_type: str = "qwen3"

    @property
    def q_dim(self) -> int:
        return self.num_attention_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_key_value_heads * self.head_dim

    @property
    def qkv_dim(self) -> int:
        return self.q_dim + 2 * self.kv_dim

    def layer_linear_params(self) -> int:
        H, F = self.hidden_size, self.intermediate_size
        return self.qkv_dim * H + H * self.q_dim + 2 * F * H + H * F

    def validate(self) -> None:
        H, F = self.hidden_size, self.intermediate_size
        if self.head_dim != 128:
            raise NotImplementedError("the tree-attention kernel is compiled for head_dim 128")
        if H % 64 or F % 64 or self.q_dim % 64:
            raise ValueError("hidden, intermediate and q dims must be multiples of 64")
        if self.vocab_size % 32:
            raise ValueError("vocab_size must be a multiple of 32")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")


# Qwen3-4B (mlx-community/Qwen3-4B-bf16 architecture, random-init here).
QWEN3_4B = Qwen3Config()


def tiny_qwen3(**kw) -> Qwen3Config:
    """Small Qwen3-shaped config with the real head geometry, for parity tests."""
    base = Qwen3Config(hidden_size=1024, num_hidden_layers=2, intermediate_size=2048,
                       num_attention_heads=8, num_key_value_heads=2, vocab_size=4096)
    return replace(base, **kw)
