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


@dataclass(frozen=True)
class Qwen35Config:
    """Qwen3.5 hybrid text model (mlx-lm qwen3_5 TextModelArgs field names;
    custom_qwen35_model.py:715-774). Layer i is full attention when
    (i + 1) % full_attention_interval == 0, GatedDeltaNet otherwise
    (custom_qwen35_model.py:896)."""
    hidden_size: int = 2560
    num_hidden_layers: int = 32
    intermediate_size: int = 9216
    num_attention_heads: int = 16
    num_key_value_heads: int = 4
    head_dim: int = 256
    partial_rotary_factor: float = 0.25
    linear_num_key_heads: int = 16
    linear_num_value_heads: int = 32
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_conv_kernel_dim: int = 4
    full_attention_interval: int = 4
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 100_000.0
    tie_word_embeddings: bool = True
    model_type: str = "qwen3_5"

    @property
    def rope_dims(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    @property
    def q_dim(self) -> int:
        return self.num_attention_heads * self.head_dim

    @property
    def attn_qkv_dim(self) -> int:
        """Fused q_proj ([q | gate] per head) + k_proj + v_proj rows."""
        return 2 * self.q_dim + 2 * self.num_key_value_heads * self.head_dim

    @property
    def key_dim(self) -> int:
        return self.linear_num_key_heads * self.linear_key_head_dim

    @property
    def value_dim(self) -> int:
        return self.linear_num_value_heads * self.linear_value_head_dim

    @property
    def conv_dim(self) -> int:
        return 2 * self.key_dim + self.value_dim

    @property
    def in_proj_dim(self) -> int:
        """Fused in_proj rows [qkv | z | b | a], zero-padded to a multiple of 64."""
        n = self.conv_dim + self.value_dim + 2 * self.linear_num_value_heads
        return (n + 63) // 64 * 64

    def is_linear(self, i: int) -> bool:
        return (i + 1) % self.full_attention_interval != 0

    @property
    def linear_layers(self) -> list[int]:
        return [i for i in range(self.num_hidden_layers) if self.is_linear(i)]

    @property
    def attention_layers(self) -> list[int]:
        return [i for i in range(self.num_hidden_layers) if not self.is_linear(i)]

    def validate(self) -> None:
        H, F = self.hidden_size, self.intermediate_size
        if self.head_dim != 256 or self.rope_dims != 64:
            raise NotImplementedError("the gated tree-attention kernel is compiled for head_dim 256, 64 rotary dims")
        if self.linear_key_head_dim != 128 or self.linear_value_head_dim != 128:
            raise NotImplementedError("the GatedDeltaNet kernels are compiled for 128-dim key and value heads")
        if H % 64 or F % 64 or self.q_dim % 64 or self.value_dim % 64:
            raise ValueError("hidden, intermediate, q and value dims must be multiples of 64")
        if self.vocab_size % 32:
            raise ValueError("vocab_size must be a multiple of 32")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        if self.linear_num_value_heads % self.linear_num_key_heads:
            raise ValueError("linear value heads must be a multiple of linear key heads")


# Qwen3.5-4B-shaped hybrid: 32 layers (24 GatedDeltaNet + 8 gated attention),
# hidden 2560, GatedDeltaNet 16 key / 32 value heads of 128, conv width 4.
# Attention 16 / 4 heads of 256 with 64 rotary dims, intermediate 9216,
# vocab 151936 (tied), rope theta 1e5 are this build's choices for the fields
# the workload leaves open.
QWEN35_4B = Qwen35Config()

# Qwen3.5-9B-shaped hybrid: hidden 4096 (same layer pattern and heads),
# intermediate 12288.
QWEN35_9B = Qwen35Config(hidden_size=4096, intermediate_size=12288)


def tiny_qwen35(**kw) -> Qwen35Config:
    """Small hybrid with the real head geometry (3 GatedDeltaNet + 1 attention
    layer), for parity tests."""
    base = Qwen35Config(hidden_size=512, num_hidden_layers=4, intermediate_size=1024, num_attention_heads=4,
                        num_key_value_heads=2, linear_num_key_heads=2, linear_num_value_heads=4, vocab_size=4096)
    return replace(base, **kw)
