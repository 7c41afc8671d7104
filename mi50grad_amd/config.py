"""Model constants of the full-attention layers (Qwen3.5 family).

``AttnConfig`` carries the subset of ``QwenConfig`` (qwen.py:26-111) this path
reads, with the same attribute names, so the reference's own config object
can be passed wherever an ``AttnConfig`` is expected.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class AttnConfig:
    hidden_size: int = 5120
    num_hidden_layers: int = 64
    num_attention_heads: int = 24
    num_key_value_heads: int = 4
    head_dim: int = 256
    rope_theta: float = 10000000.0
    rms_norm_eps: float = 1e-6
    partial_rotary_factor: float = 0.25
    full_attention_interval: int = 4
    layer_types: list = field(default_factory=list)

    def __post_init__(self):
        # Default hybrid pattern: three linear-attention layers then one full
        # attention layer (qwen.py:66-74).
        if not self.layer_types:
            self.layer_types = ["full_attention" if (i + 1) % self.full_attention_interval == 0
                                else "linear_attention" for i in range(self.num_hidden_layers)]

    def is_full_attention(self, layer_idx: int) -> bool:
        return self.layer_types[layer_idx] == "full_attention"

    @property
    def num_full_attention_layers(self) -> int:
        return sum(1 for t in self.layer_types if t == "full_attention")

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    @property
    def kv_heads_per_group(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads
