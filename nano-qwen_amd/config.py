"""Attention fields of nano-qwen's ModelConfig (model/config.py:14-83).

``Attention`` only reads these attributes, so the reference's own
``ModelConfig`` instances work unchanged; this dataclass is for users who do
not carry the rest of the model configuration.  ``from_yaml`` reads the
reference's configs/model/*.yaml files and keeps the attention fields.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from typing import Optional

import yaml


@dataclass
class AttentionConfig:
    hidden_size: int = 4096
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: Optional[int] = None
    max_position_embeddings: int = 32768
    rms_norm_eps: float = 1e-6
    attention_bias: bool = False
    attention_dropout: float = 0.0
    qk_norm: bool = True
    rope_theta: float = 1_000_000.0
    rope_scaling: Optional[dict] = None

    def __post_init__(self):
        # model/config.py:73-75
        if self.head_dim is None:
            self.head_dim = self.hidden_size // self.num_attention_heads

    @property
    def num_kv_groups(self) -> int:
        # model/config.py:81-83
        return self.num_attention_heads // self.num_key_value_heads

    @classmethod
    def from_dict(cls, data: dict) -> "AttentionConfig":
        names = {f.name for f in fields(cls)}
        return cls(**{k: v for k, v in data.items() if k in names})

    @classmethod
    def from_yaml(cls, path) -> "AttentionConfig":
        with open(path) as f:
            return cls.from_dict(yaml.safe_load(f))


def num_kv_groups(config) -> int:
    g = getattr(config, "num_kv_groups", None)
    return int(g) if g is not None else config.num_attention_heads // config.num_key_value_heads
