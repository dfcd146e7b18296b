"""RoPE / YaRN tables and the rotate-half rotation (model/rope.py:17-161).

The tables are built once, on the host, in fp32 with the same sequence of torch
operations as the reference (so they are bit-identical to its
``cos_cached``/``sin_cached``) and are then read by the HIP kernels by
position; no sine or cosine is evaluated on the GPU.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import ops


def _plain_inv_freq(dim: int, base: float) -> torch.Tensor:
    # model/rope.py:25
    return 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))


def yarn_range(dim: int, base: float, original_max: int, beta_fast: float = 32.0,
               beta_slow: float = 1.0) -> Tuple[int, int]:
    """Pair-index range [low, high] over which YaRN blends (model/rope.py:31-43)."""
    def dim_at(rotations: float) -> float:
        return dim * math.log(original_max / (rotations * 2 * math.pi)) / (2 * math.log(base))
    return max(math.floor(dim_at(beta_fast)), 0), min(math.ceil(dim_at(beta_slow)), dim - 1)


def yarn_inv_freq(dim: int, base: float, scale: float, original_max: int) -> torch.Tensor:
    """YaRN inverse frequencies, fixed betas 32/1, no mscale (model/rope.py:53-75)."""
    expo = torch.arange(0, dim, 2, dtype=torch.float32) / dim
    extra = 1.0 / (base ** expo)
    inter = 1.0 / (scale * base ** expo)
    low, high = yarn_range(dim, base, original_max)
    span = (high + 0.001 if low == high else high) - low
    ramp = ((torch.arange(dim // 2, dtype=torch.float32) - low) / span).clamp(0, 1)
    keep = 1.0 - ramp
    return inter * (1 - keep) + extra * keep


def build_tables(dim: int, max_positions: int, base: float,
                 rope_scaling: Optional[dict] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 (max_positions, dim/2) cos and sin tables (model/rope.py:81-107)."""
    if rope_scaling is not None and rope_scaling.get("type") == "yarn":
        inv = yarn_inv_freq(dim, base, rope_scaling.get("factor", 4.0),
                            rope_scaling.get("original_max_position_embeddings", 32768))
    else:
        inv = _plain_inv_freq(dim, base)
    angles = torch.outer(torch.arange(max_positions, dtype=torch.float32), inv)
    return angles.cos(), angles.sin()


class RotaryEmbedding(torch.nn.Module):
    """Same constructor, buffers and forward as model/rope.py:78-130.

    ``cos_cached``/``sin_cached`` are non-persistent fp32 buffers.  A module
    cast such as ``.to(torch.bfloat16)`` casts them too (as in the
    reference); the fused kernels always take fp32 tables, which
    ``tables_f32`` rebuilds on the host in that case.  ``forward`` returns
    rows cast to ``x.dtype`` exactly like the reference.
    """

    def __init__(self, dim: int, max_position_embeddings: int = 32768, base: float = 1_000_000.0,
                 rope_scaling: Optional[dict] = None, device: Optional[torch.device] = None):
        super().__init__()
        self.dim = dim
        self.max_position_embeddings = max_position_embeddings
        self.base = base
        self.rope_scaling = rope_scaling
        cos, sin = build_tables(dim, max_position_embeddings, base, rope_scaling)
        self.register_buffer("cos_cached", cos.to(device) if device else cos, persistent=False)
        self.register_buffer("sin_cached", sin.to(device) if device else sin, persistent=False)
        self._f32 = None

    def tables_f32(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """fp32 tables on the module's device (cached across calls)."""
        c = self.cos_cached
        if c.dtype == torch.float32:
            return c, self.sin_cached
        if self._f32 is None or self._f32[0].device != c.device:
            cos, sin = build_tables(self.dim, self.max_position_embeddings, self.base, self.rope_scaling)
            self._f32 = (cos.to(c.device), sin.to(c.device))
        return self._f32

    def forward(self, x: torch.Tensor, position_ids: Optional[torch.Tensor] = None):
        if position_ids is None:
            seq_len = x.shape[-2]
            return self.cos_cached[:seq_len].to(x.dtype), self.sin_cached[:seq_len].to(x.dtype)
        return self.cos_cached[position_ids].to(x.dtype), self.sin_cached[position_ids].to(x.dtype)


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """model/rope.py:133-161 on the gfx950 row kernel (out of place).

    q/k: (B, H, S, D) device tensors; cos/sin: (S, D/2) or (B, S, D/2) rows
    (as returned by RotaryEmbedding.forward).  Rotation runs in fp32 and is
    rounded once to the input dtype.
    """
    qo, ko = q.clone(memory_format=torch.contiguous_format), k.clone(memory_format=torch.contiguous_format)
    return ops.apply_rope(qo, ko, cos, sin)
