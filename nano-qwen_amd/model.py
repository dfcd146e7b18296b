"""Dense Qwen3 language model around the drop-in attention (model/transformer.py:24-162).

A mirror of the reference's ``Qwen3Model`` / ``TransformerBlock`` with the same
submodule names, so the reference's state dicts load unchanged:
``embed.embed_tokens``, ``layers.{i}.input_layernorm``, ``layers.{i}.attention``
(the drop-in ``Attention``), ``layers.{i}.post_attention_layernorm``,
``layers.{i}.feed_forward.{gate,up,down}_proj``, ``norm``, ``lm_head``.  The
forward signature and the returned dict are the reference's
(transformer.py:107-156).

Only attention runs on the gfx950 kernels; embedding, the layer RMSNorms,
SwiGLU and the LM head are the reference's torch ops (hipBLASLt GEMMs).  MoE
layers (model/moe.py) are outside the attention hot path and not provided.
``gradient_checkpointing`` (config field and attribute, transformer.py:92,
121-127) recomputes each block in the backward when training, as the
reference does.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
import torch.utils.checkpoint as checkpoint_utils

from .attention import Attention, KVCache
from .config import AttentionConfig


@dataclass
class ModelConfig(AttentionConfig):
    """The dense-model fields of model/config.py:14-83 on top of the attention ones."""

    vocab_size: int = 151936
    num_hidden_layers: int = 32
    intermediate_size: int = 11008
    tie_word_embeddings: bool = False
    initializer_range: float = 0.02
    gradient_checkpointing: bool = False


class LayerRMSNorm(nn.Module):
    """RMSNorm over the hidden size, the reference's arithmetic (model/norm.py:17-22):
    fp32 statistic, cast back to the input dtype before the weight multiply."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return y.to(x.dtype) * self.weight


class SwiGLU(nn.Module):
    """model/ffn.py:17-28: down(silu(gate(x)) * up(x))."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class TokenEmbedding(nn.Module):
    """model/embedding.py:9-16."""

    def __init__(self, config):
        super().__init__()
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return self.embed_tokens(input_ids)


def _check_dense(config) -> None:
    if getattr(config, "is_moe", False):
        raise NotImplementedError("MoE layers are outside the attention hot path; dense models only")


class TransformerBlock(nn.Module):
    """Pre-norm block (transformer.py:24-76): x += Attn(norm(x)); x += FFN(norm(x))."""

    def __init__(self, config, layer_idx: int = 0):
        super().__init__()
        _check_dense(config)
        self.layer_idx = layer_idx
        self.config = config
        self.input_layernorm = LayerRMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.attention = Attention(config, layer_idx=layer_idx)
        self.post_attention_layernorm = LayerRMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.feed_forward = SwiGLU(config.hidden_size, config.intermediate_size)

    def forward(self, hidden_states: torch.Tensor, position_ids: Optional[torch.Tensor] = None,
                attention_mask: Optional[torch.Tensor] = None,
                kv_cache: Optional[KVCache] = None):
        residual = hidden_states
        hidden_states = self.attention(self.input_layernorm(hidden_states), position_ids,
                                       attention_mask, kv_cache)
        hidden_states = residual + hidden_states
        residual = hidden_states
        hidden_states = residual + self.feed_forward(self.post_attention_layernorm(hidden_states))
        return hidden_states, None


class Qwen3Model(nn.Module):
    """Embedding -> blocks -> RMSNorm -> LM head (transformer.py:78-156)."""

    def __init__(self, config):
        super().__init__()
        _check_dense(config)
        self.config = config
        self.embed = TokenEmbedding(config)
        self.layers = nn.ModuleList([TransformerBlock(config, layer_idx=i)
                                     for i in range(config.num_hidden_layers)])
        self.norm = LayerRMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if getattr(config, "tie_word_embeddings", False):
            self.lm_head.weight = self.embed.embed_tokens.weight
        # transformer.py:92: each block recomputed in the backward when training
        self.gradient_checkpointing = getattr(config, "gradient_checkpointing", False)
        self.apply(self._init_weights)

    def _init_weights(self, module: nn.Module) -> None:
        std = getattr(self.config, "initializer_range", 0.02)
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=std)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=std)

    def set_cache_semantics(self, fixed: bool) -> None:
        """``fixed=True``: a prefill into a cache is causal and positions continue
        from the cache length (``Attention.rope_positions = "cache"``,
        ``cache_prefill_causal = True``).  ``False`` keeps the reference's
        behaviour (bidirectional cache prefill, positions from 0)."""
        for layer in self.layers:
            layer.attention.rope_positions = "cache" if fixed else "reference"
            layer.attention.cache_prefill_causal = bool(fixed)

    def forward(self, input_ids: torch.Tensor, position_ids: Optional[torch.Tensor] = None,
                attention_mask: Optional[torch.Tensor] = None,
                kv_caches: Optional[List[KVCache]] = None,
                labels: Optional[torch.Tensor] = None) -> dict:
        hidden_states = self.embed(input_ids)
        for i, layer in enumerate(self.layers):
            kv_cache = kv_caches[i] if kv_caches is not None else None
            if self.gradient_checkpointing and self.training:
                # transformer.py:121-127: the block's activations (the attention
                # kernels' Q-hat, K-hat, O and LSE included) are dropped and the
                # block's forward runs again inside the backward
                hidden_states, _ = checkpoint_utils.checkpoint(
                    layer, hidden_states, position_ids, attention_mask, kv_cache, use_reentrant=False)
            else:
                hidden_states, _ = layer(hidden_states, position_ids, attention_mask, kv_cache)
        hidden_states = self.norm(hidden_states)
        logits = self.lm_head(hidden_states)
        loss = None
        if labels is not None:
            loss = F.cross_entropy(logits[..., :-1, :].contiguous().view(-1, logits.shape[-1]),
                                   labels[..., 1:].contiguous().view(-1), ignore_index=-100)
        return {"logits": logits, "loss": loss, "aux_loss": None, "hidden_states": hidden_states}

    @torch.no_grad()
    def count_parameters(self) -> dict:
        """transformer.py:158-162."""
        total = sum(p.numel() for p in self.parameters())
        trainable = sum(p.numel() for p in self.parameters() if p.requires_grad)
        return {"total": total, "trainable": trainable}
