"""nano-qwen's GQA attention hot path on MI355X (gfx950), as a drop-in.

QK-Norm, RoPE/YaRN, causal FlashAttention-2-style prefill and split-K
single-token decode against a KV cache, as hand-written HIP kernels in
libnqattn.so (C ABI in include/nq_attn.h), called from PyTorch-ROCm through
ctypes.  Build with ``python -m nano_qwen_amd.build``.

Public surface, mirroring the reference:
  Attention, KVCache           model/attention.py:24-118
  RMSNorm                      model/norm.py:11-22
  RotaryEmbedding, apply_rotary_pos_emb   model/rope.py:78-161
  flash_attention, apply_rope  kernels/flash_attn.py:130, kernels/rope.py:99
  AttentionConfig              attention fields of model/config.py:14-83
  Qwen3Model, TransformerBlock, ModelConfig   model/transformer.py:24-162 (dense)
  TextGenerator                eval/generate.py:20-183
  RingAttention, split_sequence   distributed/context_parallel.py:17-140 (one GPU's share)

Training: ``Attention`` with autograd and ``flash_attention`` on tensors that
require grad run the FlashAttention-2 backward kernels (``attention_backward``,
``qk_norm_rope_backward``; autograd Functions ``attention_core`` and
``flash_attention_train``) where the reference runs SDPA's autograd.

Extensions with no reference counterpart: ``generate_greedy_batch`` (ragged
batched greedy decoding against per-row cache lengths), ``PagedKVCache``
(block-table page pool), ``attention_decode_paged`` (decode with the new
token's K/V append fused in) and ``kv_append_paged``.
"""

from .config import AttentionConfig
from .ops import (apply_rope, attention_decode, attention_decode_paged, attention_prefill,
                  attention_prefill_paged,
                  decode_workspace_bytes, flash_attention, kv_append_paged, qk_norm_rope)
from .norm import RMSNorm
from .rope import RotaryEmbedding, apply_rotary_pos_emb, build_tables
from .attention import Attention, KVCache, PagedKVCache, stats
from .model import ModelConfig, Qwen3Model, TransformerBlock
from .generate import TextGenerator, generate_greedy_batch
from .ops import attention_backward, attention_merge_, qk_norm_rope_backward
from .autograd import attention_core, flash_attention_train
from .ring import RingAttention, ring_attention_all_ranks, ring_schedule, ring_step, split_sequence

__all__ = [
    "Attention", "KVCache", "RMSNorm", "RotaryEmbedding", "AttentionConfig",
    "apply_rotary_pos_emb", "build_tables", "flash_attention", "apply_rope",
    "qk_norm_rope", "attention_prefill", "attention_prefill_paged", "attention_decode", "decode_workspace_bytes", "stats",
    "ModelConfig", "Qwen3Model", "TransformerBlock", "TextGenerator", "generate_greedy_batch",
    "PagedKVCache", "attention_decode_paged", "kv_append_paged",
    "attention_merge_", "RingAttention", "ring_step", "ring_schedule", "split_sequence",
    "ring_attention_all_ranks", "attention_backward", "qk_norm_rope_backward", "attention_core",
    "flash_attention_train",
]
