"""Training path on the kernels: autograd Functions with HIP forward and backward.

The reference trains through F.scaled_dot_product_attention's autograd
(model/attention.py:110-115, called by the training loops' loss.backward())
and torch's autograd of QK-Norm and RoPE (model/norm.py:17-22,
model/rope.py:133-161).  Here:

  * ``attention_core`` -- QK-Norm + RoPE of q and k (row kernel), then the
    GQA prefill (causal, or over each sequence's unpadded keys) with its LSE;
    backward: the FlashAttention-2 backward kernels, then the QK-Norm + RoPE
    backward kernel (gradients for the pre-norm q, k and for both norm
    weights).
  * ``flash_attention_train`` -- the plain attention of kernels/flash_attn.py
    (inputs already normed), forward + backward on the kernels.

Saved for backward: the pre-norm q and k, Q-hat, K-hat, V, O and the fp32
LSE (the FlashAttention-2 recomputation scheme: no S x T matrix is stored).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import ops


class _AttentionCore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, q_weight, k_weight, cos, sin, position_ids, pos_offset: int, eps: float,
                causal: bool, key_lens):
        q_hat, k_hat, _ = ops.qk_norm_rope(q=q, k=k, q_weight=q_weight, k_weight=k_weight, eps=eps,
                                           cos=cos, sin=sin, position_ids=position_ids,
                                           pos_offset=pos_offset)
        o, lse = ops.attention_prefill(q_hat, k_hat, v, causal=causal, key_lens=key_lens, return_lse=True)
        ctx.save_for_backward(q, k, v, q_hat, k_hat, o, lse, q_weight, k_weight, cos, sin, position_ids,
                              key_lens)
        ctx.pos_offset, ctx.eps, ctx.causal = pos_offset, eps, causal
        return o

    @staticmethod
    def backward(ctx, dout):
        q, k, v, q_hat, k_hat, o, lse, qw, kw, cos, sin, pos, key_lens = ctx.saved_tensors
        dq_hat, dk_hat, dv = ops.attention_backward(q_hat, k_hat, v, o, dout.to(o.dtype), lse,
                                                    causal=ctx.causal, key_lens=key_lens)
        kw_args = dict(eps=ctx.eps, cos=cos, sin=sin, position_ids=pos, pos_offset=ctx.pos_offset)
        dq, dqw = ops.qk_norm_rope_backward(q, dq_hat, weight=qw, **kw_args)
        dk, dkw = ops.qk_norm_rope_backward(k, dk_hat, weight=kw, **kw_args)
        gqw = dqw.to(qw.dtype) if (qw is not None and ctx.needs_input_grad[3]) else None
        gkw = dkw.to(kw.dtype) if (kw is not None and ctx.needs_input_grad[4]) else None
        return dq, dk, dv, gqw, gkw, None, None, None, None, None, None, None


def attention_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   q_weight: Optional[torch.Tensor], k_weight: Optional[torch.Tensor], *,
                   cos: torch.Tensor, sin: torch.Tensor,
                   position_ids: Optional[torch.Tensor] = None, pos_offset: int = 0,
                   eps: float = 1e-6, causal: bool = True,
                   key_lens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """o = attention(rope(norm(q)), rope(norm(k)), v) with gradients for q, k, v and
    both norm weights.  q: (B, Hq, S, D), k/v: (B, Hkv, S, D) pre-norm;
    key_lens (int32 (B,)) limits sequence b to keys [0, key_lens[b]).
    Returns (B, Hq, S, D) (a view of (B, S, Hq, D) storage)."""
    return _AttentionCore.apply(q, k, v, q_weight, k_weight, cos, sin, position_ids, pos_offset, eps,
                                causal, key_lens)


class _FlashAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal: bool, sm_scale: Optional[float]):
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
        o, lse = ops.attention_prefill(q, k, v, causal=causal, sm_scale=sm_scale, out=out,
                                       return_lse=True)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.causal, ctx.sm_scale = causal, sm_scale
        return o

    @staticmethod
    def backward(ctx, dout):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = ops.attention_backward(q, k, v, o, dout.to(o.dtype), lse, causal=ctx.causal,
                                            sm_scale=ctx.sm_scale)
        return dq, dk, dv, None, None


def flash_attention_train(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = True,
                          sm_scale: Optional[float] = None) -> torch.Tensor:
    """Attention over already-normed q (B, H, S, D) and k/v (B, Hkv, T, D), with
    the backward on the kernels."""
    return _FlashAttention.apply(q, k, v, causal, sm_scale)
