"""Training path on the kernels: autograd Functions with HIP forward and backward.

The reference trains through F.scaled_dot_product_attention's autograd
(model/attention.py:110-115, called by the training loops' loss.backward())
and torch's autograd of QK-Norm and RoPE (model/norm.py:17-22,
model/rope.py:133-161).  Here:

  * ``attention_core`` -- QK-Norm + RoPE of q and k (row kernel), then the
    GQA prefill (causal, or over each sequence's unpadded keys, or with a
    general attention-mask bias) with its LSE; backward: the
    FlashAttention-2 backward kernels, then the QK-Norm + RoPE backward
    kernel (gradients for the pre-norm q, k and for both norm weights).
    With a cache (``kv_store``) the new K-hat/V rows are appended to it and
    the queries attend every cached row, as KVCache.update + SDPA do
    (model/attention.py:31-38, 102-115); gradients reach the new rows' k and
    v (the cache holds values, not graph nodes, so rows cached by earlier
    calls get none -- the reference's concatenation would carry them to an
    earlier call's graph, a case no training loop of the reference uses).
  * ``flash_attention_train`` -- the plain attention of kernels/flash_attn.py
    (inputs already normed), forward + backward on the kernels.

Saved for backward: the pre-norm q and k, Q-hat, K-hat, V, O and the fp32
LSE (the FlashAttention-2 recomputation scheme: no S x T matrix is stored).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import ops


class _AttentionCore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, q_weight, k_weight, cos, sin, position_ids, pos_offset: int, eps: float,
                causal: bool, key_lens, bias, kv_store):
        pos = dict(position_ids=position_ids, pos_offset=pos_offset)
        if kv_store is None:
            past = 0
            q_hat, k_att, _ = ops.qk_norm_rope(q=q, k=k, q_weight=q_weight, k_weight=k_weight, eps=eps,
                                               cos=cos, sin=sin, **pos)
            v_att = v
        else:
            # the new K-hat / V rows go to rows past .. past + S - 1 of the cache
            kc, vc, past = kv_store
            q_hat, _, _ = ops.qk_norm_rope(q=q, k=k, v=v, k_out=kc, v_out=vc, q_weight=q_weight,
                                           k_weight=k_weight, eps=eps, cos=cos, sin=sin,
                                           kv_row_offset=past, **pos)
            T = past + q.shape[2]
            k_att, v_att = kc[:, :, :T], vc[:, :, :T]
        o, lse = ops.attention_prefill(q_hat, k_att, v_att, causal=causal, key_lens=key_lens, bias=bias,
                                       return_lse=True)
        ctx.save_for_backward(q, k, q_hat, k_att, v_att, o, lse, q_weight, k_weight, cos, sin, position_ids,
                              key_lens)
        ctx.pos_offset, ctx.eps, ctx.causal, ctx.bias, ctx.past = pos_offset, eps, causal, bias, past
        return o

    @staticmethod
    def backward(ctx, dout):
        q, k, q_hat, k_att, v_att, o, lse, qw, kw, cos, sin, pos, key_lens = ctx.saved_tensors
        dq_hat, dk_att, dv_att = ops.attention_backward(q_hat, k_att, v_att, o, dout.to(o.dtype), lse,
                                                        causal=ctx.causal, key_lens=key_lens, bias=ctx.bias)
        past = ctx.past
        dk_hat, dv = dk_att[:, :, past:], dv_att[:, :, past:]
        kw_args = dict(eps=ctx.eps, cos=cos, sin=sin, position_ids=pos, pos_offset=ctx.pos_offset)
        dq, dqw = ops.qk_norm_rope_backward(q, dq_hat, weight=qw, **kw_args)
        dk, dkw = ops.qk_norm_rope_backward(k, dk_hat, weight=kw, **kw_args)
        gqw = dqw.to(qw.dtype) if (qw is not None and ctx.needs_input_grad[3]) else None
        gkw = dkw.to(kw.dtype) if (kw is not None and ctx.needs_input_grad[4]) else None
        return dq, dk, dv, gqw, gkw, None, None, None, None, None, None, None, None, None


def attention_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   q_weight: Optional[torch.Tensor], k_weight: Optional[torch.Tensor], *,
                   cos: torch.Tensor, sin: torch.Tensor,
                   position_ids: Optional[torch.Tensor] = None, pos_offset: int = 0,
                   eps: float = 1e-6, causal: bool = True,
                   key_lens: Optional[torch.Tensor] = None,
                   bias: Optional[ops.AttnBias] = None,
                   kv_store: Optional[Tuple[torch.Tensor, torch.Tensor, int]] = None) -> torch.Tensor:
    """o = attention(rope(norm(q)), rope(norm(k)), v) with gradients for q, k, v and
    both norm weights.  q: (B, Hq, S, D), k/v: (B, Hkv, S, D) pre-norm;
    key_lens (int32 (B,)) limits sequence b to keys [0, key_lens[b]); bias (an
    ``ops.AttnBias`` built with ``transpose=True``) adds a general attention
    mask.  ``kv_store = (k_cache, v_cache, past)``: the new K-hat / V rows are
    written at rows past .. past + S - 1 of the (B, Hkv, T_cap, D) caches and
    the queries attend rows 0 .. past + S - 1.
    Returns (B, Hq, S, D) (a view of (B, S, Hq, D) storage)."""
    return _AttentionCore.apply(q, k, v, q_weight, k_weight, cos, sin, position_ids, pos_offset, eps,
                                causal, key_lens, bias, kv_store)


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
