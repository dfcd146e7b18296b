"""CPU restatement of nano-qwen's dense Qwen3 forward and greedy decoding -- TEST
INFRASTRUCTURE ONLY (imported by ``tests/`` alone, as the checker).

Built on ``attention_module_forward`` (model/attention.py:82-118) so that the
attention inside the model is the already-pinned oracle; the rest restates
model/transformer.py:24-156 (pre-norm blocks, final norm, LM head),
model/ffn.py:17-28 (SwiGLU) and model/norm.py:17-22 (RMSNorm cast order) in
plain torch CPU arithmetic.

Pinning status (tests/test_oracle_model.py):
  * model_forward            -- logits from the reference's own
                                ``Qwen3Model.forward`` (no cache, and with
                                explicit position_ids) in
                                tests/golden/model_forward.npz.
  * greedy_reference_protocol -- the greedy tokens and per-step logits of the
                                reference's ``TextGenerator.generate`` cache
                                protocol (eval/generate.py:75-136), same file.
  * greedy_full_recompute    -- causality invariant: every step's logits equal
                                the matching row of ONE no-cache forward over
                                the final sequence (itself pinned above), and
                                its first step equals the no-cache prompt
                                forward.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from .attention_oracle import OracleKVCache, attention_module_forward, rms_norm, rope_tables


def _layer_weights(weights: Dict[str, torch.Tensor], i: int) -> Dict[str, torch.Tensor]:
    p = f"layers.{i}.attention."
    return {k: weights[p + k + ".weight"] for k in ("q_proj", "k_proj", "v_proj", "o_proj",
                                                    "q_norm", "k_norm")}


def swiglu(x: torch.Tensor, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """model/ffn.py:17-28: down(silu(x gate^T) * (x up^T))."""
    return (F.silu(x @ gate.t()) * (x @ up.t())) @ down.t()


def model_forward(weights: Dict[str, torch.Tensor], cfg: dict, input_ids: torch.Tensor,
                  position_ids: Optional[torch.Tensor] = None,
                  kv_caches: Optional[List[OracleKVCache]] = None) -> torch.Tensor:
    """Logits (B, S, vocab) of Qwen3Model.forward (transformer.py:107-156), dense layers.

    ``weights`` is keyed by the reference's state-dict names.  With
    ``kv_caches`` the attention follows the reference's cache semantics
    (attention.py:103-113: the cached prefill is not causally masked and, with
    no position_ids, new tokens are rotated at positions 0..S-1).
    """
    H, Hkv, D = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    eps = cfg["rms_norm_eps"]
    cos, sin = rope_tables(D, cfg["max_position_embeddings"], cfg["rope_theta"],
                           cfg.get("rope_scaling"))
    h = weights["embed.embed_tokens.weight"][input_ids]
    for i in range(cfg["num_hidden_layers"]):
        p = f"layers.{i}."
        x = rms_norm(h, weights[p + "input_layernorm.weight"], eps)
        a, _ = attention_module_forward(
            x, _layer_weights(weights, i), num_heads=H, num_kv_heads=Hkv, head_dim=D, eps=eps,
            cos_table=cos, sin_table=sin, position_ids=position_ids,
            kv_cache=kv_caches[i] if kv_caches is not None else None)
        h = h + a
        x = rms_norm(h, weights[p + "post_attention_layernorm.weight"], eps)
        h = h + swiglu(x, weights[p + "feed_forward.gate_proj.weight"],
                       weights[p + "feed_forward.up_proj.weight"],
                       weights[p + "feed_forward.down_proj.weight"])
    h = rms_norm(h, weights["norm.weight"], eps)
    return h @ weights["lm_head.weight"].t()


def greedy_reference_protocol(weights: Dict[str, torch.Tensor], cfg: dict, prompt: Sequence[int],
                              new_tokens: int, forced: Optional[Sequence[int]] = None
                              ) -> Tuple[List[int], torch.Tensor]:
    """Greedy decoding as eval/generate.py:75-136 runs it at temperature 0.

    A fresh cache per layer, the whole prompt through the model with the
    caches, then one token per call with no position_ids.  Returns the tokens
    and the (new_tokens, vocab) logits each token was chosen from.  With
    ``forced``, token i fed back is ``forced[i]`` instead of the argmax
    (teacher forcing: the logits of another run's token sequence).
    """
    caches = [OracleKVCache() for _ in range(cfg["num_hidden_layers"])]
    logits = model_forward(weights, cfg, torch.tensor([list(prompt)]), kv_caches=caches)[0, -1]
    toks, steps = [], []
    for i in range(new_tokens):
        steps.append(logits)
        t = int(logits.argmax()) if forced is None else int(forced[i])
        toks.append(t)
        logits = model_forward(weights, cfg, torch.tensor([[t]]), kv_caches=caches)[0, -1]
    return toks, torch.stack(steps)


def greedy_full_recompute(weights: Dict[str, torch.Tensor], cfg: dict, prompt: Sequence[int],
                          new_tokens: int) -> Tuple[List[int], torch.Tensor]:
    """Greedy decoding with no cache: each step runs the causal forward over the
    whole sequence at positions 0..L-1 and takes the last row.  This is what a
    correct cache (causal prefill, true positions) must reproduce."""
    seq = list(prompt)
    toks, steps = [], []
    for _ in range(new_tokens):
        logits = model_forward(weights, cfg, torch.tensor([seq]))[0, -1]
        steps.append(logits)
        t = int(logits.argmax())
        toks.append(t)
        seq.append(t)
    return toks, torch.stack(steps)
