"""Autoregressive generation on the drop-in attention (eval/generate.py:20-183).

``TextGenerator`` keeps the reference's constructor, ``generate`` arguments
(temperature / top-k / top-p sampling, repetition penalty, thinking budget,
stop tokens, streaming callback), ``_sample`` and ``generate_batch``, and its
cache protocol: one ``KVCache`` per layer, the prompt through the model with
the caches, then one token per call.  The caches are preallocated for the
whole generation (prompt + ``max_new_tokens``), so the decode steps never
reallocate.  Which attention semantics that protocol gets (the reference's
bidirectional cached prefill with positions restarting at 0, or causal with
true positions) is the model's setting, ``Qwen3Model.set_cache_semantics``.

``generate_greedy_batch`` is an extension for batched serving with no
counterpart in the reference: prompts of different lengths decode together in
one right-padded batch against a ragged cache (per-row lengths on the device),
always with causal prefill and true positions.
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Callable, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from .attention import KVCache, PagedKVCache


def _device_of(model) -> torch.device:
    return next(model.parameters()).device


class TextGenerator:
    """Autoregressive text generator with KV cache (eval/generate.py:20-183)."""

    def __init__(self, model, tokenizer, device: Optional[torch.device] = None):
        self.model = model
        self.tokenizer = tokenizer
        self.device = torch.device(device) if device is not None else _device_of(model)
        self.model.eval()

    def _caches(self, total: int) -> List[KVCache]:
        return [KVCache(max_seq_len=total) for _ in range(len(self.model.layers))]

    def _step(self, ids: List[int], caches: List[KVCache]) -> torch.Tensor:
        x = torch.tensor([ids], dtype=torch.long, device=self.device)
        return self.model(input_ids=x, kv_caches=caches)["logits"][:, -1, :]

    @torch.no_grad()
    def generate(self, prompt: str, max_new_tokens: int = 512, temperature: float = 0.7,
                 top_k: int = 50, top_p: float = 0.9, repetition_penalty: float = 1.0,
                 enable_thinking: bool = False, thinking_budget: Optional[int] = None,
                 stop_tokens: Optional[List[int]] = None,
                 stream_callback: Optional[Callable[[str], None]] = None) -> str:
        """eval/generate.py:35-136: the same loop, decisions and stop rules."""
        if enable_thinking:
            prompt = prompt + "<think>\n"
        prompt_ids = list(self.tokenizer.encode(prompt, allowed_special="all"))
        think_end = (list(self.tokenizer.encode("</think>\n", allowed_special="all"))
                     if enable_thinking and thinking_budget else [])
        caches = self._caches(len(prompt_ids) + max_new_tokens + len(think_end) + 1)
        logits = self._step(prompt_ids, caches)

        generated: List[int] = []
        thinking_tokens = 0
        thinking_ended = False
        eos_id = getattr(self.tokenizer, "eos_id", None)
        stop_set = set(stop_tokens or [])
        if eos_id is not None:
            stop_set.add(eos_id)

        for _ in range(max_new_tokens):
            if repetition_penalty != 1.0 and generated:
                for t in set(generated):
                    if logits[0, t] > 0:
                        logits[0, t] /= repetition_penalty
                    else:
                        logits[0, t] *= repetition_penalty
            token_id = int(self._sample(logits, temperature, top_k, top_p).item())

            if enable_thinking and not thinking_ended:
                thinking_tokens += 1
                if thinking_budget and thinking_tokens >= thinking_budget:
                    generated.extend(think_end)
                    thinking_ended = True
                    logits = self._step([think_end[-1]], caches)
                    continue

            if token_id in stop_set:
                break
            generated.append(token_id)
            if stream_callback:
                stream_callback(self.tokenizer.decode([token_id]))
            if enable_thinking and not thinking_ended:
                if "</think>" in self.tokenizer.decode(generated[-10:]):
                    thinking_ended = True
            logits = self._step([token_id], caches)

        return self.tokenizer.decode(generated)

    @staticmethod
    def _sample(logits: torch.Tensor, temperature: float, top_k: int, top_p: float) -> torch.Tensor:
        """eval/generate.py:138-170: greedy at temperature 0, else top-k then
        nucleus filtering (a token is dropped once the mass before it reaches
        top_p) and a multinomial draw."""
        if temperature == 0:
            return logits.argmax(dim=-1, keepdim=True)
        logits = logits / temperature
        if top_k > 0:
            top_k = min(top_k, logits.shape[-1])
            kth = torch.topk(logits, top_k, dim=-1).values[..., -1:]
            logits = logits.masked_fill(logits < kth, float("-inf"))
        if top_p < 1.0:
            sorted_logits, order = torch.sort(logits, descending=True, dim=-1)
            p = F.softmax(sorted_logits, dim=-1)
            drop = (p.cumsum(dim=-1) - p) >= top_p
            sorted_logits = sorted_logits.masked_fill(drop, float("-inf"))
            logits = sorted_logits.scatter(1, order, sorted_logits)
        return torch.multinomial(F.softmax(logits, dim=-1), num_samples=1)

    @torch.no_grad()
    def generate_batch(self, prompts: List[str], max_new_tokens: int = 512,
                       temperature: float = 0.7, top_k: int = 50,
                       top_p: float = 0.9) -> List[str]:
        """eval/generate.py:172-183: ``generate`` per prompt."""
        return [self.generate(p, max_new_tokens, temperature, top_k, top_p) for p in prompts]


@contextmanager
def _fixed_semantics(model):
    """Causal cached prefill and true positions for the duration of a call."""
    saved = [(l.attention.rope_positions, l.attention.cache_prefill_causal) for l in model.layers]
    model.set_cache_semantics(True)
    try:
        yield
    finally:
        for l, (rp, cc) in zip(model.layers, saved):
            l.attention.rope_positions, l.attention.cache_prefill_causal = rp, cc


@torch.no_grad()
def generate_greedy_batch(model, prompts: Sequence[Sequence[int]], max_new_tokens: int,
                          stop_tokens: Optional[Sequence[int]] = None,
                          return_logits: bool = False, page_size: Optional[int] = None
                          ) -> Tuple[List[List[int]], Optional[List[torch.Tensor]]]:
    """Greedy decoding of several prompts at once against a ragged KV cache.

    The prompts are right-padded to the longest and prefilled in one causal
    pass (row b's last real token sits at ``len_b - 1`` and never sees the
    padding); each cache is then made ragged with the true lengths, so every
    decode step appends row b's key at slot ``len_b + t``, rotates it at that
    position and attends exactly its own keys.  With ``page_size`` the caches
    are ``PagedKVCache`` page pools (the padding's pages are returned after
    the prefill) instead of dense per-row buffers.  A row stops at its first
    stop token (not included) or after ``max_new_tokens``.  Returns the
    generated tokens per row and, with ``return_logits``, the fp32 logits each
    token was chosen from (one (n_b, vocab) tensor per row).
    """
    if not prompts or any(len(p) == 0 for p in prompts):
        raise ValueError("every prompt needs at least one token")
    dev = _device_of(model)
    B = len(prompts)
    lens = [len(p) for p in prompts]
    L = max(lens)
    ids = torch.zeros(B, L, dtype=torch.long)
    for b, p in enumerate(prompts):
        ids[b, :len(p)] = torch.as_tensor(list(p), dtype=torch.long)
    ids = ids.to(dev)
    stop = set(stop_tokens or [])
    if page_size is None:
        caches = [KVCache(max_seq_len=L + max_new_tokens) for _ in range(len(model.layers))]
    else:
        per_seq = -(-(L + max_new_tokens) // page_size)
        caches = [PagedKVCache(B * per_seq, page_size=page_size, max_pages_per_seq=per_seq)
                  for _ in range(len(model.layers))]
    out: List[List[int]] = [[] for _ in range(B)]
    steps: List[List[torch.Tensor]] = [[] for _ in range(B)]
    done = [False] * B

    with _fixed_semantics(model):
        logits = model(input_ids=ids, kv_caches=caches)["logits"]
        last = torch.as_tensor(lens, device=dev) - 1
        logits = logits[torch.arange(B, device=dev), last]
        lens_t = torch.as_tensor(lens, dtype=torch.int32, device=dev)
        for c in caches:
            c.set_lengths(lens_t.clone() if page_size is None else lens)
        for _ in range(max_new_tokens):
            nxt = logits.argmax(dim=-1)
            toks = nxt.tolist()
            lg = logits.float().cpu() if return_logits else None
            for b in range(B):
                if done[b]:
                    continue
                if toks[b] in stop:
                    done[b] = True
                    continue
                out[b].append(toks[b])
                if lg is not None:
                    steps[b].append(lg[b])
                if len(out[b]) == max_new_tokens:
                    done[b] = True
            if all(done):
                break
            logits = model(input_ids=nxt[:, None], kv_caches=caches)["logits"][:, -1, :]
    if not return_logits:
        return out, None
    vocab = logits.shape[-1]
    return out, [torch.stack(s) if s else torch.empty(0, vocab) for s in steps]
