"""Drop-in GQA attention and KV cache for nano-qwen (model/attention.py:24-118).

``Attention`` keeps the reference's constructor, submodule names (so state
dicts load unchanged: ``q_proj``, ``k_proj``, ``v_proj``, ``o_proj``,
``q_norm``, ``k_norm``) and ``forward(hidden_states, position_ids=None,
attention_mask=None, kv_cache=None)`` signature.  ``KVCache`` keeps
``update(key, value) -> (K, V)``, ``seq_len`` and ``reset()`` and the
(B, Hkv, T, D) layout, but stores rows in a preallocated buffer instead of
concatenating on every step.

Every forward runs on the gfx950 kernels; there is no second backend:
  * no attention_mask, no autograd: one row-kernel launch (K-Norm + RoPE ->
    K-hat, plus the V copy when a cache is used), then the prefill kernel
    (Q-Norm + RoPE fused into the Q load), or the split-K decode kernel when
    a cache is present and S == 1;
  * autograd (training, with or without a plain KVCache): the same kernels
    through an autograd Function whose backward is the FlashAttention-2
    backward kernels plus the QK-Norm + RoPE backward kernel
    (nano_qwen_amd.autograd);
  * an attention_mask, non-causal as SDPA is with a mask (attention.py:113):
    a key-padding mask (the same prefix [0, L_b) of each sequence's keys for
    every head and query, as a right-padded batch gives) as per-sequence key
    counts; any other bool or float mask as an additive bias the kernels read
    per tile (``ops.AttnBias``), forward and backward;
  * attention dropout while training -> NotImplementedError (no reference
    config sets it; the kernels have no dropout);
  * host tensors -> RuntimeError (the kernels are the product; there is no
    CPU path).

Reference semantics reproduced by default (quirks of the reference, kept for
parity, each switchable):
  * ``position_ids=None`` rotates at positions 0..S-1 even when a cache
    already holds rows (model/rope.py:123-126).  ``rope_positions="cache"``
    continues from the cache length instead.
  * A forward with a cache is not causal (attention.py:113), so a multi-token
    prefill into a cache is bidirectional.  ``cache_prefill_causal=True``
    makes it causal.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import autograd, ops
from .config import num_kv_groups
from .norm import RMSNorm
from .rope import RotaryEmbedding

# Counters of which path forward() took.  "torch_forward" counts forwards
# that left the kernels; no path does, so it stays 0 (kept for callers that
# read it).
stats = {"kernel_forward": 0, "kernel_train_forward": 0, "torch_forward": 0}


def key_padding_lengths(mask: torch.Tensor, B: int, T: int) -> Optional[torch.Tensor]:
    """Per-sequence key counts (int32 (B,), on the mask's device) when ``mask``,
    broadcast as SDPA broadcasts attn_mask against (B, H, S, T), keeps for
    every head and query the same prefix [0, L_b) of sequence b's keys with
    L_b >= 1 (a right-padded batch); None for any other mask (a query-dependent
    or head-dependent pattern, holes, an all-padding row, a float mask with
    values other than 0 and -inf, or a dtype SDPA refuses), which then runs
    as an additive bias read by the kernels (``ops.AttnBias``, which refuses
    what SDPA refuses).  The answer is cached on the mask tensor (keyed by its
    version), so a model that hands one mask to every layer pays one host sync.
    """
    if mask.dim() > 4 or mask.dim() == 0:
        return None
    cached = getattr(mask, "_nq_key_lens", None)
    if cached is not None and cached[0] == mask._version and cached[1] == (B, T):
        return cached[2]
    lens = _prefix_lengths(mask, B, T)
    try:
        mask._nq_key_lens = (mask._version, (B, T), lens)
    except (AttributeError, RuntimeError):
        pass
    return lens


def _prefix_lengths(mask: torch.Tensor, B: int, T: int) -> Optional[torch.Tensor]:
    m = mask.reshape((1,) * (4 - mask.dim()) + tuple(mask.shape))  # SDPA's broadcast alignment
    if m.shape[1] != 1 or m.shape[2] != 1 or m.shape[3] != T or m.shape[0] not in (1, B):
        return None
    m = m[:, 0, 0]
    if m.dtype == torch.bool:
        keep = m
    elif m.is_floating_point():
        keep = m == 0
        if not bool((keep | (m == float("-inf"))).all()):
            return None  # an additive bias, not a keep / drop mask
    else:
        return None  # SDPA refuses other dtypes; so does AttnBias
    lens = keep.sum(-1, dtype=torch.int32)
    prefix = torch.arange(T, device=m.device)[None, :] < lens[:, None]
    if not bool(((keep == prefix).all() & (lens >= 1).all()).item()):
        return None
    return lens.expand(B).contiguous()


class KVCache:
    """Preallocated (B, Hkv, T_cap, D) cache with the reference's API.

    ``key``/``value`` are views of the valid rows (B, Hkv, seq_len, D), like
    the tensors the reference's KVCache holds.  Capacity grows by doubling
    when an update does not fit (one copy); pass ``max_seq_len`` to size it
    once.

    Ragged caches (an extension for batched serving, not in the reference):
    after a right-padded prefill, ``set_lengths(lens)`` records per-row
    lengths (an int32 device tensor).  Each one-token ``Attention`` step then
    appends row b's key at slot ``lens[b]``, rotates it at position
    ``lens[b]`` (unless position_ids are given), attends keys
    ``[0, lens[b] + 1)`` and advances ``lens`` on the device.  ``seq_len`` is
    then the storage extent (the largest row); rows past a row's length hold
    padding and are never read.
    """

    def __init__(self, max_seq_len: Optional[int] = None):
        self.max_seq_len = max_seq_len
        self._k: Optional[torch.Tensor] = None
        self._v: Optional[torch.Tensor] = None
        self._len = 0
        self.key: Optional[torch.Tensor] = None
        self.value: Optional[torch.Tensor] = None
        self.lens: Optional[torch.Tensor] = None
        self._lens_spare: Optional[torch.Tensor] = None
        self._ident: Optional[torch.Tensor] = None
        # device copy of seq_len for every row, kept by the fused one-token
        # step (which writes lens + 1 into the spare); valid while _dev_at == seq_len
        self._dev_lens: Optional[torch.Tensor] = None
        self._dev_spare: Optional[torch.Tensor] = None
        self._dev_at = -1

    @property
    def seq_len(self) -> int:
        return self._len

    @property
    def capacity(self) -> int:
        return 0 if self._k is None else self._k.shape[2]

    def reserve(self, B: int, H: int, total: int, D: int, dtype, device) -> None:
        """Make room for ``total`` rows (allocating or growing the storage)."""
        if self._k is not None:
            if (self._k.shape[0], self._k.shape[1], self._k.shape[3]) != (B, H, D):
                raise ValueError(f"cache holds {tuple(self._k.shape)}, update needs B={B} H={H} D={D}")
            if self._k.dtype != dtype or self._k.device != torch.device(device):
                raise TypeError("cache dtype/device differ from the update")
            if total <= self.capacity:
                return
        cap = max(total, self.max_seq_len or 0, 2 * self.capacity, 64)
        cap = (cap + 63) // 64 * 64
        k = torch.empty(B, H, cap, D, dtype=dtype, device=device)
        v = torch.empty(B, H, cap, D, dtype=dtype, device=device)
        if self._len:
            k[:, :, :self._len] = self._k[:, :, :self._len]
            v[:, :, :self._len] = self._v[:, :, :self._len]
        self._k, self._v = k, v
        self._refresh()

    def storage(self) -> Tuple[torch.Tensor, torch.Tensor]:
        return self._k, self._v

    def advance(self, n: int) -> None:
        self._len += n
        self._refresh()

    def _refresh(self) -> None:
        if self._k is None:
            self.key = self.value = None
        else:
            self.key = self._k[:, :, :self._len]
            self.value = self._v[:, :, :self._len]

    def set_lengths(self, lens: torch.Tensor) -> None:
        """Make the cache ragged: row b holds ``lens[b]`` (<= seq_len) valid keys."""
        if self._k is None:
            raise ValueError("set_lengths needs a filled cache")
        lens = lens.to(device=self._k.device, dtype=torch.int32).contiguous()
        if lens.shape != (self._k.shape[0],):
            raise ValueError(f"lens must have shape ({self._k.shape[0]},), got {tuple(lens.shape)}")
        if int(lens.max()) > self._len or int(lens.min()) < 1:
            raise ValueError(f"lens must lie in [1, seq_len={self._len}]")
        self.lens = lens
        self._lens_spare = None

    def _spare_lens(self) -> torch.Tensor:
        """The second lengths buffer: a fused decode step writes lens + 1 into it."""
        if self._lens_spare is None:
            self._lens_spare = torch.empty_like(self.lens)
        return self._lens_spare

    def _step_lengths(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(lens, lens_next) for a fused one-token step of an unragged cache:
        lens holds seq_len for every row (refilled only when it went stale, e.g.
        after a prefill or update()); the step writes seq_len + 1 to lens_next."""
        B = self._k.shape[0]
        if self._dev_lens is None or self._dev_lens.shape[0] != B or self._dev_lens.device != self._k.device:
            self._dev_lens = torch.empty(B, dtype=torch.int32, device=self._k.device)
            self._dev_spare = torch.empty_like(self._dev_lens)
            self._dev_at = -1
        if self._dev_at != self._len:
            self._dev_lens.fill_(self._len)
            self._dev_at = self._len
        return self._dev_lens, self._dev_spare

    def _step_done(self) -> None:
        """After a fused one-token step: the spare holds the new lengths."""
        self._dev_lens, self._dev_spare = self._dev_spare, self._dev_lens
        self.advance(1)
        self._dev_at = self._len

    def _identity_table(self) -> torch.Tensor:
        """Block table [[0], [1], ...]: row b of the storage is page b."""
        B = self._k.shape[0]
        t = self._ident
        if t is None or t.shape[0] != B or t.device != self._k.device:
            t = torch.arange(B, dtype=torch.int32, device=self._k.device).view(B, 1)
            self._ident = t
        return t

    def update(self, key: torch.Tensor, value: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Append (B, Hkv, S, D) rows; returns all valid rows (attention.py:31-38)."""
        if self.lens is not None:
            raise NotImplementedError("update() appends one slot for all rows; a ragged cache "
                                      "is advanced by Attention's kernel path only")
        B, H, S, D = key.shape
        self.reserve(B, H, self._len + S, D, key.dtype, key.device)
        self._k[:, :, self._len:self._len + S] = key
        self._v[:, :, self._len:self._len + S] = value
        self.advance(S)
        return self.key, self.value

    def reset(self) -> None:
        self._len = 0
        self.lens = None
        self._lens_spare = None
        self._dev_at = -1
        self._refresh()


class PagedKVCache:
    """KV cache held in fixed-size pages of a pool, addressed through a block table.

    An extension for batched serving with no counterpart in the reference
    (whose KVCache, model/attention.py:24-46, is one dense tensor per layer):
    K-hat and V of sequence b, row t, live in page ``block_table[b, t //
    page_size]`` at row ``t % page_size`` of the pools ``k_pool`` /
    ``v_pool`` of shape (num_pages, Hkv, page_size, D).  Pages are taken from
    a free list as sequences grow and returned by ``free`` / ``reset``, so
    sequences of very different lengths share one pool without padding to
    the longest.  ``page_size`` is a multiple of 32.

    Semantics are the causal ones with true positions: a multi-token forward
    appends its rows after each sequence's current length (causal attention
    over the cache), and a one-token forward appends, rotates at and attends
    up to each sequence's own length in one launch.  ``lens`` holds the
    per-sequence lengths on the device; ``host_lens`` mirrors them (every
    step adds a known number of rows), so page allocation never reads the
    device.  ``set_lengths`` trims right-padded prompts after a batched
    prefill, as ``KVCache.set_lengths`` does.
    """

    def __init__(self, num_pages: int, page_size: int = 64, max_pages_per_seq: Optional[int] = None):
        if page_size <= 0 or page_size % 32:
            raise ValueError(f"page_size must be a positive multiple of 32, got {page_size}")
        if num_pages <= 0:
            raise ValueError("num_pages must be positive")
        self.num_pages = num_pages
        self.page_size = page_size
        self.max_pages_per_seq = max_pages_per_seq or num_pages
        self.k_pool: Optional[torch.Tensor] = None
        self.v_pool: Optional[torch.Tensor] = None
        self.block_table: Optional[torch.Tensor] = None
        self.lens: Optional[torch.Tensor] = None
        self._lens_spare: Optional[torch.Tensor] = None
        self.host_lens: list = []
        self._pages: list = []
        self._free = list(range(num_pages - 1, -1, -1))

    # -- sizes
    @property
    def seq_len(self) -> int:
        """Longest sequence held (the reference KVCache's seq_len for B = 1)."""
        return max(self.host_lens, default=0)

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def _setup(self, B: int, H: int, D: int, dtype, device) -> None:
        if self.k_pool is None:
            shape = (self.num_pages, H, self.page_size, D)
            self.k_pool = torch.empty(shape, dtype=dtype, device=device)
            self.v_pool = torch.empty(shape, dtype=dtype, device=device)
        elif (self.k_pool.shape[1], self.k_pool.shape[3]) != (H, D) or self.k_pool.dtype != dtype:
            raise ValueError(f"pool holds {tuple(self.k_pool.shape)} {self.k_pool.dtype}, "
                             f"rows have Hkv={H} D={D} {dtype}")
        if self.block_table is None:
            self.block_table = torch.zeros(B, self.max_pages_per_seq, dtype=torch.int32, device=device)
            self.lens = torch.zeros(B, dtype=torch.int32, device=device)
            self.host_lens = [0] * B
            self._pages = [[] for _ in range(B)]
        elif self.block_table.shape[0] != B:
            raise ValueError(f"cache holds {self.block_table.shape[0]} sequences, the batch has {B}")

    def _grow(self, new_lens) -> None:
        """Map pages so that sequence b can hold new_lens[b] rows."""
        changed = False
        for b, n in enumerate(new_lens):
            need = -(-n // self.page_size)
            if need > self.max_pages_per_seq:
                raise ValueError(f"sequence {b} needs {need} pages, max_pages_per_seq is {self.max_pages_per_seq}")
            while len(self._pages[b]) < need:
                if not self._free:
                    raise RuntimeError("PagedKVCache is out of pages")
                self._pages[b].append(self._free.pop())
                changed = True
        if changed:
            host = torch.zeros(self.block_table.shape, dtype=torch.int32)
            for b, pages in enumerate(self._pages):
                if pages:
                    host[b, :len(pages)] = torch.tensor(pages, dtype=torch.int32)
            self.block_table.copy_(host, non_blocking=False)

    def _spare_lens(self) -> torch.Tensor:
        if self._lens_spare is None:
            self._lens_spare = torch.empty_like(self.lens)
        return self._lens_spare

    def set_lengths(self, lens) -> None:
        """Trim each sequence to lens[b] rows (<= its current length); freed tail pages return to the pool."""
        if self.lens is None:
            raise ValueError("set_lengths needs a filled cache")
        vals = [int(x) for x in (lens.tolist() if torch.is_tensor(lens) else lens)]
        if len(vals) != len(self.host_lens):
            raise ValueError(f"lens must have {len(self.host_lens)} entries")
        for b, n in enumerate(vals):
            if not 0 <= n <= self.host_lens[b]:
                raise ValueError(f"lens[{b}] = {n} outside [0, {self.host_lens[b]}]")
        for b, n in enumerate(vals):
            keep = -(-n // self.page_size)
            while len(self._pages[b]) > keep:
                self._free.append(self._pages[b].pop())
        self.host_lens = vals
        self.lens.copy_(torch.tensor(vals, dtype=torch.int32))

    def free(self, b: int) -> None:
        """Drop sequence b (its pages return to the pool; its length becomes 0)."""
        self.set_lengths([0 if i == b else n for i, n in enumerate(self.host_lens)])

    def reset(self) -> None:
        self._free = list(range(self.num_pages - 1, -1, -1))
        self.block_table = None
        self.lens = None
        self._lens_spare = None
        self.host_lens = []
        self._pages = []

    def gather(self, b: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Sequence b's K-hat and V as dense (Hkv, lens[b], D) tensors (a device copy)."""
        n = self.host_lens[b]
        pages = torch.tensor(self._pages[b], dtype=torch.long, device=self.k_pool.device)
        k = self.k_pool.index_select(0, pages).transpose(0, 1).reshape(self.k_pool.shape[1], -1, self.k_pool.shape[3])
        v = self.v_pool.index_select(0, pages).transpose(0, 1).reshape(self.v_pool.shape[1], -1, self.v_pool.shape[3])
        return k[:, :n], v[:, :n]


class Attention(nn.Module):
    """Multi-head attention with GQA and QK-Norm (model/attention.py:49-118)."""

    def __init__(self, config, layer_idx: int = 0):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.hidden_size = config.hidden_size
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.num_kv_groups = num_kv_groups(config)
        bias = getattr(config, "attention_bias", False)
        self.q_proj = nn.Linear(self.hidden_size, self.num_heads * self.head_dim, bias=bias)
        self.k_proj = nn.Linear(self.hidden_size, self.num_kv_heads * self.head_dim, bias=bias)
        self.v_proj = nn.Linear(self.hidden_size, self.num_kv_heads * self.head_dim, bias=bias)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, self.hidden_size, bias=bias)
        self.qk_norm = getattr(config, "qk_norm", True)
        if self.qk_norm:
            self.q_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)
            self.k_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(
            dim=self.head_dim,
            max_position_embeddings=config.max_position_embeddings,
            base=config.rope_theta,
            rope_scaling=getattr(config, "rope_scaling", None),
        )
        dropout = getattr(config, "attention_dropout", 0.0)
        self.attn_dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()
        self.rope_positions = "reference"     # or "cache"
        self.cache_prefill_causal = False

    # ------------------------------------------------------------------ forward
    def forward(self, hidden_states: torch.Tensor, position_ids: Optional[torch.Tensor] = None,
                attention_mask: Optional[torch.Tensor] = None,
                kv_cache: Optional[KVCache] = None) -> torch.Tensor:
        if not hidden_states.is_cuda:
            raise RuntimeError("nano_qwen_amd.Attention runs on HIP devices only")
        B, S, _ = hidden_states.shape
        H, Hkv, D = self.num_heads, self.num_kv_heads, self.head_dim
        q = self.q_proj(hidden_states)
        k = self.k_proj(hidden_states)
        v = self.v_proj(hidden_states)
        if B == 0 or S == 0:
            # no query rows: the reference's SDPA returns an empty output and its
            # cache update appends nothing (attention.py:103-118); no launch here
            return self.o_proj(q.new_zeros(B, S, H * D))
        if self.training and getattr(self.config, "attention_dropout", 0.0) > 0:
            # attention.py:114 applies dropout_p while training; no reference
            # config sets attention_dropout above 0, and the kernels have no
            # dropout
            raise NotImplementedError(
                f"attention_dropout={self.config.attention_dropout} while training: the HIP attention "
                "kernels implement no dropout; set config.attention_dropout = 0.0 (every reference "
                "config does) or evaluate with model.eval()")
        qw = self.q_norm.weight if self.qk_norm else None
        kw = self.k_norm.weight if self.qk_norm else None
        needs_grad = torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (q, k, v, qw, kw))
        paged = isinstance(kv_cache, PagedKVCache)
        ragged = kv_cache is not None and not paged and kv_cache.lens is not None
        if (paged or ragged) and (attention_mask is not None or needs_grad):
            raise NotImplementedError("ragged and paged caches take no attention mask and no autograd "
                                      "(serving caches); use a plain KVCache or none")
        past = kv_cache.seq_len if (kv_cache is not None and not paged) else 0
        T = past + S
        # attention.py:110-113: SDPA takes the mask as given.  A mask that keeps
        # the same prefix of each sequence's keys for every head and query runs
        # as per-sequence key counts; any other as an additive bias read by the
        # kernels, per tile.
        key_lens, bias = None, None
        if attention_mask is not None:
            key_lens = key_padding_lengths(attention_mask, B, T)
            if key_lens is None:
                bias = ops.AttnBias(attention_mask, B, H, S, T, q.dtype, q.device, transpose=needs_grad)
        # is_causal only without a mask and a cache (attention.py:113), or for
        # a multi-token step into a cache under the fixed semantics
        causal = attention_mask is None and (kv_cache is None or (self.cache_prefill_causal and S > 1))

        q4 = q.view(B, S, H, D).transpose(1, 2)
        k4 = k.view(B, S, Hkv, D).transpose(1, 2)
        v4 = v.view(B, S, Hkv, D).transpose(1, 2)
        cos, sin = self.rotary_emb.tables_f32()
        eps = self.config.rms_norm_eps
        pos_offset = past if (self.rope_positions == "cache" and position_ids is None) else 0
        if needs_grad:
            # training: the forward and backward both on the kernels; with a
            # cache the new rows are appended and every cached row attended
            stats["kernel_train_forward"] += 1
            kv_store = None
            if kv_cache is not None:
                kv_cache.reserve(B, Hkv, T, D, k.dtype, k.device)
                kc, vc = kv_cache.storage()
                kv_store = (kc, vc, past)
                kv_cache.advance(S)
            o = autograd.attention_core(q4, k4, v4, qw, kw, cos=cos, sin=sin,
                                        position_ids=position_ids, pos_offset=pos_offset, eps=eps,
                                        causal=causal, key_lens=key_lens, bias=bias, kv_store=kv_store)
            return self.o_proj(o.transpose(1, 2).reshape(B, S, H * D))
        stats["kernel_forward"] += 1
        if paged:
            return self._paged_forward(q4, k4, v4, position_ids, kv_cache, cos, sin, qw, kw, eps)

        if kv_cache is None:
            k_hat = torch.empty(B, S, Hkv, D, dtype=k.dtype, device=k.device).transpose(1, 2)
            ops.qk_norm_rope(k=k4, k_out=k_hat, k_weight=kw, eps=eps, cos=cos, sin=sin,
                             position_ids=position_ids, pos_offset=pos_offset)
            o = ops.attention_prefill(q4, k_hat, v4, q_weight=qw, eps=eps, cos=cos, sin=sin,
                                      position_ids=position_ids, pos_offset=pos_offset, causal=causal,
                                      key_lens=key_lens, bias=bias)
            return self.o_proj(o.transpose(1, 2).reshape(B, S, H * D))

        if ragged:
            return self._ragged_decode(q4, k4, v4, position_ids, kv_cache, cos, sin, qw, kw, eps)
        kv_cache.reserve(B, Hkv, past + S, D, k.dtype, k.device)
        kc, vc = kv_cache.storage()
        if S == 1 and attention_mask is None:
            # one launch pair: the new K-hat/V row is built, written to row
            # `past` and attended inside the decode kernel (the storage is a
            # pool of B pages of `capacity` rows); positions as the row kernel
            # path: position_ids (any shape broadcasting to (B, 1)), else pos_offset
            lens, lens_next = kv_cache._step_lengths()
            o = ops.attention_decode_paged(q4, kc, vc, kv_cache._identity_table(), lens,
                                           max_len=past + 1, k_new=k4, v_new=v4, k_weight=kw,
                                           lens_out=lens_next, q_weight=qw, eps=eps, cos=cos,
                                           sin=sin, q_pos=position_ids, q_pos0=pos_offset)
            kv_cache._step_done()
            return self.o_proj(o.reshape(B, 1, H * D))
        ops.qk_norm_rope(k=k4, v=v4, k_out=kc, v_out=vc, k_weight=kw, eps=eps, cos=cos, sin=sin,
                         position_ids=position_ids, pos_offset=pos_offset, kv_row_offset=past)
        kv_cache.advance(S)
        o = ops.attention_prefill(q4, kc[:, :, :T], vc[:, :, :T], q_weight=qw, eps=eps, cos=cos,
                                  sin=sin, position_ids=position_ids, pos_offset=pos_offset,
                                  causal=causal, key_lens=key_lens, bias=bias)
        return self.o_proj(o.transpose(1, 2).reshape(B, S, H * D))

    def _ragged_decode(self, q4, k4, v4, position_ids, kv_cache, cos, sin, qw, kw, eps):
        """One token per row against a ragged cache (see ``KVCache``)."""
        B, H, S, D = q4.shape
        if S != 1:
            raise NotImplementedError("a ragged cache takes one token per row per step")
        Hkv = k4.shape[1]
        if position_ids is None:
            # the new rows sit at positions lens[b] <= seq_len
            ops.check_position_span(0, kv_cache.seq_len + 1, self.rotary_emb.max_position_embeddings)
        kv_cache.reserve(B, Hkv, kv_cache.seq_len + 1, D, k4.dtype, k4.device)
        kc, vc = kv_cache.storage()
        kv_cache.advance(1)
        # the dense storage is a pool of B pages of capacity rows each; one
        # launch appends K-hat/V at row lens[b], attends lens[b] + 1 keys and
        # writes lens + 1 into the spare lengths buffer
        lens, lens_next = kv_cache.lens, kv_cache._spare_lens()
        qp = position_ids
        o = ops.attention_decode_paged(q4, kc, vc, kv_cache._identity_table(), lens,
                                       max_len=kv_cache.seq_len, k_new=k4, v_new=v4, k_weight=kw,
                                       lens_out=lens_next, q_weight=qw, eps=eps, cos=cos, sin=sin,
                                       q_pos=qp, q_pos0=-1)
        kv_cache.lens = lens_next
        kv_cache._lens_spare = lens
        return self.o_proj(o.reshape(B, 1, H * D))

    def _paged_forward(self, q4, k4, v4, position_ids, cache, cos, sin, qw, kw, eps):
        """Prefill into / decode against a PagedKVCache (causal, true positions)."""
        B, H, S, D = q4.shape
        Hkv = k4.shape[1]
        cache._setup(B, Hkv, D, k4.dtype, k4.device)
        past = list(cache.host_lens)
        new = [n + S for n in past]
        if position_ids is None:  # positions continue from each sequence's length
            ops.check_position_span(0, max(new), self.rotary_emb.max_position_embeddings)
        cache._grow(new)
        if S == 1:
            lens, lens_next = cache.lens, cache._spare_lens()
            qp = position_ids
            o = ops.attention_decode_paged(q4, cache.k_pool, cache.v_pool, cache.block_table, lens,
                                           max_len=max(new), k_new=k4, v_new=v4, k_weight=kw,
                                           lens_out=lens_next, q_weight=qw, eps=eps, cos=cos, sin=sin,
                                           q_pos=qp, q_pos0=-1)
            cache.lens, cache._lens_spare = lens_next, lens
            cache.host_lens = new
            return self.o_proj(o.reshape(B, 1, H * D))
        if len(set(past)) != 1:
            raise NotImplementedError("a multi-token forward into a PagedKVCache needs every sequence "
                                      "at the same length")
        p0 = past[0]
        pos = {"position_ids": position_ids} if position_ids is not None else {"pos_offset": p0}
        # the chunk's K-hat (QK-Norm + RoPE fused) and V rows go into their
        # pages, then its queries attend all p0 + S keys through the block
        # table: no dense copy of the cache
        ops.kv_append_paged(k4, v4, cache.k_pool, cache.v_pool, cache.block_table, k_weight=kw,
                            eps=eps, cos=cos, sin=sin, row_offset=p0, **pos)
        o = ops.attention_prefill_paged(q4, cache.k_pool, cache.v_pool, cache.block_table, T=p0 + S,
                                        q_weight=qw, eps=eps, cos=cos, sin=sin, causal=True, **pos)
        cache.lens.add_(S)
        cache.host_lens = new
        return self.o_proj(o.transpose(1, 2).reshape(B, S, H * D))
