"""CPU restatement of nano-qwen's GQA attention path -- TEST INFRASTRUCTURE ONLY.

This module is the oracle the HIP kernels are checked against.  It is imported
only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg; the product package never imports it.

Every function restates one piece of the reference (paths relative to the
nano-qwen source tree) in plain torch CPU arithmetic: explicit matmul +
softmax, no ``scaled_dot_product_attention`` and no fused kernels, so that the
library routine the reference calls can itself be used as an independent check
in the tests.

Pinning status (what checks each function, see tests/test_oracle_*.py):
  * rms_norm          -- golden vectors from the reference (fp32 and bf16 cast
                         order), closed form w=1, scale invariance.
  * rope_inv_freq /
    yarn_inv_freq /
    rope_tables       -- golden table rows from the reference (plain and YaRN,
                         incl. positions 32767/32768/131071), YaRN closed-form
                         correction range (low=23, high=40 at D=128, theta=1e6,
                         L0=32768), factor 1 == plain RoPE.
  * rotate_half       -- position 0 is the identity, pair norms preserved,
                         relative-position property, D=2 textbook rotation.
  * attention         -- fp64 brute force (pure-Python loops) on tiny inputs,
                         torch SDPA (the routine the reference calls) in fp64,
                         special cases (S=1, constant scores, causal row 0).
  * attention_path /
    attention_module_forward / OracleKVCache
                      -- golden vectors from the reference's own
                         Attention.forward (no cache, position_ids, KVCache
                         prefill + decode protocol, bf16 module).
  * decode_path       -- equals the last row of a causal prefill over the same
                         keys; ragged rows equal their B=1 slices.
  * reference_path_sdpa -- the reference's composition with torch SDPA (the
                         CPU baseline's timed routine): equals attention_path
                         (golden-pinned) on seeded inputs, causal and not,
                         S == T and S < T.
  * reference_decode_sdpa -- the reference's decode step with SDPA (the
                         decode CPU baseline): equals decode_path over the
                         grown cache, and its appended row is the k-hat of
                         attention_path at that position.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

__all__ = [
    "rms_norm",
    "rope_inv_freq",
    "yarn_correction_range",
    "yarn_inv_freq",
    "rope_tables",
    "rotate_half",
    "attention",
    "attention_path",
    "reference_path_sdpa",
    "reference_decode_sdpa",
    "decode_path",
    "attention_module_forward",
    "OracleKVCache",
]


# ---------------------------------------------------------------------------
# QK-Norm  (model/norm.py:17-22)
# ---------------------------------------------------------------------------

def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float = 1e-6,
             compute_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """RMSNorm over the last dim, following model/norm.py:17-22.

    ``y = (x_c * rsqrt(mean(x_c^2) + eps)).to(x.dtype) * w`` with x_c the input
    upcast to ``compute_dtype`` (fp32 in the reference).  The cast back to the
    input dtype happens BEFORE the weight multiply (norm.py:21-22), so an fp32
    weight promotes a bf16 input to fp32.
    """
    xc = x.to(compute_dtype)
    y = xc * torch.rsqrt(xc.pow(2).mean(-1, keepdim=True) + eps)
    y = y.to(x.dtype)
    if weight is None:
        return y
    return y * weight


# ---------------------------------------------------------------------------
# RoPE tables, plain and YaRN  (model/rope.py:17-107)
# ---------------------------------------------------------------------------

def rope_inv_freq(dim: int, theta: float) -> torch.Tensor:
    """Plain RoPE inverse frequencies in fp32 (model/rope.py:25)."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))


def yarn_correction_range(dim: int, theta: float, original_max: int,
                          beta_fast: float = 32.0, beta_slow: float = 1.0) -> Tuple[int, int]:
    """YaRN correction range (model/rope.py:31-43).

    The dim index at which ``num_rot`` full rotations happen over
    ``original_max`` positions is ``dim*ln(L0/(2*pi*num_rot)) / (2*ln(theta))``;
    low uses floor at beta_fast, high uses ceil at beta_slow, clamped to
    [0, dim-1].
    """
    def corr(num_rot: float) -> float:
        return (dim * math.log(original_max / (num_rot * 2 * math.pi))) / (2 * math.log(theta))

    low = math.floor(corr(beta_fast))
    high = math.ceil(corr(beta_slow))
    return max(low, 0), min(high, dim - 1)


def yarn_inv_freq(dim: int, theta: float, factor: float, original_max: int) -> torch.Tensor:
    """YaRN-blended inverse frequencies in fp32 (model/rope.py:46-75).

    Fixed beta_fast=32, beta_slow=1 and NO attention-temperature (mscale)
    factor, as in the reference (rope.py:58-59, 98-100).
    """
    expo = torch.arange(0, dim, 2, dtype=torch.float32) / dim
    freq_extra = 1.0 / (theta ** expo)
    freq_inter = 1.0 / (factor * theta ** expo)
    low, high = yarn_correction_range(dim, theta, original_max)
    hi = float(high)
    if low == high:
        hi += 0.001
    ramp = ((torch.arange(dim // 2, dtype=torch.float32) - low) / (hi - low)).clamp(0, 1)
    extrap_mask = 1.0 - ramp
    return freq_inter * (1 - extrap_mask) + freq_extra * extrap_mask


def rope_tables(dim: int, max_pos: int, theta: float,
                rope_scaling: Optional[dict] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin tables of shape (max_pos, dim/2) (model/rope.py:81-107).

    YaRN is selected only by ``rope_scaling["type"] == "yarn"``, with defaults
    factor 4.0 and original_max_position_embeddings 32768 (rope.py:95-100).
    """
    if rope_scaling is not None and rope_scaling.get("type") == "yarn":
        inv = yarn_inv_freq(dim, theta, rope_scaling.get("factor", 4.0),
                            rope_scaling.get("original_max_position_embeddings", 32768))
    else:
        inv = rope_inv_freq(dim, theta)
    t = torch.arange(max_pos, dtype=torch.float32)
    freqs = torch.outer(t, inv)
    return freqs.cos(), freqs.sin()


def rotate_half(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half (NeoX) RoPE on the last dim (model/rope.py:144-159).

    ``cos``/``sin`` must already broadcast against ``x[..., :D/2]``; the pair is
    ``(i, i + D/2)``: ``[x1*c - x2*s, x2*c + x1*s]``.
    """
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


# ---------------------------------------------------------------------------
# Attention arithmetic  (model/attention.py:105-115 + SDPA semantics)
# ---------------------------------------------------------------------------

def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
              causal: bool = False, causal_offset: int = 0,
              mask: Optional[torch.Tensor] = None,
              scale: Optional[float] = None,
              key_lens: Optional[torch.Tensor] = None,
              compute_dtype: torch.dtype = torch.float32,
              q_block: int = 512) -> torch.Tensor:
    """softmax(q k^T * scale + mask) v for GQA inputs, in ``compute_dtype``.

    q: (B, Hq, S, D); k, v: (B, Hkv, T, D); Hq % Hkv == 0 and q head h reads
    kv head h // (Hq/Hkv) -- the ``repeat_interleave`` of attention.py:106-108.
    Scale defaults to 1/sqrt(D), SDPA's default, since attention.py:110 passes
    none.  ``causal`` keeps key j for query i iff j <= i + causal_offset
    (offset 0 is SDPA's is_causal, used by the reference only with S == T).
    ``mask`` follows SDPA: bool True = keep, float = additive; it broadcasts to
    (B, Hq, S, T).  ``key_lens`` (B,) hides keys j >= key_lens[b] (ragged
    caches).  Queries are processed in blocks of ``q_block`` rows to bound
    memory at long sequence lengths.  Returns (B, Hq, S, D) in compute_dtype.
    """
    B, Hq, S, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    assert Hq % Hkv == 0
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    qc, kc, vc = (t.to(compute_dtype) for t in (q, k, v))
    kc = kc.repeat_interleave(G, dim=1)
    vc = vc.repeat_interleave(G, dim=1)
    out = torch.empty(B, Hq, S, D, dtype=compute_dtype)
    kidx = torch.arange(T)
    for s0 in range(0, S, q_block):
        s1 = min(S, s0 + q_block)
        sc = torch.matmul(qc[:, :, s0:s1], kc.transpose(-1, -2)) * scale
        keep = torch.ones(s1 - s0, T, dtype=torch.bool)
        if causal:
            qidx = torch.arange(s0, s1)
            keep = kidx[None, :] <= (qidx[:, None] + causal_offset)
        keep = keep[None, None].expand(B, Hq, s1 - s0, T)
        if key_lens is not None:
            keep = keep & (kidx[None, None, None, :] < key_lens.view(B, 1, 1, 1))
        if mask is not None:
            mb = mask[..., s0:s1, :] if mask.dim() >= 2 and mask.shape[-2] == S else mask
            if mb.dtype == torch.bool:
                keep = keep & mb
            else:
                sc = sc + mb.to(compute_dtype)
        sc = sc.masked_fill(~keep, float("-inf"))
        # a row with every key masked (all scores -inf) attends nothing: zeros,
        # as torch's SDPA returns (softmax alone would give NaN); its scores are
        # made finite first so that no NaN reaches autograd either
        none = torch.isneginf(sc).all(-1, keepdim=True)
        p = torch.softmax(sc.masked_fill(none, 0.0), dim=-1).masked_fill(none, 0.0)
        out[:, :, s0:s1] = torch.matmul(p, vc)
    return out


def _gather_table(tab: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """Rows ``tab[pos]`` shaped to broadcast over (B, H, S, D/2) (rope.py:123-130, 149-154)."""
    rows = tab[pos.long()]            # (S, D/2) or (B, S, D/2)
    if rows.dim() == 2:
        return rows[None, None]
    return rows[:, None]


def attention_path(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                   q_weight: Optional[torch.Tensor], k_weight: Optional[torch.Tensor],
                   eps: float, cos: torch.Tensor, sin: torch.Tensor,
                   q_pos: torch.Tensor, k_pos: Optional[torch.Tensor] = None,
                   causal: bool = True, causal_offset: int = 0,
                   scale: Optional[float] = None,
                   compute_dtype: torch.dtype = torch.float32,
                   return_khat: bool = False, q_block: int = 512):
    """The post-projection part of Attention.forward (model/attention.py:95-115).

    q: (B, Hq, S, D), k/v: (B, Hkv, T, D) pre-norm projections; QK-Norm
    (weights may be None to skip it, the ``qk_norm=False`` branch), then
    rotate-half RoPE from the fp32 tables at ``q_pos``/``k_pos`` ((S,) or
    (B, S) int), then GQA attention.  All arithmetic is done in
    ``compute_dtype`` from the inputs' values (the "reference run in fp32" the
    kernels are held to).  Returns o (B, Hq, S, D) and optionally k-hat.
    """
    if k_pos is None:
        k_pos = q_pos
    qc, kc = q.to(compute_dtype), k.to(compute_dtype)
    if q_weight is not None:
        qc = rms_norm(qc, q_weight.to(compute_dtype), eps, compute_dtype)
    if k_weight is not None:
        kc = rms_norm(kc, k_weight.to(compute_dtype), eps, compute_dtype)
    ct, st = cos.to(compute_dtype), sin.to(compute_dtype)
    qh = rotate_half(qc, _gather_table(ct, q_pos), _gather_table(st, q_pos))
    kh = rotate_half(kc, _gather_table(ct, k_pos), _gather_table(st, k_pos))
    o = attention(qh, kh, v, causal=causal, causal_offset=causal_offset, scale=scale,
                  compute_dtype=compute_dtype, q_block=q_block)
    return (o, kh) if return_khat else o


def reference_path_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                        q_weight: Optional[torch.Tensor], k_weight: Optional[torch.Tensor],
                        eps: float, cos: torch.Tensor, sin: torch.Tensor,
                        q_pos: torch.Tensor, k_pos: Optional[torch.Tensor] = None,
                        causal: bool = True) -> torch.Tensor:
    """The reference's own composition of the post-projection path, as the CPU
    baseline times it: QK-Norm (norm.py:17-22), rotate-half RoPE from the fp32
    tables (rope.py:133-161), ``repeat_interleave`` of the KV heads
    (attention.py:105-108) and ``F.scaled_dot_product_attention``
    (attention.py:110-115), all in the inputs' dtype.  Causal with S < T is
    bottom-right aligned (an explicit mask, since SDPA's is_causal is
    top-left).  Pinned against ``attention_path`` in the oracle tests.
    """
    import torch.nn.functional as F
    if k_pos is None:
        k_pos = q_pos
    if q_weight is not None:
        q = rms_norm(q, q_weight, eps)
    if k_weight is not None:
        k = rms_norm(k, k_weight, eps)
    q = rotate_half(q, _gather_table(cos, q_pos), _gather_table(sin, q_pos))
    k = rotate_half(k, _gather_table(cos, k_pos), _gather_table(sin, k_pos))
    G = q.shape[1] // k.shape[1]
    if G > 1:
        k = k.repeat_interleave(G, dim=1)
        v = v.repeat_interleave(G, dim=1)
    S, T = q.shape[2], k.shape[2]
    if causal and S != T:
        keep = torch.ones(S, T, dtype=torch.bool).tril(T - S)
        return F.scaled_dot_product_attention(q, k, v, attn_mask=keep)
    return F.scaled_dot_product_attention(q, k, v, is_causal=causal)


def reference_decode_sdpa(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                          k_cache: torch.Tensor, v_cache: torch.Tensor, *,
                          q_weight: Optional[torch.Tensor], k_weight: Optional[torch.Tensor],
                          eps: float, cos: torch.Tensor, sin: torch.Tensor,
                          repeat_kv: bool = True):
    """One decode step of the reference, as the CPU baseline times it, for one
    sequence: QK-Norm and RoPE of the new token at position ``T - 1``
    (attention.py:95-100), the cache's concatenation (KVCache.update,
    attention.py:35-44), ``repeat_interleave`` (attention.py:105-108) and SDPA
    with no mask (attention.py:110-115).

    q: (1, Hq, 1, D), k_new/v_new: (1, Hkv, 1, D) pre-norm projections;
    k_cache/v_cache: (1, Hkv, T - 1, D) holding earlier K-hat and V.  Returns
    (o (1, Hq, 1, D), k_all, v_all) with the grown cache.  Pinned against
    ``decode_path`` in the oracle tests.  ``repeat_kv=False`` lets SDPA group
    the heads itself (``enable_gqa``) instead of materialising the repeated
    cache: the same function without the reference's copy.
    """
    import torch.nn.functional as F
    pos = torch.tensor([k_cache.shape[2]])
    if q_weight is not None:
        q = rms_norm(q, q_weight, eps)
    if k_weight is not None:
        k_new = rms_norm(k_new, k_weight, eps)
    c, s_ = _gather_table(cos, pos), _gather_table(sin, pos)
    q, k_new = rotate_half(q, c, s_), rotate_half(k_new, c, s_)
    k_all = torch.cat([k_cache, k_new], dim=2)
    v_all = torch.cat([v_cache, v_new], dim=2)
    G = q.shape[1] // k_all.shape[1]
    k, v = k_all, v_all
    if G > 1 and not repeat_kv:
        return F.scaled_dot_product_attention(q, k, v, enable_gqa=True), k_all, v_all
    if G > 1:
        k = k.repeat_interleave(G, dim=1)
        v = v.repeat_interleave(G, dim=1)
    return F.scaled_dot_product_attention(q, k, v), k_all, v_all


def reference_chunk_sdpa(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                         k_cache: torch.Tensor, v_cache: torch.Tensor, *,
                         q_weight: Optional[torch.Tensor], k_weight: Optional[torch.Tensor],
                         eps: float, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """A prompt continuation in the reference's composition, as the CPU baseline
    times it: the chunk's S new tokens sit at positions T0 .. T0+S-1 (T0 =
    k_cache.shape[2], the rows already cached as K-hat and V); QK-Norm and RoPE
    of the chunk's q and k (attention.py:95-100), KVCache.update's
    concatenation (attention.py:35-44), ``repeat_interleave``
    (attention.py:105-108) and SDPA (attention.py:110-115) with the
    bottom-right causal mask of true positions (the reference passes none with
    a cache, quirk Q8; the build's chunked prefill is causal).  Pinned against
    ``attention_path`` in the oracle tests.
    """
    import torch.nn.functional as F
    T0, S = k_cache.shape[2], q.shape[2]
    pos = torch.arange(T0, T0 + S)
    if q_weight is not None:
        q = rms_norm(q, q_weight, eps)
    if k_weight is not None:
        k_new = rms_norm(k_new, k_weight, eps)
    c, s_ = _gather_table(cos, pos), _gather_table(sin, pos)
    q, k_new = rotate_half(q, c, s_), rotate_half(k_new, c, s_)
    k = torch.cat([k_cache, k_new], dim=2)
    v = torch.cat([v_cache, v_new], dim=2)
    G = q.shape[1] // k.shape[1]
    if G > 1:
        k = k.repeat_interleave(G, dim=1)
        v = v.repeat_interleave(G, dim=1)
    keep = torch.ones(S, T0 + S, dtype=torch.bool).tril(T0)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=keep)


def decode_path(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                lens: torch.Tensor, *, q_weight: Optional[torch.Tensor], eps: float,
                cos: torch.Tensor, sin: torch.Tensor, q_pos: torch.Tensor,
                scale: Optional[float] = None,
                compute_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Single-token decode against a ragged cache (attention.py:95-115 at S=1).

    q: (B, Hq, D) pre-norm; k_cache/v_cache: (B, Hkv, Tcap, D) holding
    post-norm post-RoPE K and raw V (attention.py:99-103); lens: (B,) valid
    rows per batch entry; q_pos: (B,) position of the query token.  Each row
    attends keys [0, lens[b]) with no causal mask (attention.py:113 passes
    is_causal=False whenever a cache is present).  Rows are computed one at a
    time on their own length so that padded cache rows are never read.
    Returns (B, Hq, D).
    """
    B, Hq, D = q.shape
    out = torch.empty(B, Hq, D, dtype=compute_dtype)
    qc = q.to(compute_dtype)
    if q_weight is not None:
        qc = rms_norm(qc, q_weight.to(compute_dtype), eps, compute_dtype)
    ct, st = cos.to(compute_dtype), sin.to(compute_dtype)
    for b in range(B):
        p = int(q_pos[b])
        qh = rotate_half(qc[b], ct[p], st[p])                       # (Hq, D)
        L = int(lens[b])
        kb = k_cache[b:b + 1, :, :L]
        vb = v_cache[b:b + 1, :, :L]
        out[b] = attention(qh[None, :, None, :], kb, vb, scale=scale,
                           compute_dtype=compute_dtype)[0, :, 0]
    return out


# ---------------------------------------------------------------------------
# Whole Attention.forward with the reference's dtype flow (golden comparisons)
# ---------------------------------------------------------------------------

class OracleKVCache:
    """The reference KVCache (model/attention.py:24-46): grows by concatenation."""

    def __init__(self):
        self.key = None
        self.value = None

    def update(self, key, value):
        if self.key is None:
            self.key, self.value = key, value
        else:
            self.key = torch.cat([self.key, key], dim=2)
            self.value = torch.cat([self.value, value], dim=2)
        return self.key, self.value

    @property
    def seq_len(self) -> int:
        return 0 if self.key is None else self.key.shape[2]


def attention_module_forward(hidden: torch.Tensor, weights: dict, *, num_heads: int,
                             num_kv_heads: int, head_dim: int, eps: float,
                             cos_table: torch.Tensor, sin_table: torch.Tensor,
                             position_ids: Optional[torch.Tensor] = None,
                             attention_mask: Optional[torch.Tensor] = None,
                             kv_cache: Optional[OracleKVCache] = None,
                             qk_norm: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention.forward (model/attention.py:82-118) with the reference's dtype flow.

    ``weights`` holds q_proj/k_proj/v_proj/o_proj weight matrices (no bias,
    config.attention_bias=False) and q_norm/k_norm weights, all in the module
    dtype.  Ops run in the dtype the reference runs them in: projections and
    RoPE in the activation dtype, the norm statistic in fp32 then cast back
    before the weight multiply (norm.py:21-22), cos/sin cast to the activation
    dtype (rope.py:125-129).  The softmax/attention itself is evaluated in
    fp32 from the (possibly bf16) operands and cast back to the activation
    dtype.  Returns (output (B,S,hidden), attention output before o_proj
    (B,S,Hq*D)).
    """
    B, S, _ = hidden.shape
    dt = hidden.dtype
    q = (hidden @ weights["q_proj"].t()).view(B, S, num_heads, head_dim).transpose(1, 2)
    k = (hidden @ weights["k_proj"].t()).view(B, S, num_kv_heads, head_dim).transpose(1, 2)
    v = (hidden @ weights["v_proj"].t()).view(B, S, num_kv_heads, head_dim).transpose(1, 2)
    if qk_norm:
        q = rms_norm(q, weights["q_norm"], eps)
        k = rms_norm(k, weights["k_norm"], eps)
    if position_ids is None:
        cos = cos_table[:S].to(q.dtype)[None, None]
        sin = sin_table[:S].to(q.dtype)[None, None]
    else:
        cos = cos_table[position_ids].to(q.dtype)[:, None]
        sin = sin_table[position_ids].to(q.dtype)[:, None]
    q = rotate_half(q, cos, sin)
    k = rotate_half(k, cos, sin)
    if kv_cache is not None:
        k, v = kv_cache.update(k, v)
    causal = attention_mask is None and kv_cache is None
    o = attention(q, k, v, causal=causal, mask=attention_mask,
                  compute_dtype=torch.float32).to(q.dtype)
    attn = o.transpose(1, 2).contiguous().view(B, S, -1)
    out = attn @ weights["o_proj"].t().to(attn.dtype)
    return out, attn
