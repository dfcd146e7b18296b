"""torch-facing wrappers over the gfx950 attention kernels (libnqattn.so).

Tensors are passed to the C ABI as raw device pointers plus element strides;
the kernels never allocate.  Every function here requires HIP device tensors
and raises if the library is missing -- there is no CPU or eager fallback.

Mirrors of the reference's kernel-level API (kernels/flash_attn.py:130-143,
kernels/rope.py:99-108) keep their names and argument meaning:
``flash_attention(q, k, v, causal=True, sm_scale=None)`` and
``apply_rope(q, k, cos, sin)`` (in place).  The fused entry points used by the
drop-in ``Attention`` module are ``qk_norm_rope``, ``attention_prefill`` and
``attention_decode``.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib

__all__ = [
    "KernelCall",
    "qk_norm_rope",
    "AttnBias",
    "attention_prefill",
    "attention_prefill_paged",
    "attention_decode",
    "attention_decode_paged",
    "kv_append_paged",
    "attention_merge_",
    "attention_backward",
    "qk_norm_rope_backward",
    "decode_workspace_bytes",
    "flash_attention",
    "apply_rope",
]

_DTYPES = {torch.bfloat16: _lib.NQ_DTYPE_BF16, torch.float32: _lib.NQ_DTYPE_F32}


def _code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; the kernels take bfloat16 or float32") from None


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require_device(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("nano_qwen_amd attention kernels need HIP device tensors "
                               f"(got a tensor on {t.device}); there is no CPU path")


def _aligned(t: torch.Tensor) -> bool:
    es = t.element_size()
    if t.data_ptr() % 16:
        return False
    if t.stride(-1) != 1:
        return False
    return all((s * es) % 16 == 0 for s in t.stride()[:-1])


def _rows_in(t: torch.Tensor) -> torch.Tensor:
    """An input operand the kernels can read: last dim contiguous, 16-byte aligned rows."""
    return t if _aligned(t) else t.contiguous()


def _rows_out(t: torch.Tensor, name: str) -> torch.Tensor:
    if not _aligned(t):
        raise ValueError(f"{name}: output rows must be contiguous in the last dim and 16-byte aligned")
    return t


def _f32(t: Optional[torch.Tensor], device) -> Optional[torch.Tensor]:
    if t is None:
        return None
    if (t.dtype != torch.float32 or t.device != device or not t.is_contiguous()
            or t.data_ptr() % 16):  # the kernels DMA weights and table rows in 16-byte pieces
        t = t.to(device=device, dtype=torch.float32).contiguous()
        if t.data_ptr() % 16:
            t = t.clone()
    return t


def _i32(t: Optional[torch.Tensor], device) -> Optional[torch.Tensor]:
    if t is None:
        return None
    if t.dtype != torch.int32 or t.device != device or not t.is_contiguous():
        t = t.to(device=device, dtype=torch.int32).contiguous()
    return t


def _key_lens(key_lens: Optional[torch.Tensor], B: int, device) -> Optional[torch.Tensor]:
    """int32 (B,) per-sequence key counts on the device, or None."""
    if key_lens is None:
        return None
    kl = _i32(key_lens.reshape(-1), device)
    if kl.numel() != B:
        raise ValueError(f"key_lens must hold one count per sequence ({B}), got {kl.numel()}")
    return kl


def _tables(cos, sin, device):
    if cos is None:
        return None, None, 0
    c, s = _f32(cos, device), _f32(sin, device)
    if c.dim() != 2 or c.shape != s.shape:
        raise ValueError("cos/sin tables must both be (max_pos, head_dim/2)")
    return c, s, c.shape[0]


def _range_error(lo: int, hi: int, max_pos: int) -> IndexError:
    return IndexError(f"positions {lo}..{hi} lie outside the RoPE table of {max_pos} positions "
                      "(max_position_embeddings)")


def check_position_span(first: int, count: int, max_pos: int) -> None:
    """Raise IndexError unless positions first .. first+count-1 index the table.

    The reference's table lookup (model/rope.py:123-129) fails on such
    positions; the kernels cannot raise, and rotate a row at an out-of-range
    position with NaN instead.
    """
    if count > 0 and max_pos > 0 and (first < 0 or first + count > max_pos):
        raise _range_error(first, first + count - 1, max_pos)


def _check_host_positions(pos: Optional[torch.Tensor], max_pos: int) -> None:
    """Range check of positions held on the host (a device tensor is not read back)."""
    if pos is None or max_pos <= 0 or pos.is_cuda or pos.numel() == 0:
        return
    lo, hi = int(pos.min()), int(pos.max())
    if lo < 0 or hi >= max_pos:
        raise _range_error(lo, hi, max_pos)


def _positions(position_ids: Optional[torch.Tensor], pos_offset: int, pos_base: Optional[torch.Tensor],
               B: int, S: int, max_pos: int, dev) -> Optional[torch.Tensor]:
    """int32 (B, S) device positions, or None when they follow pos_base / pos_offset.

    Positions the host knows are range-checked here: explicit host
    ``position_ids``, and ``pos_offset .. pos_offset + S - 1``.
    """
    if position_ids is not None:
        _check_host_positions(position_ids, max_pos)
        pos = _i32(position_ids, dev)
        if tuple(pos.shape) != (B, S):
            pos = pos.expand(B, S).contiguous()
        return pos
    if pos_base is None:
        check_position_span(int(pos_offset), S, max_pos)
    return None


class KernelCall:
    """A validated, fully bound call into libnqattn.so.

    Built by the ops below with ``plan=True``: argument checks, output
    allocation and the ctypes argument tuple are done once, so ``launch()``
    is a single foreign call (for serving loops and benchmarks).  It keeps
    every tensor it points at alive.  ``result`` holds what the op returns.
    """

    __slots__ = ("fn", "args", "stream_index", "name", "keep", "result")

    def __init__(self, fn, args, stream_index, name, keep, result):
        self.fn, self.args, self.stream_index = fn, list(args), stream_index
        self.name, self.keep, self.result = name, keep, result

    def launch(self, stream: Optional[torch.cuda.Stream] = None):
        """Run the kernel(s) on ``stream`` (default: the stream current at planning time)."""
        if stream is not None:
            self.args[self.stream_index] = ctypes.c_void_p(stream.cuda_stream)
        _lib.check(self.fn(*self.args), self.name)
        return self.result


# ---------------------------------------------------------------------------
# QK-Norm + RoPE + cache placement
# ---------------------------------------------------------------------------

def qk_norm_rope(q: Optional[torch.Tensor] = None, k: Optional[torch.Tensor] = None,
                 v: Optional[torch.Tensor] = None, *,
                 q_out: Optional[torch.Tensor] = None, k_out: Optional[torch.Tensor] = None,
                 v_out: Optional[torch.Tensor] = None,
                 q_weight: Optional[torch.Tensor] = None, k_weight: Optional[torch.Tensor] = None,
                 eps: float = 1e-6, cos: torch.Tensor, sin: torch.Tensor,
                 position_ids: Optional[torch.Tensor] = None, pos_offset: int = 0,
                 pos_base: Optional[torch.Tensor] = None,
                 kv_row_offset: int = 0, kv_row_base: Optional[torch.Tensor] = None,
                 plan: bool = False):
    """QK-Norm + rotate-half RoPE of Q/K rows and a row copy of V, in one launch.

    q: (B, Hq, S, D), k/v: (B, Hkv, S, D), any (b, h, s) strides.  Outputs
    default to fresh (B, H, S, D) tensors; K/V rows land at row
    ``kv_row_offset + s`` (or ``kv_row_base[b] + s``) of k_out/v_out, which may
    be a preallocated cache (B, Hkv, T_cap, D) -- the append of
    KVCache.update (model/attention.py:31-38).  Positions are
    ``position_ids[b, s]``, else ``pos_base[b] + s``, else ``pos_offset + s``
    (model/rope.py:123-129).  Norm weights None skip the norm.
    Returns (q_out, k_out, v_out), or with ``plan=True`` a KernelCall whose
    ``launch()`` runs it.
    """
    ref = next(t for t in (q, k, v) if t is not None)
    _require_device(q, k, v, q_out, k_out, v_out)
    dev = ref.device
    B, _, S, D = ref.shape
    Hq = q.shape[1] if q is not None else 0
    Hkv = (k if k is not None else v).shape[1] if (k is not None or v is not None) else 0
    dt_in = _code(ref)
    for t in (q, k, v):
        if t is not None and t.dtype != ref.dtype:
            raise TypeError("q, k and v must share one dtype")
    q = _rows_in(q) if q is not None else None
    k = _rows_in(k) if k is not None else None
    v = _rows_in(v) if v is not None else None
    if q is not None and q_out is None:
        q_out = torch.empty(B, Hq, S, D, dtype=ref.dtype, device=dev)
    if k is not None and k_out is None:
        k_out = torch.empty(B, Hkv, S, D, dtype=ref.dtype, device=dev)
    if v is not None and v_out is None:
        v_out = torch.empty(B, Hkv, S, D, dtype=ref.dtype, device=dev)
    outs = [t for t in (q_out, k_out, v_out) if t is not None]
    dt_out = _code(outs[0])
    for t in outs:
        if t.dtype != outs[0].dtype:
            raise TypeError("outputs must share one dtype")
    for name, t in (("q_out", q_out), ("k_out", k_out), ("v_out", v_out)):
        if t is not None:
            _rows_out(t, name)
    for name, src, dst in (("k", k, k_out), ("v", v, v_out)):
        if src is not None and kv_row_base is None and kv_row_offset + S > dst.shape[2]:
            raise ValueError(f"{name}_out has {dst.shape[2]} rows; rows up to {kv_row_offset + S} needed")
    cos_t, sin_t, max_pos = _tables(cos, sin, dev)
    pos = _positions(position_ids, pos_offset, pos_base, B, S, max_pos, dev)
    pb = _i32(pos_base, dev)
    rb = _i32(kv_row_base, dev)
    qw, kw = _f32(q_weight, dev), _f32(k_weight, dev)
    lib = _lib.load()
    st = _lib.strides3
    args = (
        _ptr(q), st(q.stride()[:3]) if q is not None else None,
        _ptr(q_out), st(q_out.stride()[:3]) if q is not None else None,
        _ptr(k), st(k.stride()[:3]) if k is not None else None,
        _ptr(k_out), st(k_out.stride()[:3]) if k is not None else None,
        _ptr(v), st(v.stride()[:3]) if v is not None else None,
        _ptr(v_out), st(v_out.stride()[:3]) if v is not None else None,
        B, S, max(Hq, 1), max(Hkv, 1), D, dt_in, dt_out,
        _ptr(qw), _ptr(kw), float(eps),
        _ptr(cos_t), _ptr(sin_t), max_pos,
        _ptr(pos), _ptr(pb), int(pos_offset), _ptr(rb), int(kv_row_offset), _stream(ref))
    call = KernelCall(lib.nq_qk_norm_rope, args, len(args) - 1, "nq_qk_norm_rope",
                      (q, k, v, cos_t, sin_t, pos, pb, rb, qw, kw), (q_out, k_out, v_out))
    return call if plan else call.launch()


# ---------------------------------------------------------------------------
# Prefill
# ---------------------------------------------------------------------------

class AttnBias:
    """SDPA's ``attn_mask`` in the form the kernels read: an additive bias.

    model/attention.py:110-113 hands ``attention_mask`` to SDPA, which takes a
    bool keep-mask (True = attend) or a float mask added to the scores, either
    broadcastable to (B, Hq, S, T).  Here a bool mask becomes 0 / -inf and a
    float mask keeps its values, in the kernels' element type.  ``bias`` keeps
    the mask's broadcast batch / head / query axes (stride 0) and materialises
    the key axis, padded to a multiple of 8 keys (the kernels read 8 keys at a
    time); ``bias_t`` (built when ``transpose``) holds the transpose
    (B|1, Hq|1, T, S padded to 8) for the backward's dK/dV kernel, whose lanes
    hold keys.  A row whose keys are all masked gives zeros (and LSE -inf), as
    SDPA does.
    """

    def __init__(self, mask: torch.Tensor, B: int, Hq: int, S: int, T: int, dtype: torch.dtype, device,
                 transpose: bool = False):
        if mask.dim() > 4 or mask.dim() == 0:
            raise ValueError(f"attn_mask must have 1 to 4 dims, got shape {tuple(mask.shape)}")
        m = mask.reshape((1,) * (4 - mask.dim()) + tuple(mask.shape))  # SDPA's broadcast alignment
        for got, want, name in zip(m.shape, (B, Hq, S, T), ("batch", "heads", "queries", "keys")):
            if got not in (1, want):
                raise ValueError(f"attn_mask of shape {tuple(mask.shape)} does not broadcast to "
                                 f"(B, Hq, S, T) = {(B, Hq, S, T)} on the {name} axis")
        m = m.to(device)
        if m.dtype == torch.bool:
            add = torch.zeros(m.shape, dtype=dtype, device=device).masked_fill_(~m, float("-inf"))
        elif m.is_floating_point():
            add = m.to(dtype)
        else:
            raise TypeError(f"attn_mask must be bool or floating point, got {m.dtype}")
        Bm, Hm, Sm = add.shape[:3]
        self.shape = (B, Hq, S, T)
        self.bias = torch.zeros(Bm, Hm, Sm, -(-T // 8) * 8, dtype=dtype, device=device)
        self.bias[..., :T] = add
        self.strides = self._strides(self.bias, (Bm, Hm, Sm))
        self.bias_t, self.t_strides = None, None
        if transpose:
            self.bias_t = torch.zeros(Bm, Hm, T, -(-S // 8) * 8, dtype=dtype, device=device)
            self.bias_t[..., :S] = add.expand(Bm, Hm, S, T).transpose(-1, -2)
            self.t_strides = self._strides(self.bias_t, (Bm, Hm, T))

    @staticmethod
    def _strides(t: torch.Tensor, sizes):
        return tuple(t.stride(i) if sizes[i] > 1 else 0 for i in range(3))


def attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                      q_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                      cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                      position_ids: Optional[torch.Tensor] = None, pos_offset: int = 0,
                      pos_base: Optional[torch.Tensor] = None,
                      causal: bool = True, sm_scale: Optional[float] = None,
                      key_lens: Optional[torch.Tensor] = None,
                      bias: Optional[AttnBias] = None,
                      out: Optional[torch.Tensor] = None, return_lse: bool = False,
                      plan: bool = False):
    """GQA prefill attention with QK-Norm + RoPE of Q fused into its load.

    q: (B, Hq, S, D) pre-norm queries (norm/rope skipped when q_weight / cos
    are None); k: (B, Hkv, T, D) keys as stored (already normed and rotated);
    v: (B, Hkv, T, D).  ``causal`` keeps key j for query i iff j <= i + T - S.
    ``key_lens`` (int, (B,)) limits sequence b to keys [0, key_lens[b]): key
    padding.  ``bias`` (an ``AttnBias``) adds SDPA's general attn_mask to the
    scores.  Returns o shaped (B, Hq, S, D); by default it is a transposed view of a
    contiguous (B, S, Hq, D) buffer, so ``o.transpose(1, 2).reshape(B, S, -1)``
    (o_proj's input, model/attention.py:117) costs nothing.  With
    ``return_lse`` also returns the fp32 (B, Hq, S) log-sum-exp.  With
    ``plan=True`` returns a KernelCall whose ``launch()`` runs it.
    """
    _require_device(q, k, v, out)
    B, Hq, S, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    if k.shape != v.shape or k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"k {tuple(k.shape)} / v {tuple(v.shape)} do not match q {tuple(q.shape)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError("q, k and v must share one dtype")
    dt = _code(q)
    q, k, v = _rows_in(q), _rows_in(k), _rows_in(v)
    if out is None:
        out = torch.empty(B, S, Hq, D, dtype=q.dtype, device=q.device).transpose(1, 2)
    elif tuple(out.shape) != (B, Hq, S, D) or out.dtype != q.dtype:
        raise ValueError(f"out must be (B, Hq, S, D) = {(B, Hq, S, D)} in {q.dtype}")
    _rows_out(out, "out")
    lse = torch.empty(B, Hq, S, dtype=torch.float32, device=q.device) if return_lse else None
    dev = q.device
    kl = _key_lens(key_lens, B, dev)
    cos_t, sin_t, max_pos = _tables(cos, sin, dev)
    pos = _positions(position_ids, pos_offset, pos_base, B, S, max_pos, dev)
    pb = _i32(pos_base, dev)
    qw = _f32(q_weight, dev)
    st = _lib.strides3
    head = (_ptr(q), st(q.stride()[:3]), _ptr(k), st(k.stride()[:3]), _ptr(v), st(v.stride()[:3]),
            _ptr(out), st(out.stride()[:3]), _ptr(lse), _ptr(kl))
    tail = (B, Hq, Hkv, S, T, D, dt, _ptr(qw), float(eps), _ptr(cos_t), _ptr(sin_t), max_pos,
            _ptr(pos), _ptr(pb), int(pos_offset), int(bool(causal)),
            float(sm_scale) if sm_scale is not None else 0.0, _stream(q))
    keep = (q, k, v, cos_t, sin_t, pos, pb, qw, kl)
    if bias is not None:
        _check_bias(bias, B, Hq, S, T, q.dtype)
        args = head + (_ptr(bias.bias), st(bias.strides)) + tail
        call = KernelCall(_lib.load().nq_attn_prefill_bias_fwd, args, len(args) - 1, "nq_attn_prefill_bias_fwd",
                          keep + (bias.bias,), (out, lse) if return_lse else out)
    else:
        args = head + tail
        call = KernelCall(_lib.load().nq_attn_prefill_fwd, args, len(args) - 1, "nq_attn_prefill_fwd",
                          keep, (out, lse) if return_lse else out)
    return call if plan else call.launch()


def _check_bias(bias: AttnBias, B: int, Hq: int, S: int, T: int, dtype: torch.dtype, transpose: bool = False):
    if not isinstance(bias, AttnBias):
        raise TypeError("bias must be an AttnBias (build one from the attn_mask)")
    if bias.shape != (B, Hq, S, T):
        raise ValueError(f"the bias was built for (B, Hq, S, T) = {bias.shape}, the call has {(B, Hq, S, T)}")
    if bias.bias.dtype != dtype:
        raise TypeError(f"the bias holds {bias.bias.dtype}, the call computes in {dtype}")
    if transpose and bias.bias_t is None:
        raise ValueError("the backward needs the bias built with transpose=True")


def attention_prefill_paged(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                            block_table: torch.Tensor, *, T: int,
                            q_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                            cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                            position_ids: Optional[torch.Tensor] = None, pos_offset: int = 0,
                            pos_base: Optional[torch.Tensor] = None,
                            causal: bool = True, sm_scale: Optional[float] = None,
                            out: Optional[torch.Tensor] = None, return_lse: bool = False,
                            plan: bool = False):
    """``attention_prefill`` with K/V read from paged pools through the block table.

    q: (B, Hq, S, D) pre-norm queries of a chunk; k_pool/v_pool:
    (pages, Hkv, page_size, D) holding every sequence's T keys (K-hat and V,
    the chunk's own rows already appended); block_table: (B, pages per
    sequence).  ``causal`` keeps key j for query i iff j <= i + T - S.  This is
    the continuation of a prompt into a ``PagedKVCache`` without a dense copy
    of its pages (the reference concatenates, model/attention.py:31-38).
    """
    _require_device(q, k_pool, v_pool, block_table, out)
    B, Hq, S, D = q.shape
    for name, pool in (("k_pool", k_pool), ("v_pool", v_pool)):
        _pool_check(pool, name)
    if k_pool.shape != v_pool.shape or k_pool.shape[3] != D:
        raise ValueError(f"pools {tuple(k_pool.shape)} / {tuple(v_pool.shape)} do not match q {tuple(q.shape)}")
    if q.dtype != k_pool.dtype or q.dtype != v_pool.dtype:
        raise TypeError("q and the pools must share one dtype")
    Hkv, P = k_pool.shape[1], k_pool.shape[2]
    bt = _block_table(block_table, B, q.device)
    if not 0 < T <= bt.shape[1] * P:
        raise ValueError(f"T={T} must be in [1, {bt.shape[1] * P}] (block-table pages x page_size)")
    dt = _code(q)
    q = _rows_in(q)
    if out is None:
        out = torch.empty(B, S, Hq, D, dtype=q.dtype, device=q.device).transpose(1, 2)
    elif tuple(out.shape) != (B, Hq, S, D) or out.dtype != q.dtype:
        raise ValueError(f"out must be (B, Hq, S, D) = {(B, Hq, S, D)} in {q.dtype}")
    _rows_out(out, "out")
    lse = torch.empty(B, Hq, S, dtype=torch.float32, device=q.device) if return_lse else None
    dev = q.device
    cos_t, sin_t, max_pos = _tables(cos, sin, dev)
    pos = _positions(position_ids, pos_offset, pos_base, B, S, max_pos, dev)
    pb = _i32(pos_base, dev)
    qw = _f32(q_weight, dev)
    st = _lib.strides3
    args = (
        _ptr(q), st(q.stride()[:3]), _ptr(k_pool), st(k_pool.stride()[:3]), _ptr(v_pool),
        st(v_pool.stride()[:3]), _ptr(bt), bt.stride(0), P, _ptr(out), st(out.stride()[:3]), _ptr(lse),
        B, Hq, Hkv, S, int(T), D, dt, _ptr(qw), float(eps), _ptr(cos_t), _ptr(sin_t), max_pos,
        _ptr(pos), _ptr(pb), int(pos_offset), int(bool(causal)),
        float(sm_scale) if sm_scale is not None else 0.0, _stream(q))
    call = KernelCall(_lib.load().nq_attn_prefill_paged_fwd, args, len(args) - 1, "nq_attn_prefill_paged_fwd",
                      (q, k_pool, v_pool, bt, cos_t, sin_t, pos, pb, qw), (out, lse) if return_lse else out)
    return call if plan else call.launch()


# ---------------------------------------------------------------------------
# Decode
# ---------------------------------------------------------------------------

def _decode_q_pos(q_pos: Optional[torch.Tensor], q_pos0: int, B: int, max_pos: int, dev):
    """int32 (B,) query positions from q_pos (any shape broadcastable to (B, 1),
    e.g. position_ids of a one-token step), with the host-known ones range-checked."""
    if q_pos is None:
        if q_pos0 >= 0:
            check_position_span(int(q_pos0), 1, max_pos)
        return None
    _check_host_positions(q_pos, max_pos)
    qp = q_pos.reshape(-1, q_pos.shape[-1])[:, -1] if q_pos.dim() > 1 else q_pos.reshape(-1)
    if qp.numel() == 1 and B > 1:
        qp = qp.expand(B)
    if qp.numel() != B:
        raise ValueError(f"q_pos must give one position per batch row ({B}), got shape {tuple(q_pos.shape)}")
    return _i32(qp, dev)


def decode_workspace_bytes(B: int, Hq: int, Hkv: int, D: int, max_len: int, chunk: int = 0) -> int:
    """Workspace size attention_decode needs for these sizes."""
    return int(_lib.load().nq_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, chunk))


def attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     lens: Optional[torch.Tensor] = None, *, max_len: int,
                     q_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                     cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                     q_pos: Optional[torch.Tensor] = None, q_pos0: int = -1,
                     sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None, chunk: int = 0,
                     plan: bool = False):
    """Single-token GQA decode against a ragged (B, Hkv, T_cap, D) cache.

    q: (B, Hq, D) or (B, Hq, 1, D) pre-norm query; keys [0, lens[b]) of the
    cache are attended (all ``max_len`` rows when lens is None).  The query
    is rotated at q_pos[b], else q_pos0, else lens[b] - 1 (q_pos0 < 0).
    Returns (B, Hq, D), or with ``plan=True`` a KernelCall whose ``launch()``
    runs it.
    """
    _require_device(q, k_cache, v_cache, lens, out)
    if q.dim() == 4:
        q = q[:, :, 0]
    B, Hq, D = q.shape
    Hkv, Tcap = k_cache.shape[1], k_cache.shape[2]
    if k_cache.shape != v_cache.shape or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise ValueError("cache shapes do not match q")
    if not 0 < max_len <= Tcap:
        raise ValueError(f"max_len must be in [1, T_cap={Tcap}], got {max_len}")
    if q.dtype != k_cache.dtype or q.dtype != v_cache.dtype:
        raise TypeError("q and the caches must share one dtype")
    dt = _code(q)
    q = _rows_in(q)
    _rows_out(k_cache, "k_cache")
    _rows_out(v_cache, "v_cache")
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=q.device)
    dev = q.device
    # fp32 caches keep no partials: the library neither needs nor reads a workspace
    need = 0 if q.dtype == torch.float32 else decode_workspace_bytes(B, Hq, Hkv, D, max_len, chunk)
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    wbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    cos_t, sin_t, max_pos = _tables(cos, sin, dev)
    lens_t = _i32(lens, dev)
    qp = _decode_q_pos(q_pos, q_pos0, B, max_pos, dev)
    qw = _f32(q_weight, dev)
    q_str = (ctypes.c_int64 * 2)(q.stride(0), q.stride(1))
    o_str = (ctypes.c_int64 * 2)(out.stride(0), out.stride(1))
    st = _lib.strides3
    args = (
        _ptr(q), q_str, _ptr(k_cache), st(k_cache.stride()[:3]), _ptr(v_cache),
        st(v_cache.stride()[:3]), _ptr(lens_t), _ptr(out), o_str, _ptr(workspace), wbytes,
        B, Hq, Hkv, D, int(max_len), int(chunk), dt, _ptr(qw), float(eps),
        _ptr(cos_t), _ptr(sin_t), max_pos, _ptr(qp), int(q_pos0),
        float(sm_scale) if sm_scale is not None else 0.0, _stream(q))
    call = KernelCall(_lib.load().nq_attn_decode_fwd, args, len(args) - 1, "nq_attn_decode_fwd",
                      (q, k_cache, v_cache, lens_t, workspace, cos_t, sin_t, qp, qw, q_str, o_str), out)
    return call if plan else call.launch()


# ---------------------------------------------------------------------------
# Paged caches
# ---------------------------------------------------------------------------

def _pool_check(pool: torch.Tensor, name: str) -> None:
    if pool.dim() != 4:
        raise ValueError(f"{name} must be (pages, Hkv, page_size, D), got {tuple(pool.shape)}")
    _rows_out(pool, name)


def _block_table(bt: torch.Tensor, B: int, dev) -> torch.Tensor:
    if bt.dim() != 2 or bt.shape[0] != B:
        raise ValueError(f"block_table must be (B={B}, pages per sequence), got {tuple(bt.shape)}")
    bt = _i32(bt, dev)
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    return bt


def kv_append_paged(k: Optional[torch.Tensor], v: Optional[torch.Tensor], k_pool: torch.Tensor,
                    v_pool: torch.Tensor, block_table: torch.Tensor, *,
                    k_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                    cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                    position_ids: Optional[torch.Tensor] = None, pos_offset: int = 0,
                    pos_base: Optional[torch.Tensor] = None,
                    row_offset: int = 0, row_base: Optional[torch.Tensor] = None,
                    plan: bool = False):
    """Write K-hat (QK-Norm + RoPE of k) and V rows into a paged pool.

    k/v: (B, Hkv, S, D), any (b, h, s) strides; k_pool/v_pool:
    (pages, Hkv, page_size, D).  Token s of sequence b is row
    ``t = row_base[b] + s`` (else ``row_offset + s``) of that sequence and
    lands in page ``block_table[b, t // page_size]``, row ``t % page_size``.
    Positions as in ``qk_norm_rope``.  k_weight None skips the norm and
    cos/sin None skip the rotation (a plain copy).
    """
    ref = k if k is not None else v
    if ref is None:
        raise ValueError("nothing to append")
    _require_device(k, v, k_pool, v_pool, block_table)
    dev = ref.device
    B, Hkv, S, D = ref.shape
    for name, pool in (("k_pool", k_pool), ("v_pool", v_pool)):
        _pool_check(pool, name)
        if pool.shape[1] != Hkv or pool.shape[3] != D:
            raise ValueError(f"{name} holds Hkv={pool.shape[1]} D={pool.shape[3]}, rows have Hkv={Hkv} D={D}")
    if k_pool.dtype != v_pool.dtype:
        raise TypeError("k_pool and v_pool must share one dtype")
    if k is not None and v is not None and k.dtype != v.dtype:
        raise TypeError("k and v must share one dtype")
    bt = _block_table(block_table, B, dev)
    k = _rows_in(k) if k is not None else None
    v = _rows_in(v) if v is not None else None
    cos_t, sin_t, max_pos = _tables(cos, sin, dev)
    pos = _positions(position_ids, pos_offset, pos_base, B, S, max_pos, dev)
    pb = _i32(pos_base, dev)
    rb = _i32(row_base, dev)
    kw = _f32(k_weight, dev)
    st = _lib.strides3
    args = (
        _ptr(k), st(k.stride()[:3]) if k is not None else None,
        _ptr(v), st(v.stride()[:3]) if v is not None else None,
        _ptr(k_pool), st(k_pool.stride()[:3]), _ptr(v_pool), st(v_pool.stride()[:3]),
        _ptr(bt), bt.stride(0), k_pool.shape[2],
        B, S, Hkv, D, _code(ref), _code(k_pool), _ptr(kw), float(eps),
        _ptr(cos_t), _ptr(sin_t), max_pos, _ptr(pos), _ptr(pb), int(pos_offset),
        _ptr(rb), int(row_offset), _stream(ref))
    call = KernelCall(_lib.load().nq_kv_append_paged, args, len(args) - 1, "nq_kv_append_paged",
                      (k, v, bt, cos_t, sin_t, pos, pb, rb, kw), (k_pool, v_pool))
    return call if plan else call.launch()


def attention_decode_paged(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                           block_table: torch.Tensor, lens: torch.Tensor, *, max_len: int,
                           k_new: Optional[torch.Tensor] = None, v_new: Optional[torch.Tensor] = None,
                           k_weight: Optional[torch.Tensor] = None,
                           lens_out: Optional[torch.Tensor] = None,
                           q_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                           cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                           q_pos: Optional[torch.Tensor] = None, q_pos0: int = -1,
                           sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                           workspace: Optional[torch.Tensor] = None, chunk: int = 0,
                           plan: bool = False):
    """Single-token GQA decode against a paged cache, with an optional fused append.

    q: (B, Hq, D) or (B, Hq, 1, D) pre-norm query; k_pool/v_pool:
    (pages, Hkv, page_size, D) with page_size a multiple of 32; row t of
    sequence b is page ``block_table[b, t // page_size]``, row
    ``t % page_size``.  A dense (B, Hkv, T_cap, D) cache is the pool of B
    pages of T_cap rows with block_table ``[[0], [1], ...]``.

    Without k_new: attends keys [0, lens[b]); the query is rotated at
    q_pos[b], else q_pos0, else lens[b] - 1.  With k_new/v_new (B, Hkv, D) or
    (B, Hkv, 1, D), the new token's K (normed with k_weight, rotated at the
    query's position, which defaults to lens[b]) and V are written to row
    lens[b] and attended together with keys [0, lens[b]); ``lens_out`` (not
    aliasing lens) then receives lens + 1.  ``max_len`` bounds the keys
    attended per sequence (the appended one included); the block table must
    map every page up to it.  Returns (B, Hq, D).
    """
    _require_device(q, k_pool, v_pool, block_table, lens, k_new, v_new, lens_out, out)
    if q.dim() == 4:
        q = q[:, :, 0]
    B, Hq, D = q.shape
    for name, pool in (("k_pool", k_pool), ("v_pool", v_pool)):
        _pool_check(pool, name)
    if k_pool.shape != v_pool.shape or k_pool.shape[3] != D:
        raise ValueError("pool shapes do not match q")
    Hkv, page = k_pool.shape[1], k_pool.shape[2]
    if q.dtype != k_pool.dtype or q.dtype != v_pool.dtype:
        raise TypeError("q and the pools must share one dtype")
    bt = _block_table(block_table, B, dev := q.device)
    if not 0 < max_len <= bt.shape[1] * page:
        raise ValueError(f"max_len must be in [1, {bt.shape[1] * page}] (block table columns x page_size)")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new go together")
    if k_new is not None:
        if k_new.dim() == 4:
            k_new, v_new = k_new[:, :, 0], v_new[:, :, 0]
        if tuple(k_new.shape) != (B, Hkv, D) or tuple(v_new.shape) != (B, Hkv, D):
            raise ValueError(f"k_new/v_new must be (B={B}, Hkv={Hkv}, D={D})")
        if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
            raise TypeError("k_new/v_new must have q's dtype")
        k_new, v_new = _rows_in(k_new), _rows_in(v_new)
    elif lens_out is not None:
        raise ValueError("lens_out is written only with an append (k_new/v_new)")
    dt = _code(q)
    q = _rows_in(q)
    lens_t = _i32(lens, dev)
    if lens_out is not None:
        if lens_out.dtype != torch.int32 or not lens_out.is_contiguous() or lens_out.numel() != B:
            raise ValueError("lens_out must be a contiguous int32 tensor of B elements")
        if lens_out.data_ptr() == lens_t.data_ptr():
            raise ValueError("lens_out must not alias lens")
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=dev)
    # fp32 caches keep no partials: the library neither needs nor reads a workspace
    need = 0 if q.dtype == torch.float32 else decode_workspace_bytes(B, Hq, Hkv, D, max_len, chunk)
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    wbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    cos_t, sin_t, max_pos = _tables(cos, sin, dev)
    qp = _decode_q_pos(q_pos, q_pos0, B, max_pos, dev)
    qw, kw = _f32(q_weight, dev), _f32(k_weight, dev)
    q_str = (ctypes.c_int64 * 2)(q.stride(0), q.stride(1))
    o_str = (ctypes.c_int64 * 2)(out.stride(0), out.stride(1))
    kn_str = vn_str = None
    if k_new is not None:
        kn_str = (ctypes.c_int64 * 2)(k_new.stride(0), k_new.stride(1))
        vn_str = (ctypes.c_int64 * 2)(v_new.stride(0), v_new.stride(1))
    st = _lib.strides3
    args = (
        _ptr(q), q_str, _ptr(k_new), kn_str, _ptr(v_new), vn_str, _ptr(kw),
        _ptr(k_pool), st(k_pool.stride()[:3]), _ptr(v_pool), st(v_pool.stride()[:3]),
        _ptr(bt), bt.stride(0), page, _ptr(lens_t), _ptr(lens_out),
        _ptr(out), o_str, _ptr(workspace), wbytes,
        B, Hq, Hkv, D, int(max_len), int(chunk), dt, _ptr(qw), float(eps),
        _ptr(cos_t), _ptr(sin_t), max_pos, _ptr(qp), int(q_pos0),
        float(sm_scale) if sm_scale is not None else 0.0, _stream(q))
    call = KernelCall(_lib.load().nq_attn_decode_paged_fwd, args, len(args) - 1,
                      "nq_attn_decode_paged_fwd",
                      (q, k_new, v_new, bt, lens_t, workspace, cos_t, sin_t, qp, qw, kw,
                       q_str, o_str, kn_str, vn_str), out)
    return call if plan else call.launch()


def attention_merge_(o: torch.Tensor, lse: torch.Tensor, o_part: torch.Tensor,
                     lse_part: torch.Tensor, plan: bool = False):
    """Merge a partial (o_part, lse_part) into (o, lse) in place.

    Both are attention over disjoint key sets: o/o_part (B, H, S, D)
    normalised outputs, lse/lse_part fp32 (B, H, S) natural-log sum-exp of the
    scaled scores (``attention_prefill(..., return_lse=True)``).  The
    online-softmax combine of ring attention (distributed/context_parallel.py:
    120-127).  Returns (o, lse).
    """
    _require_device(o, lse, o_part, lse_part)
    B, H, S, D = o.shape
    if tuple(o_part.shape) != (B, H, S, D) or o_part.dtype != o.dtype:
        raise ValueError("o_part must match o in shape and dtype")
    for name, t in (("lse", lse), ("lse_part", lse_part)):
        if tuple(t.shape) != (B, H, S) or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 (B, H, S) tensor")
    _rows_out(o, "o")
    o_part = _rows_in(o_part)
    st = _lib.strides3
    args = (_ptr(o), st(o.stride()[:3]), _ptr(lse), _ptr(o_part), st(o_part.stride()[:3]),
            _ptr(lse_part), B, H, S, D, _code(o), _stream(o))
    call = KernelCall(_lib.load().nq_attn_merge, args, len(args) - 1, "nq_attn_merge",
                      (o_part, lse_part), (o, lse))
    return call if plan else call.launch()


# ---------------------------------------------------------------------------
# Backward
# ---------------------------------------------------------------------------

def attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                       dout: torch.Tensor, lse: torch.Tensor, *, causal: bool = True,
                       sm_scale: Optional[float] = None, key_lens: Optional[torch.Tensor] = None,
                       bias: Optional[AttnBias] = None,
                       workspace: Optional[torch.Tensor] = None, plan: bool = False):
    """FlashAttention-2 backward: (dq, dk, dv) of o = softmax(scale q k^T + bias) v.

    q: (B, Hq, S, D), k/v: (B, Hkv, T, D) as the forward attended them (after
    QK-Norm and RoPE); o, dout: (B, Hq, S, D); lse: the forward's fp32
    (B, Hq, S) log-sum-exp (``attention_prefill(..., return_lse=True)`` with
    the same causal, sm_scale, key_lens and bias; the bias built with
    ``transpose=True``).  dk/dv sum the gradients of the
    G query heads that share a kv head; keys past key_lens[b] get zeros.
    Returns fresh (dq, dk, dv) in q's dtype.
    """
    _require_device(q, k, v, o, dout, lse)
    B, Hq, S, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    if k.shape != v.shape or k.shape[0] != B or k.shape[3] != D:
        raise ValueError("k/v do not match q")
    if tuple(o.shape) != (B, Hq, S, D) or tuple(dout.shape) != (B, Hq, S, D):
        raise ValueError("o and dout must be (B, Hq, S, D)")
    for t in (k, v, o, dout):
        if t.dtype != q.dtype:
            raise TypeError("q, k, v, o and dout must share one dtype")
    if tuple(lse.shape) != (B, Hq, S) or lse.dtype != torch.float32:
        raise ValueError("lse must be fp32 (B, Hq, S)")
    q, k, v, o, dout = (_rows_in(t) for t in (q, k, v, o, dout))
    lse = lse.contiguous()
    dev = q.device
    kl = _key_lens(key_lens, B, dev)
    dq = torch.empty(B, S, Hq, D, dtype=q.dtype, device=dev).transpose(1, 2)
    dk = torch.empty(B, T, Hkv, D, dtype=q.dtype, device=dev).transpose(1, 2)
    dv = torch.empty(B, T, Hkv, D, dtype=q.dtype, device=dev).transpose(1, 2)
    lib = _lib.load()
    need = int(lib.nq_attn_bwd_workspace_bytes(B, Hq, S))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    st = _lib.strides3
    head = (_ptr(q), st(q.stride()[:3]), _ptr(k), st(k.stride()[:3]), _ptr(v), st(v.stride()[:3]),
            _ptr(o), st(o.stride()[:3]), _ptr(dout), st(dout.stride()[:3]), _ptr(lse), _ptr(kl))
    tail = (_ptr(dq), st(dq.stride()[:3]), _ptr(dk), st(dk.stride()[:3]), _ptr(dv), st(dv.stride()[:3]),
            _ptr(workspace), workspace.numel() * workspace.element_size(),
            B, Hq, Hkv, S, T, D, _code(q), int(bool(causal)),
            float(sm_scale) if sm_scale is not None else 0.0, _stream(q))
    keep = (q, k, v, o, dout, lse, workspace, kl)
    if bias is not None:
        _check_bias(bias, B, Hq, S, T, q.dtype, transpose=True)
        args = head + (_ptr(bias.bias), st(bias.strides), _ptr(bias.bias_t), st(bias.t_strides)) + tail
        call = KernelCall(lib.nq_attn_bwd_bias, args, len(args) - 1, "nq_attn_bwd_bias",
                          keep + (bias.bias, bias.bias_t), (dq, dk, dv))
    else:
        args = head + tail
        call = KernelCall(lib.nq_attn_bwd, args, len(args) - 1, "nq_attn_bwd", keep, (dq, dk, dv))
    return call if plan else call.launch()


def qk_norm_rope_backward(x: torch.Tensor, dy: torch.Tensor, *, weight: Optional[torch.Tensor] = None,
                          eps: float = 1e-6, cos: Optional[torch.Tensor] = None,
                          sin: Optional[torch.Tensor] = None,
                          position_ids: Optional[torch.Tensor] = None, pos_offset: int = 0,
                          pos_base: Optional[torch.Tensor] = None):
    """Backward of y = rope(rmsnorm(x) * weight) over (B, H, S, D) rows.

    Returns (dx, dweight): dx in x's dtype, dweight fp32 (D,) summed over all
    rows (None without a weight).  Positions as in ``qk_norm_rope``.
    """
    _require_device(x, dy)
    B, H, S, D = x.shape
    if tuple(dy.shape) != (B, H, S, D) or dy.dtype != x.dtype:
        raise ValueError("dy must match x")
    x, dy = _rows_in(x), _rows_in(dy)
    dev = x.device
    dx = torch.empty(B, S, H, D, dtype=x.dtype, device=dev).transpose(1, 2)
    w = _f32(weight, dev)
    lib = _lib.load()
    dw, ws, wbytes = None, None, 0
    if w is not None:
        dw = torch.empty(D, dtype=torch.float32, device=dev)
        wbytes = int(lib.nq_qk_norm_rope_bwd_workspace_bytes(B, S, H, D))
        ws = torch.empty(wbytes, dtype=torch.uint8, device=dev)
    cos_t, sin_t, max_pos = _tables(cos, sin, dev)
    pos = _positions(position_ids, pos_offset, pos_base, B, S, max_pos, dev)
    pb = _i32(pos_base, dev)
    st = _lib.strides3
    rc = lib.nq_qk_norm_rope_bwd(
        _ptr(x), st(x.stride()[:3]), _ptr(dy), st(dy.stride()[:3]), _ptr(dx), st(dx.stride()[:3]),
        _ptr(w), _ptr(dw), _ptr(ws), wbytes, B, S, H, D, _code(x), float(eps), _ptr(cos_t), _ptr(sin_t),
        max_pos, _ptr(pos), _ptr(pb), int(pos_offset), _stream(x))
    _lib.check(rc, "nq_qk_norm_rope_bwd")
    return dx, dw


# ---------------------------------------------------------------------------
# Mirrors of the reference kernel API
# ---------------------------------------------------------------------------

def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = True,
                    sm_scale: Optional[float] = None, use_triton: bool = True) -> torch.Tensor:
    """kernels/flash_attn.py:130-143 on the gfx950 prefill kernel.

    q: (B, H, N, D), k/v: (B, Hkv, N, D) with H % Hkv == 0 (the reference
    requires Hkv == H; GQA is accepted here).  Where the reference hands inputs
    that require grad to torch's SDPA (flash_attn.py:139), this runs them
    through the kernels' autograd Function (FlashAttention-2 backward).
    ``use_triton`` is accepted for signature compatibility (flash_attn.py:136)
    and selects nothing: the HIP kernels are the only backend, so True and
    False give the same bits.
    head_dim 16, which the reference's kernel accepts (flash_attn.py:106), runs
    on the head_dim-32 kernels with q, k and v zero-padded to 32: the padded
    dimensions add exact zeros to every score and give output columns that are
    dropped, and autograd passes through the pad and the slice.  head_dim 256
    runs on kernels of its own, forward and backward (bf16).
    Returns a contiguous (B, H, N, D) tensor.
    """
    del use_triton
    _require_device(q, k, v)
    if q.shape[-1] == 16 and k.shape[-1] == 16 and v.shape[-1] == 16 and q.numel() > 0:
        scale = sm_scale if sm_scale is not None else 0.25  # 1 / sqrt(16)
        pad = [torch.nn.functional.pad(t, (0, 16)) for t in (q, k, v)]
        return flash_attention(*pad, causal=causal, sm_scale=scale)[..., :16].contiguous()
    if q.numel() == 0:
        # no query rows: an empty output, as the reference's grid of zero blocks gives
        return torch.empty_like(q, memory_format=torch.contiguous_format)
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        from .autograd import flash_attention_train
        return flash_attention_train(q, k, v, causal=causal, sm_scale=sm_scale)
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    return attention_prefill(q, k, v, causal=causal, sm_scale=sm_scale, out=out)


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
               sin: torch.Tensor, use_triton: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """kernels/rope.py:99-108: rotate-half RoPE of q and k, in place.

    q: (B, Hq, S, D), k: (B, Hk, S, D); cos/sin: (S, D/2) rows for positions
    0..S-1, or (B, S, D/2) per-batch rows.  Arithmetic is fp32.
    ``use_triton`` is accepted for signature compatibility (rope.py:104) and
    selects nothing: the row kernel is the only backend.
    """
    del use_triton
    _require_device(q, k)
    B, _, S, D = q.shape
    if cos.dim() == 3:
        tab_c, tab_s = cos.reshape(B * S, D // 2), sin.reshape(B * S, D // 2)
        pos_base = torch.arange(B, device=q.device, dtype=torch.int32) * S
    else:
        tab_c, tab_s, pos_base = cos, sin, None
    qq, kk = _rows_in(q), _rows_in(k)
    qk_norm_rope(q=qq, k=kk, q_out=qq, k_out=kk, cos=tab_c, sin=tab_s, pos_base=pos_base)
    if qq is not q:
        q.copy_(qq)
    if kk is not k:
        k.copy_(kk)
    return q, k
