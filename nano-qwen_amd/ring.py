"""Ring attention's per-GPU compute on the gfx950 kernels (distributed/context_parallel.py:17-140).

In context parallelism every rank holds one contiguous chunk of the sequence
(``split_sequence``) and the K/V chunks travel round the ring; at each step a
rank attends its queries to the chunk it holds and folds the result into its
running output.  This module is that per-rank work:

  * ``ring_schedule(rank, cp_size)``: which chunk a rank holds at each step.
    It receives from rank - 1 and forwards what it held, so at step s it holds
    chunk ``(rank - s) % cp_size``.  (The reference labels that chunk
    ``(rank + s) % cp_size`` when masking, context_parallel.py:104; the two
    agree only for cp_size <= 2, so for three or more ranks the reference
    masks the wrong chunks.  The true source is used here.)
  * ``ring_step``: causal masking per chunk as in context_parallel.py:112-117
    -- chunks after the rank's own are skipped, the rank's own chunk is
    causal, earlier chunks are attended in full -- computed by the prefill
    kernel with its log-sum-exp, then merged into the running (o, lse) by the
    merge kernel (the rescale of lines 120-127).
  * ``RingAttention``: the reference module's interface.  With one rank (or
    no group) it is the plain causal attention, as in the reference (line 84).
    The K/V exchange between GPUs (isend/irecv over RCCL) is not part of this
    one-GPU build; a rank drives ``ring_step`` itself as chunks arrive.
  * ``ring_attention_all_ranks``: every rank's work for a cp_size ring run
    one after another on one GPU (what the ring computes, without the
    transport), used to check the pieces against full attention.

Unlike the reference (which broadcasts q against k with a plain matmul), the
K/V chunks may have fewer heads than q (GQA, kv head = h / G).
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch
import torch.nn as nn

from . import ops


def split_sequence(hidden_states: torch.Tensor, cp_rank: int, cp_size: int) -> torch.Tensor:
    """context_parallel.py:17-35: rank cp_rank's contiguous chunk of dim 1."""
    B, S = hidden_states.shape[:2]
    if S % cp_size:
        raise ValueError(f"seq_len={S} not divisible by cp_size={cp_size}")
    c = S // cp_size
    return hidden_states[:, cp_rank * c:(cp_rank + 1) * c].contiguous()


def ring_schedule(rank: int, cp_size: int) -> List[int]:
    """The chunk a rank holds at steps 0 .. cp_size-1 of the ring."""
    return [(rank - s) % cp_size for s in range(cp_size)]


def ring_step(q: torch.Tensor, k_chunk: torch.Tensor, v_chunk: torch.Tensor, *, src: int, rank: int,
              causal: bool = True, o: Optional[torch.Tensor] = None,
              lse: Optional[torch.Tensor] = None, sm_scale: Optional[float] = None
              ) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
    """Fold the attention of q (B, H, S, D) to chunk ``src`` into (o, lse).

    q holds rank ``rank``'s queries (already normed and rotated), k/v_chunk
    (B, Hkv, S, D) the keys and values of chunk ``src``.  Returns the updated
    (o, lse); (None, None) as input means nothing accumulated yet.
    """
    if causal and src > rank:
        return o, lse  # every key of a later chunk is in this rank's future
    o_part, lse_part = ops.attention_prefill(q, k_chunk, v_chunk, causal=causal and src == rank,
                                             sm_scale=sm_scale, return_lse=True)
    if o is None:
        return o_part, lse_part
    return ops.attention_merge_(o, lse, o_part, lse_part)


class RingAttention(nn.Module):
    """context_parallel.py:52-140: ring attention for context parallelism."""

    def __init__(self, cp_group=None):
        super().__init__()
        self.cp_group = cp_group
        if cp_group is not None:
            import torch.distributed as dist
            self.cp_size, self.cp_rank = dist.get_world_size(cp_group), dist.get_rank(cp_group)
        else:
            self.cp_size, self.cp_rank = 1, 0

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                causal: bool = True) -> torch.Tensor:
        """q, k, v: (B, H, S_local, D) local chunks; returns (B, H, S_local, D)."""
        if self.cp_size <= 1:
            return ops.flash_attention(q, k, v, causal=causal)
        raise NotImplementedError(
            "the K/V exchange between GPUs is not built in this one-GPU library; call ring_step "
            "for each chunk as it arrives (ring_schedule gives the order)")


def ring_attention_all_ranks(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cp_size: int,
                             causal: bool = True, sm_scale: Optional[float] = None) -> torch.Tensor:
    """Every rank's ring work for a cp_size ring, run in turn on this GPU.

    q: (B, H, S, D), k/v: (B, Hkv, S, D) for the whole sequence.  Each rank
    takes its chunk of q and meets the K/V chunks in ring order; the outputs
    are concatenated back.  Equals full (causal) attention.
    """
    S = q.shape[2]
    if S % cp_size:
        raise ValueError(f"seq_len={S} not divisible by cp_size={cp_size}")
    c = S // cp_size
    chunk = lambda t, i: t[:, :, i * c:(i + 1) * c]  # noqa: E731
    outs = []
    for rank in range(cp_size):
        o = lse = None
        for src in ring_schedule(rank, cp_size):
            o, lse = ring_step(chunk(q, rank), chunk(k, src), chunk(v, src), src=src, rank=rank,
                               causal=causal, o=o, lse=lse, sm_scale=sm_scale)
        outs.append(o)
    return torch.cat(outs, dim=2)
