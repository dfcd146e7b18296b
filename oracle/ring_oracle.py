"""CPU restatement of nano-qwen's ring attention -- TEST INFRASTRUCTURE ONLY
(imported by ``tests/`` alone, as the checker).

Follows distributed/context_parallel.py:52-140 (RingAttention.forward) for
every rank of a cp_size ring, with the transport replaced by indexing: at
step s rank r holds the K/V chunk that has travelled s hops from rank
r - s (isend to rank + 1, irecv from rank - 1, lines 99-108).  The online
softmax is the reference's: running max, rescaled sum and output, fp32
(lines 110-134).  ``labels`` chooses the chunk index used for the causal
mask: "reference" is the reference's ``src_rank = (rank + step) % cp_size``
(line 104), "true" is the chunk actually held, ``(rank - step) % cp_size``.

Pinning (tests/test_oracle_ring.py): with true labels the result equals the
pinned full attention (``attention``) for cp_size 1-4, causal and not; with
the reference's labels it does too for cp_size <= 2, and differs for
cp_size 3 (the mislabelled chunks), which the test records.
"""

from __future__ import annotations

import math

import torch


def ring_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cp_size: int,
                   causal: bool = True, labels: str = "true") -> torch.Tensor:
    """Outputs of all ranks of a cp_size ring, concatenated: (B, H, S, D) fp32.

    q, k, v: (B, H, S, D) for the whole sequence (the reference's matmul has
    no GQA: k and v carry q's heads).  S is split into cp_size equal chunks
    (split_sequence, context_parallel.py:17-35).
    """
    B, H, S, D = q.shape
    assert S % cp_size == 0 and labels in ("true", "reference")
    c = S // cp_size
    qf, kf, vf = (t.float() for t in (q, k, v))
    outs = []
    for rank in range(cp_size):
        ql = qf[:, :, rank * c:(rank + 1) * c]
        out = torch.zeros_like(ql)
        max_score = torch.full((B, H, c, 1), float("-inf"))
        sum_exp = torch.zeros(B, H, c, 1)
        for step in range(cp_size):
            held = (rank - step) % cp_size
            src = held if labels == "true" else (rank + step) % cp_size
            kc = kf[:, :, held * c:(held + 1) * c]
            vc = vf[:, :, held * c:(held + 1) * c]
            scores = torch.matmul(ql, kc.transpose(-2, -1)) * (D ** -0.5)
            if causal and src > rank:
                scores.fill_(float("-inf"))
            elif causal and src == rank:
                mask = torch.triu(torch.ones(c, c, dtype=torch.bool), diagonal=1)
                scores.masked_fill_(mask[None, None], float("-inf"))
            chunk_max = scores.max(dim=-1, keepdim=True).values
            new_max = torch.maximum(max_score, chunk_max)
            # a fully masked chunk before any finite score would give
            # exp(-inf - -inf); the reference never meets it (step 0 is the
            # rank's own chunk), and the guard keeps the restatement total
            safe = torch.where(torch.isfinite(new_max), new_max, torch.zeros_like(new_max))
            exp_scores = torch.exp(scores - safe)
            correction = torch.exp(max_score - safe)
            out = out * correction + torch.matmul(exp_scores, vc)
            sum_exp = sum_exp * correction + exp_scores.sum(dim=-1, keepdim=True)
            max_score = new_max
        outs.append(out / sum_exp)
    return torch.cat(outs, dim=2)


def merge_partials(o_a: torch.Tensor, lse_a: torch.Tensor, o_b: torch.Tensor,
                   lse_b: torch.Tensor):
    """Closed form of combining two attention partials over disjoint key sets:
    L = log(e^La + e^Lb), O = O_a e^(La - L) + O_b e^(Lb - L) (fp64)."""
    la, lb = lse_a.double(), lse_b.double()
    L = torch.logaddexp(la, lb)
    wa = torch.exp(la - L).unsqueeze(-1)
    wb = torch.exp(lb - L).unsqueeze(-1)
    return o_a.double() * wa + o_b.double() * wb, L


def attention_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = False):
    """fp64 attention with its natural-log sum-exp of the scaled scores (GQA)."""
    B, H, S, D = q.shape
    G = H // k.shape[1]
    kk = k.double().repeat_interleave(G, 1)
    vv = v.double().repeat_interleave(G, 1)
    sc = torch.matmul(q.double(), kk.transpose(-1, -2)) / math.sqrt(D)
    if causal:
        T = k.shape[2]
        keep = torch.arange(T)[None, :] <= torch.arange(S)[:, None] + (T - S)
        sc = sc.masked_fill(~keep, float("-inf"))
    lse = torch.logsumexp(sc, dim=-1)
    return torch.matmul(torch.softmax(sc, dim=-1), vv), lse
