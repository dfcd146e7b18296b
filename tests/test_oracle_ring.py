"""Pin the ring-attention restatement (distributed/context_parallel.py:52-140)."""

import pytest
import torch

from oracle import attention, attention_lse, merge_partials, ring_attention
from tests.helpers import randn


def _qkv(B=2, H=3, S=48, D=16, seed=401):
    return (randn(B, H, S, D, seed=seed), randn(B, H, S, D, seed=seed + 1),
            randn(B, H, S, D, seed=seed + 2))


@pytest.mark.parametrize("cp", [1, 2, 3, 4])
@pytest.mark.parametrize("causal", [True, False])
def test_true_labels_give_full_attention(cp, causal):
    q, k, v = _qkv()
    got = ring_attention(q, k, v, cp, causal=causal, labels="true")
    torch.testing.assert_close(got, attention(q, k, v, causal=causal), rtol=1e-5, atol=1e-5)


def test_reference_labels_agree_up_to_two_ranks():
    q, k, v = _qkv()
    for cp in (1, 2):
        torch.testing.assert_close(ring_attention(q, k, v, cp, labels="reference"),
                                   attention(q, k, v, causal=True), rtol=1e-5, atol=1e-5)


def test_reference_labels_mask_the_wrong_chunks_from_three_ranks():
    """Rank 1 of 3 holds chunk 0 at step 1 but masks it as chunk 2, and attends
    chunk 2 at step 2 as if it were chunk 0."""
    q, k, v = _qkv()
    ref = ring_attention(q, k, v, 3, labels="reference")
    full = attention(q, k, v, causal=True)
    c = q.shape[2] // 3
    torch.testing.assert_close(ref[:, :, :c], full[:, :, :c], rtol=1e-5, atol=1e-5)  # rank 0 unaffected
    assert (ref[:, :, c:2 * c] - full[:, :, c:2 * c]).abs().max() > 1e-2


def test_merge_closed_form_equals_attention_over_the_union():
    q, k, v = _qkv(S=40, seed=411)
    o1, l1 = attention_lse(q, k[:, :, :17], v[:, :, :17])
    o2, l2 = attention_lse(q, k[:, :, 17:], v[:, :, 17:])
    o, lse = merge_partials(o1, l1, o2, l2)
    of, lf = attention_lse(q, k, v)
    torch.testing.assert_close(o, of, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse, lf, rtol=1e-12, atol=1e-12)
