"""GPU parity of the LSE merge and of ring attention's per-rank work (one GPU)."""

import pytest
import torch

import nano_qwen_amd as nq
from oracle import attention, attention_lse, merge_partials
from tests.helpers import assert_bf16_close, randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_merge_kernel_against_closed_form(D, dtype):
    say(f"merge D={D} {dtype}")
    B, H, S, T = 2, 4, 33, 50
    q, k, v = randn(B, H, S, D, seed=421), randn(B, 2, T, D, seed=422), randn(B, 2, T, D, seed=423)
    oa, la = attention_lse(q, k[:, :, :20], v[:, :, :20])
    ob, lb = attention_lse(q, k[:, :, 20:], v[:, :, 20:])
    # rows with no keys in one part, and in both
    la[0, 1, 3] = float("-inf")
    lb[1, 2, 5] = float("-inf")
    la[1, 0, 7] = lb[1, 0, 7] = float("-inf")
    want_o, want_l = merge_partials(oa, la, ob, lb)
    want_o[1, 0, 7] = 0.0
    # accumulator in the (B, S, H, D) storage the prefill writes
    o = oa.to(dtype).transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    o[0, 1, 3] = float("nan")  # never read: its part has no keys
    part = ob.to(dtype).to(DEV)
    part[1, 2, 5] = float("nan")
    lse = la.float().to(DEV)
    nq.attention_merge_(o, lse, part, lb.float().to(DEV))
    got_l = lse.cpu().double()
    fin = torch.isfinite(want_l)
    assert torch.equal(torch.isfinite(got_l), fin)
    torch.testing.assert_close(got_l[fin], want_l[fin], rtol=0, atol=1e-5)
    assert_bf16_close(o, want_o, f"merge {dtype}", max_abs=1e-2 if dtype == torch.bfloat16 else 1e-5,
                      mean_abs=1e-3 if dtype == torch.bfloat16 else 1e-6)


@pytest.mark.parametrize("cp", [2, 3, 4])
@pytest.mark.parametrize("causal", [True, False])
def test_ring_all_ranks_equals_full_attention(cp, causal):
    say(f"ring cp={cp} causal={causal}")
    B, Hq, Hkv, S, D = 2, 16, 4, 768, 128
    q = randn(B, Hq, S, D, seed=431, dtype=torch.bfloat16)
    k = randn(B, Hkv, S, D, seed=432, dtype=torch.bfloat16)
    v = randn(B, Hkv, S, D, seed=433, dtype=torch.bfloat16)
    got = nq.ring_attention_all_ranks(q.to(DEV), k.to(DEV), v.to(DEV), cp, causal=causal)
    ref = attention(q.float(), k.float(), v.float(), causal=causal)
    assert_bf16_close(got, ref, f"ring cp={cp}")
    full = nq.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal)
    assert_bf16_close(got, full, "ring vs one prefill")


def test_ring_step_skips_future_chunks_and_single_rank_module():
    say("ring step / module")
    B, H, S, D = 1, 8, 256, 64
    q, k, v = (randn(B, H, S, D, seed=441 + i, dtype=torch.bfloat16).to(DEV) for i in range(3))
    o, lse = nq.ring_step(q, k, v, src=2, rank=1)
    assert o is None and lse is None
    out = nq.RingAttention()(q, k, v, causal=True)
    torch.testing.assert_close(out, nq.flash_attention(q, k, v, causal=True), rtol=0, atol=0)
    assert nq.ring_schedule(2, 4) == [2, 1, 0, 3]
