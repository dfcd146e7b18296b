"""GPU parity of the split-K decode kernel against the oracle."""

import pytest
import torch

import nano_qwen_amd as nq
from oracle import decode_path, rope_tables
from tests.helpers import assert_bf16_close, assert_close_for, randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _poison_tail(cache, lens):
    for b, L in enumerate(lens.tolist()):
        cache[b, :, L:] = float("nan")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("chunk", [32, 64, 0])
def test_decode_small_ragged(D, dtype, chunk):
    say(f"decode small D={D} {dtype} chunk={chunk}")
    B, Hq, Hkv, Tcap = 4, 16, 1, 300
    lens = torch.tensor([1, 100, 300, 64], dtype=torch.int32)
    q = randn(B, Hq, D, seed=61, dtype=dtype)
    kc = randn(B, Hkv, Tcap, D, seed=62, dtype=dtype)
    vc = randn(B, Hkv, Tcap, D, seed=63, dtype=dtype)
    _poison_tail(kc, lens), _poison_tail(vc, lens)
    qw = 1 + 0.02 * randn(D, seed=64)
    cos, sin = rope_tables(D, 512, 1e6)
    o = nq.attention_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), max_len=Tcap,
                            q_weight=qw.to(DEV), eps=1e-6, cos=cos.to(DEV), sin=sin.to(DEV),
                            chunk=chunk)
    ref = decode_path(q.float(), kc.float(), vc.float(), lens, q_weight=qw, eps=1e-6, cos=cos,
                      sin=sin, q_pos=lens.long() - 1)
    assert torch.isfinite(o.float().cpu()).all()
    assert_close_for(dtype, o, ref, "decode small")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (8, 2), (64, 4), (32, 1)])
def test_decode_group_sizes(Hq, Hkv):
    say(f"decode G={Hq // Hkv}")
    B, D, Tcap = 3, 128, 2100
    lens = torch.tensor([2100, 1025, 33], dtype=torch.int32)
    q = randn(B, Hq, D, seed=71, dtype=torch.bfloat16)
    kc = randn(B, Hkv, Tcap, D, seed=72, dtype=torch.bfloat16)
    vc = randn(B, Hkv, Tcap, D, seed=73, dtype=torch.bfloat16)
    cos, sin = rope_tables(D, 4096, 1e6)
    qpos = torch.tensor([5, 4000, 17], dtype=torch.int32)
    o = nq.attention_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), max_len=Tcap,
                            cos=cos.to(DEV), sin=sin.to(DEV), q_pos=qpos.to(DEV))
    ref = decode_path(q.float(), kc.float(), vc.float(), lens, q_weight=None, eps=1e-6, cos=cos,
                      sin=sin, q_pos=qpos.long())
    assert_bf16_close(o, ref, f"G={Hq // Hkv}")


@pytest.mark.parametrize("delta", [-1, 0, 1])
def test_decode_at_the_weighted_split_threshold(delta):
    """Total step counts N around the point where the persistent split turns to
    the XCD weights (N * 22 >= the weight of all waves; below it the split is
    even).  At the threshold the waves on odd XCDs take a single step each, and
    rows are cut into the most partials the merge sees."""
    from tests.test_decode_schedule import ODD_W, _split_weight
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    waves = min(cus * 4, 1024)  # the persistent grid: one 4-wave workgroup per CU
    N = -(-_split_weight(waves) // ODD_W) + delta
    say(f"decode weighted-split threshold N={N} waves={waves}")
    B, Hq, Hkv, D = 2, 16, 1, 128
    n0 = N // 2
    lens = torch.tensor([n0 * 32, (N - n0) * 32 - 5], dtype=torch.int32)  # the second ends mid-step
    Tcap = int(lens.max())
    q = randn(B, Hq, D, seed=85, dtype=torch.bfloat16)
    kc = randn(B, Hkv, Tcap, D, seed=86, dtype=torch.bfloat16)
    vc = randn(B, Hkv, Tcap, D, seed=87, dtype=torch.bfloat16)
    _poison_tail(kc, lens), _poison_tail(vc, lens)
    qw = 1 + 0.02 * randn(D, seed=88)
    cos, sin = rope_tables(D, Tcap, 1e6)
    o = nq.attention_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), max_len=Tcap,
                            q_weight=qw.to(DEV), eps=1e-6, cos=cos.to(DEV), sin=sin.to(DEV))
    ref = decode_path(q.float(), kc.float(), vc.float(), lens, q_weight=qw, eps=1e-6, cos=cos,
                      sin=sin, q_pos=lens.long() - 1)
    assert torch.isfinite(o.float().cpu()).all()
    assert_bf16_close(o, ref, f"threshold N={N}")


def test_split_count_does_not_change_the_result():
    say("decode split invariance")
    B, Hq, Hkv, D, Tcap = 2, 16, 2, 128, 5000
    lens = torch.tensor([5000, 3333], dtype=torch.int32, device=DEV)
    q = randn(B, Hq, D, seed=81, dtype=torch.bfloat16).to(DEV)
    kc = randn(B, Hkv, Tcap, D, seed=82, dtype=torch.bfloat16).to(DEV)
    vc = randn(B, Hkv, Tcap, D, seed=83, dtype=torch.bfloat16).to(DEV)
    outs = [nq.attention_decode(q, kc, vc, lens, max_len=Tcap, chunk=c).float().cpu()
            for c in (32, 256, 1024, 8192)]
    for o in outs[1:]:
        torch.testing.assert_close(o, outs[0], rtol=0, atol=8e-3)


def test_decode_equals_last_row_of_prefill():
    """Size-independent property: decode of token T-1 == row T-1 of causal prefill."""
    say("decode == last prefill row")
    B, T, Hq, Hkv, D = 2, 777, 16, 4, 128
    q = randn(B, T, Hq, D, seed=91, dtype=torch.bfloat16).transpose(1, 2).to(DEV)
    k = randn(B, T, Hkv, D, seed=92, dtype=torch.bfloat16).transpose(1, 2).to(DEV)
    v = randn(B, T, Hkv, D, seed=93, dtype=torch.bfloat16).transpose(1, 2).to(DEV)
    qw = (1 + 0.02 * randn(D, seed=94)).to(DEV)
    kw = (1 + 0.02 * randn(D, seed=95)).to(DEV)
    cos, sin = (t.to(DEV) for t in rope_tables(D, 1024, 1e6))
    kc = torch.empty(B, Hkv, 1024, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.empty_like(kc)
    nq.qk_norm_rope(k=k, v=v, k_out=kc, v_out=vc, k_weight=kw, eps=1e-6, cos=cos, sin=sin)
    pre = nq.attention_prefill(q, kc[:, :, :T], vc[:, :, :T], q_weight=qw, eps=1e-6, cos=cos,
                               sin=sin, causal=True)
    dec = nq.attention_decode(q[:, :, -1], kc, vc, None, max_len=T, q_weight=qw, eps=1e-6,
                              cos=cos, sin=sin)
    torch.testing.assert_close(dec.float().cpu(), pre[:, :, -1].float().cpu(), rtol=0, atol=1e-2)


def test_qwen3_235b_decode_full_size():
    """B64, Hq64/Hkv4, D128, lens ~ U[1024, 32768], T_cap 32768; tails poisoned with NaN;
    every row against the oracle, with the query's QK-Norm (weights 1 + 0.02 N(0,1)) and
    RoPE fused into its load, as the bench's decode step runs it."""
    say("decode Qwen3-235B-A22B B64 T_cap 32768")
    B, Hq, Hkv, D, Tcap = 64, 64, 4, 128, 32768
    g = torch.Generator().manual_seed(1003)
    lens = torch.randint(1024, 32769, (B,), generator=g, dtype=torch.int32)
    gd = torch.Generator(device=DEV).manual_seed(1003)
    kc = torch.randn(B, Hkv, Tcap, D, generator=gd, device=DEV, dtype=torch.bfloat16)
    vc = torch.randn(B, Hkv, Tcap, D, generator=gd, device=DEV, dtype=torch.bfloat16)
    for b in range(B):
        kc[b, :, lens[b]:] = float("nan")
        vc[b, :, lens[b]:] = float("nan")
    q = randn(B, Hq, D, seed=1005, dtype=torch.bfloat16)
    qw = 1 + 0.02 * randn(D, seed=1006)
    cos, sin = rope_tables(D, Tcap, 1e6)
    ld = lens.to(DEV)
    o = nq.attention_decode(q.to(DEV), kc, vc, ld, max_len=int(lens.max()), q_weight=qw.to(DEV), eps=1e-6,
                            cos=cos.to(DEV), sin=sin.to(DEV)).cpu()
    assert torch.isfinite(o.float()).all()
    for b in range(B):  # every row, the shortest and the longest among them
        L = int(lens[b])
        ref = decode_path(q[b:b + 1].float(), kc[b:b + 1, :, :L].float().cpu(),
                          vc[b:b + 1, :, :L].float().cpu(), lens[b:b + 1], q_weight=qw,
                          eps=1e-6, cos=cos, sin=sin, q_pos=lens[b:b + 1].long() - 1)
        assert_bf16_close(o[b:b + 1], ref, f"235B b={b} len={L}")
