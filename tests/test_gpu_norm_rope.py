"""GPU parity of the QK-Norm + RoPE row kernel against the oracle."""

import pytest
import torch

import nano_qwen_amd as nq
from oracle import rms_norm, rope_tables, rotate_half
from tests.helpers import assert_bf16_close, randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _oracle_rows(x, w, eps, cos, sin, pos):
    """x (B, H, S, D) fp32; pos (B, S) long."""
    y = rms_norm(x, w, eps) if w is not None else x
    return rotate_half(y, cos[pos][:, None], sin[pos][:, None])


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("posmode", ["none", "offset", "explicit"])
def test_qk_norm_rope_rows(D, dtype, posmode):
    say(f"qk_norm_rope D={D} {dtype} pos={posmode}")
    B, S, Hq, Hkv, eps = 2, 37, 8, 2, 1e-6
    q = randn(B, S, Hq, D, seed=1, dtype=dtype).transpose(1, 2)  # model layout view
    k = randn(B, S, Hkv, D, seed=2, dtype=dtype).transpose(1, 2)
    v = randn(B, S, Hkv, D, seed=3, dtype=dtype).transpose(1, 2)
    qw = 1 + 0.02 * randn(D, seed=4)
    kw = 1 + 0.02 * randn(D, seed=5)
    cos, sin = rope_tables(D, 512, 1e6)
    if posmode == "none":
        pos, kwargs = torch.arange(S).expand(B, S), {}
    elif posmode == "offset":
        pos, kwargs = (torch.arange(S) + 300).expand(B, S), {"pos_offset": 300}
    else:
        pos = torch.stack([torch.randperm(512, generator=torch.Generator().manual_seed(b))[:S]
                           for b in range(B)])
        kwargs = {"position_ids": pos.to(DEV)}
    qo, ko, vo = nq.qk_norm_rope(q.to(DEV), k.to(DEV), v.to(DEV), q_weight=qw.to(DEV),
                                 k_weight=kw.to(DEV), eps=eps, cos=cos.to(DEV), sin=sin.to(DEV),
                                 **kwargs)
    torch.cuda.synchronize()
    rq = _oracle_rows(q.float(), qw, eps, cos, sin, pos)
    rk = _oracle_rows(k.float(), kw, eps, cos, sin, pos)
    if dtype == torch.float32:
        torch.testing.assert_close(qo.cpu(), rq, rtol=2e-5, atol=2e-5)
        torch.testing.assert_close(ko.cpu(), rk, rtol=2e-5, atol=2e-5)
        torch.testing.assert_close(vo.cpu(), v, rtol=0, atol=0)
    else:
        # one rounding to bf16 of an fp32-exact result: within half a bf16 ulp
        assert_bf16_close(qo, rq, "q")
        assert_bf16_close(ko, rk, "k")
        assert torch.equal(vo.cpu(), v)


def test_rows_land_in_cache_slots_and_nowhere_else():
    say("qk_norm_rope cache placement")
    B, S, Hkv, D, cap = 3, 5, 2, 128, 40
    k = randn(B, Hkv, S, D, seed=6, dtype=torch.bfloat16).to(DEV)
    v = randn(B, Hkv, S, D, seed=7, dtype=torch.bfloat16).to(DEV)
    cos, sin = rope_tables(D, 64, 1e6)
    kc = torch.full((B, Hkv, cap, D), 7.0, dtype=torch.bfloat16, device=DEV)
    vc = torch.full((B, Hkv, cap, D), 7.0, dtype=torch.bfloat16, device=DEV)
    base = torch.tensor([0, 11, 30], dtype=torch.int32, device=DEV)
    nq.qk_norm_rope(k=k, v=v, k_out=kc, v_out=vc, cos=cos.to(DEV), sin=sin.to(DEV),
                    kv_row_base=base, pos_base=base)
    torch.cuda.synchronize()
    kc, vc = kc.cpu(), vc.cpu()
    for b, r0 in enumerate([0, 11, 30]):
        pos = torch.arange(r0, r0 + S)
        want = rotate_half(k[b].cpu().float(), cos[pos][None], sin[pos][None])
        assert_bf16_close(kc[b, :, r0:r0 + S], want, f"k row {b}")
        assert torch.equal(vc[b, :, r0:r0 + S], v[b].cpu())
        untouched = torch.ones(cap, dtype=torch.bool)
        untouched[r0:r0 + S] = False
        assert torch.all(kc[b, :, untouched] == 7.0) and torch.all(vc[b, :, untouched] == 7.0)


def test_apply_rope_mirror_is_in_place():
    say("apply_rope in place")
    B, H, S, D = 2, 4, 9, 64
    q = randn(B, H, S, D, seed=8).to(DEV)
    k = randn(B, 2, S, D, seed=9).to(DEV)
    cos, sin = rope_tables(D, S, 1e4)
    q0, k0 = q.clone(), k.clone()
    qr, kr = nq.apply_rope(q, k, cos.to(DEV), sin.to(DEV))
    assert qr.data_ptr() == q.data_ptr() and kr.data_ptr() == k.data_ptr()
    torch.testing.assert_close(q.cpu(), rotate_half(q0.cpu(), cos, sin), rtol=2e-5, atol=2e-5)
    torch.testing.assert_close(k.cpu(), rotate_half(k0.cpu(), cos, sin), rtol=2e-5, atol=2e-5)


def test_rmsnorm_module_matches_oracle():
    say("RMSNorm module")
    x = randn(3, 5, 128, seed=10, dtype=torch.bfloat16, scale=3.0)
    norm = nq.RMSNorm(128, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * randn(128, seed=11))
    y = norm.to(DEV)(x.to(DEV))
    # model/norm.py:21-22: `.type_as(x) * weight` promotes a bf16 input with an
    # fp32 weight to fp32 (the golden tests/golden/rmsnorm.npz records it)
    ref = rms_norm(x, norm.weight.detach().cpu(), 1e-6)
    assert y.dtype == ref.dtype == torch.float32
    assert_bf16_close(y, ref, "rmsnorm")
    y.float().sum().backward()  # autograd through the backward kernel
    assert norm.weight.grad is not None and torch.isfinite(norm.weight.grad).all()


@pytest.mark.parametrize("D,S", [(32, 40000), (64, 20000), (128, 12000)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", ["projections", "head_major"])
def test_rows_many_passes_and_out_of_range_positions(D, S, dtype, layout):
    """Enough rows that every thread of the persistent grid takes several rows, Q and K
    jobs in one launch, rows in both enumeration orders (heads adjacent in memory, or
    positions), explicit device positions of which some lie past the tables: those rows
    come out NaN and every other row matches the oracle."""
    say(f"qk_norm_rope many rows D={D} S={S} {dtype} {layout}")
    B, Hq, Hkv, eps, max_pos = 2, 8, 4, 1e-6, S + 64
    if layout == "projections":
        q = randn(B, S, Hq, D, seed=31, dtype=dtype).transpose(1, 2)
        k = randn(B, S, Hkv, D, seed=32, dtype=dtype).transpose(1, 2)
    else:
        q = randn(B, Hq, S, D, seed=31, dtype=dtype)
        k = randn(B, Hkv, S, D, seed=32, dtype=dtype)
    qw = 1 + 0.02 * randn(D, seed=33)
    kw = 1 + 0.02 * randn(D, seed=34)
    cos, sin = rope_tables(D, max_pos, 1e6)
    g = torch.Generator().manual_seed(35)
    pos = torch.randint(0, max_pos, (B, S), generator=g)
    bad = torch.rand(B, S, generator=g) < 0.01
    pos_dev = torch.where(bad, max_pos + 7, pos).to(torch.int32)
    qo, ko, _ = nq.qk_norm_rope(q.to(DEV), k.to(DEV), q_weight=qw.to(DEV), k_weight=kw.to(DEV), eps=eps,
                                cos=cos.to(DEV), sin=sin.to(DEV), position_ids=pos_dev.to(DEV))
    torch.cuda.synchronize()
    qo, ko = qo.cpu().float(), ko.cpu().float()
    for name, got, x, w in (("q", qo, q, qw), ("k", ko, k, kw)):
        nanrow = torch.isnan(got).any(-1)                     # (B, H, S)
        assert torch.equal(nanrow, bad[:, None].expand_as(nanrow)), f"{name}: NaN rows"
        assert torch.isnan(got[bad[:, None].expand_as(nanrow)]).all(), f"{name}: whole rows NaN"
        want = _oracle_rows(x.float(), w, eps, cos, sin, pos)
        ok = ~bad[:, None].expand_as(nanrow)
        if dtype == torch.float32:
            torch.testing.assert_close(got[ok], want[ok], rtol=2e-5, atol=2e-5)
        else:
            assert_bf16_close(got[ok], want[ok], name)
