"""GPU tests of the drop-in boundary: every kernel at head_dim 32 (the
reference's default model, configs/model/debug.yaml: hidden 256 over 8 heads),
out-of-range positions, the RMSNorm mirror's dtype promotion, decode
position_ids that broadcast, cache-length overflow, the widest GQA groups the
prefill accepts, decode batches past 64 rows, and the plain-KVCache one-token
step on the fused append.  References are the oracle's fp32 (or fp64) math."""

import math

import pytest
import torch

import nano_qwen_amd as nq
from nano_qwen_amd import ops
from oracle import (OracleKVCache, attention, attention_module_forward, attention_path, decode_path,
                    rms_norm, rope_tables, rotate_half)
from tests.helpers import assert_bf16_close, assert_close_for, assert_fp32_close, randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"
D32 = 32


def _prefill_case(B, S, Hq, Hkv, D, dtype, seed, causal=True, theta=1e4):
    q = randn(B, S, Hq, D, seed=seed, dtype=dtype).transpose(1, 2)
    k = randn(B, S, Hkv, D, seed=seed + 1, dtype=dtype).transpose(1, 2)
    v = randn(B, S, Hkv, D, seed=seed + 2, dtype=dtype).transpose(1, 2)
    qw = 1 + 0.02 * randn(D, seed=seed + 3)
    kw = 1 + 0.02 * randn(D, seed=seed + 4)
    cos, sin = rope_tables(D, S, theta)
    kh = nq.qk_norm_rope(k=k.to(DEV), k_weight=kw.to(DEV), eps=1e-6, cos=cos.to(DEV), sin=sin.to(DEV))[1]
    o = nq.attention_prefill(q.to(DEV), kh, v.to(DEV), q_weight=qw.to(DEV), eps=1e-6, cos=cos.to(DEV),
                             sin=sin.to(DEV), causal=causal)
    ref = attention_path(q.float(), k.float(), v.float(), q_weight=qw, k_weight=kw, eps=1e-6, cos=cos,
                         sin=sin, q_pos=torch.arange(S), causal=causal)
    return o, ref


# ------------------------------------------------------------------ head_dim 32

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_d32_row_kernel(dtype):
    say(f"D=32 row kernel {dtype}")
    B, S, Hq, Hkv = 2, 70, 8, 2
    q = randn(B, Hq, S, D32, seed=3201, dtype=dtype)
    k = randn(B, Hkv, S, D32, seed=3202, dtype=dtype)
    qw = 1 + 0.02 * randn(D32, seed=3203)
    kw = 1 + 0.02 * randn(D32, seed=3204)
    cos, sin = rope_tables(D32, 128, 1e4)
    pos = torch.randint(0, 128, (B, S), generator=torch.Generator().manual_seed(3205))
    qo, ko, _ = nq.qk_norm_rope(q=q.to(DEV), k=k.to(DEV), q_weight=qw.to(DEV), k_weight=kw.to(DEV), eps=1e-6,
                                cos=cos.to(DEV), sin=sin.to(DEV), position_ids=pos.to(DEV))
    c, s = cos[pos][:, None], sin[pos][:, None]
    assert_close_for(dtype, qo, rotate_half(rms_norm(q.float(), qw, 1e-6), c, s), "q-hat")
    assert_close_for(dtype, ko, rotate_half(rms_norm(k.float(), kw, 1e-6), c, s), "k-hat")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (8, 2), (16, 1)])
@pytest.mark.parametrize("S", [1, 77, 300])
@pytest.mark.parametrize("causal", [True, False])
def test_d32_prefill(Hq, Hkv, S, causal):
    say(f"D=32 prefill {Hq}/{Hkv} S={S} causal={causal}")
    o, ref = _prefill_case(2, S, Hq, Hkv, D32, torch.bfloat16, seed=3210 + S, causal=causal)
    assert_bf16_close(o, ref, "D=32 prefill")


def test_d32_prefill_bottom_right_and_lse():
    say("D=32 prefill S<T + lse")
    B, S, T, Hq, Hkv = 2, 45, 203, 8, 2
    q = randn(B, Hq, S, D32, seed=3221, dtype=torch.bfloat16)
    k = randn(B, Hkv, T, D32, seed=3222, dtype=torch.bfloat16)
    v = randn(B, Hkv, T, D32, seed=3223, dtype=torch.bfloat16)
    o, lse = nq.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, return_lse=True)
    assert_bf16_close(o, attention(q.float(), k.float(), v.float(), causal=True, causal_offset=T - S), "S<T")
    s = torch.matmul(q.float(), k.float().repeat_interleave(4, 1).transpose(-1, -2)) / math.sqrt(D32)
    keep = torch.arange(T)[None, :] <= torch.arange(S)[:, None] + (T - S)
    ref_lse = torch.logsumexp(s.masked_fill(~keep, float("-inf")), -1)
    torch.testing.assert_close(lse.cpu(), ref_lse, rtol=1e-3, atol=2e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("chunk", [32, 0])
@pytest.mark.parametrize("Hq,Hkv", [(8, 2), (32, 1)])
def test_d32_decode(dtype, chunk, Hq, Hkv):
    say(f"D=32 decode {dtype} chunk={chunk} {Hq}/{Hkv}")
    B, Tcap = 4, 300
    lens = torch.tensor([1, 100, 300, 64], dtype=torch.int32)
    q = randn(B, Hq, D32, seed=3231, dtype=dtype)
    kc = randn(B, Hkv, Tcap, D32, seed=3232, dtype=dtype)
    vc = randn(B, Hkv, Tcap, D32, seed=3233, dtype=dtype)
    for b, L in enumerate(lens.tolist()):
        kc[b, :, L:] = float("nan")
        vc[b, :, L:] = float("nan")
    qw = 1 + 0.02 * randn(D32, seed=3234)
    cos, sin = rope_tables(D32, 512, 1e4)
    o = nq.attention_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), max_len=Tcap, q_weight=qw.to(DEV),
                            eps=1e-6, cos=cos.to(DEV), sin=sin.to(DEV), chunk=chunk)
    ref = decode_path(q.float(), kc.float(), vc.float(), lens, q_weight=qw, eps=1e-6, cos=cos, sin=sin,
                      q_pos=lens.long() - 1)
    assert torch.isfinite(o.float().cpu()).all()
    assert_close_for(dtype, o, ref, "D=32 decode")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_d32_paged_fused_append(dtype):
    """New K/V appended inside the decode launch: output and written rows vs the oracle."""
    say(f"D=32 paged fused append {dtype}")
    B, Hq, Hkv, P, npages = 3, 8, 2, 32, 24
    lens = torch.tensor([0, 31, 70], dtype=torch.int32)
    g = torch.Generator().manual_seed(3241)
    perm = torch.randperm(npages, generator=g).to(torch.int32)
    bt = perm[:B * 4].view(B, 4)
    kpool = torch.full((npages, Hkv, P, D32), float("nan"), dtype=dtype)
    vpool = torch.full_like(kpool, float("nan"))
    kdense = randn(B, Hkv, 128, D32, seed=3242, dtype=dtype)
    vdense = randn(B, Hkv, 128, D32, seed=3243, dtype=dtype)
    for b in range(B):
        for t in range(int(lens[b])):
            kpool[int(bt[b, t // P]), :, t % P] = kdense[b, :, t]
            vpool[int(bt[b, t // P]), :, t % P] = vdense[b, :, t]
    q = randn(B, Hq, D32, seed=3244, dtype=dtype)
    kn = randn(B, Hkv, D32, seed=3245, dtype=dtype)
    vn = randn(B, Hkv, D32, seed=3246, dtype=dtype)
    qw = 1 + 0.02 * randn(D32, seed=3247)
    kw = 1 + 0.02 * randn(D32, seed=3248)
    cos, sin = rope_tables(D32, 256, 1e4)
    kp, vp, ld = kpool.to(DEV), vpool.to(DEV), lens.to(DEV)
    lens_out = torch.empty_like(ld)
    o = nq.attention_decode_paged(q.to(DEV), kp, vp, bt.to(DEV), ld, max_len=128, k_new=kn.to(DEV),
                                  v_new=vn.to(DEV), k_weight=kw.to(DEV), lens_out=lens_out,
                                  q_weight=qw.to(DEV), eps=1e-6, cos=cos.to(DEV), sin=sin.to(DEV))
    assert lens_out.cpu().tolist() == (lens + 1).tolist()
    for b in range(B):
        t = int(lens[b])
        kdense[b, :, t] = rotate_half(rms_norm(kn[b].float(), kw, 1e-6), cos[t], sin[t]).to(dtype)
        vdense[b, :, t] = vn[b]
    ref = decode_path(q.float(), kdense.float(), vdense.float(), lens + 1, q_weight=qw, eps=1e-6, cos=cos,
                      sin=sin, q_pos=lens.long())
    assert_close_for(dtype, o, ref, "D=32 fused append")
    for b in range(B):
        t = int(lens[b])
        got = kp[int(bt[b, t // P]), :, t % P].float().cpu()
        if dtype == torch.float32:
            assert_fp32_close(got, kdense[b, :, t], "appended K-hat row")
        else:
            assert_bf16_close(got, kdense[b, :, t].float(), "appended K-hat row", max_abs=1e-2, mean_abs=2e-3)
        assert torch.equal(vp[int(bt[b, t // P]), :, t % P].cpu(), vn[b])


def test_d32_merge():
    say("D=32 merge")
    B, H, S, T = 2, 4, 60, 150
    q = randn(B, H, S, D32, seed=3251, dtype=torch.bfloat16).to(DEV)
    k = randn(B, H, T, D32, seed=3252, dtype=torch.bfloat16).to(DEV)
    v = randn(B, H, T, D32, seed=3253, dtype=torch.bfloat16).to(DEV)
    o1, l1 = nq.attention_prefill(q, k[:, :, :70], v[:, :, :70], causal=False, return_lse=True)
    o2, l2 = nq.attention_prefill(q, k[:, :, 70:], v[:, :, 70:], causal=False, return_lse=True)
    o1 = o1.contiguous()
    nq.attention_merge_(o1, l1, o2, l2)
    assert_bf16_close(o1, attention(q.float().cpu(), k.float().cpu(), v.float().cpu()), "merge")


@pytest.mark.parametrize("causal", [True, False])
def test_d32_backward(causal):
    say(f"D=32 backward causal={causal}")
    B, Hq, Hkv, S = 2, 8, 2, 200
    q = randn(B, Hq, S, D32, seed=3261, dtype=torch.bfloat16)
    k = randn(B, Hkv, S, D32, seed=3262, dtype=torch.bfloat16)
    v = randn(B, Hkv, S, D32, seed=3263, dtype=torch.bfloat16)
    do = randn(B, Hq, S, D32, seed=3264, dtype=torch.bfloat16)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=causal)
    qd, kd, vd = (t.double().requires_grad_(True) for t in (q, k, v))
    attention(qd, kd, vd, causal=causal, compute_dtype=torch.float64).backward(do.double())
    for got, ref, name in ((dq, qd.grad, "dq"), (dk, kd.grad, "dk"), (dv, vd.grad, "dv")):
        d = (got.double().cpu() - ref).abs()
        sc = float(ref.abs().max())
        assert float(d.max()) <= 2e-2 * sc and float(d.mean()) <= 2e-3 * sc, f"{name}: {float(d.max()):.3e}"


def test_d32_norm_rope_backward():
    say("D=32 QK-Norm + RoPE backward")
    B, H, S = 2, 4, 50
    x = randn(B, H, S, D32, seed=3271)
    dy = randn(B, H, S, D32, seed=3272)
    w = 1 + 0.1 * randn(D32, seed=3273)
    cos, sin = rope_tables(D32, 64, 1e4)
    dx, dw = ops.qk_norm_rope_backward(x.to(DEV), dy.to(DEV), weight=w.to(DEV), eps=1e-6, cos=cos.to(DEV),
                                       sin=sin.to(DEV))
    xd, wd = x.double().requires_grad_(True), w.double().requires_grad_(True)
    y = rotate_half(rms_norm(xd, wd, 1e-6, torch.float64), cos[:S].double()[None, None], sin[:S].double()[None, None])
    y.backward(dy.double())
    torch.testing.assert_close(dx.double().cpu(), xd.grad, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(dw.double().cpu(), wd.grad, rtol=1e-4, atol=1e-3)


def _debug_yaml_module(dtype):
    """configs/model/debug.yaml's attention: hidden 256, 8 heads, 2 kv heads (head_dim 32),
    max_position_embeddings 2048, rope_theta 1e4, rms_norm_eps 1e-6, qk_norm."""
    cfg = nq.AttentionConfig(hidden_size=256, num_attention_heads=8, num_key_value_heads=2,
                             max_position_embeddings=2048, rope_theta=1e4, rms_norm_eps=1e-6)
    torch.manual_seed(3280)
    attn = nq.Attention(cfg).eval()
    with torch.no_grad():
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            getattr(attn, name).weight.normal_(0, 0.06)
        attn.q_norm.weight.copy_(1 + 0.05 * torch.randn(32))
        attn.k_norm.weight.copy_(1 + 0.05 * torch.randn(32))
    w = {n: getattr(attn, n).weight.detach().clone() for n in ("q_proj", "k_proj", "v_proj", "o_proj")}
    w["q_norm"], w["k_norm"] = attn.q_norm.weight.detach().clone(), attn.k_norm.weight.detach().clone()
    return cfg, attn.to(device=DEV, dtype=dtype), w


@torch.no_grad()
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_debug_yaml_attention_module(dtype):
    """B2 S256, no cache and the generate.py cache protocol (prefill + 3 one-token steps)."""
    say(f"debug.yaml Attention module {dtype}")
    cfg, attn, w = _debug_yaml_module(dtype)
    # the oracle runs the reference's dtype flow for the module's dtype (bf16
    # projections, norm cast and cos/sin for a bf16 module; attention in fp32)
    w = {n: t.to(dtype) for n, t in w.items()}
    cos, sin = rope_tables(32, 2048, 1e4)
    kw = dict(num_heads=8, num_kv_heads=2, head_dim=32, eps=1e-6, cos_table=cos, sin_table=sin)
    h = randn(2, 256, 256, seed=3281, dtype=dtype)
    out = attn(h.to(DEV))
    ref, _ = attention_module_forward(h, w, **kw)
    if dtype == torch.float32:  # fp32 module: fp32 attention, fp32 gate
        assert_fp32_close(out, ref, "no cache")
    else:
        assert_bf16_close(out, ref, "no cache", max_abs=3e-2)
    cache, ocache = nq.KVCache(), OracleKVCache()
    steps = [randn(1, 40, 256, seed=3282, dtype=dtype)] + [randn(1, 1, 256, seed=3283 + i, dtype=dtype)
                                                           for i in range(3)]
    for i, x in enumerate(steps):
        got = attn(x.to(DEV), kv_cache=cache)
        want, _ = attention_module_forward(x, w, kv_cache=ocache, **kw)
        if dtype == torch.float32:
            assert_fp32_close(got, want, f"cache step {i}")
        else:
            assert_bf16_close(got, want, f"cache step {i}", max_abs=3e-2)
    assert cache.seq_len == ocache.seq_len == 43


# ------------------------------------------------------------------ positions

def test_out_of_range_positions_raise_on_the_host():
    say("positions out of range (host)")
    B, S, H, D = 1, 8, 2, 64
    cos, sin = (t.to(DEV) for t in rope_tables(D, 16, 1e6))
    x = randn(B, H, S, D, seed=3301, dtype=torch.bfloat16).to(DEV)
    with pytest.raises(IndexError):
        nq.qk_norm_rope(k=x, cos=cos, sin=sin, pos_offset=9)
    with pytest.raises(IndexError):
        nq.attention_prefill(x, x, x, cos=cos, sin=sin, position_ids=torch.arange(S) + 10)
    with pytest.raises(IndexError):
        nq.attention_decode(x[:, :, 0], x, x, None, max_len=S, cos=cos, sin=sin, q_pos0=16)
    cfg = nq.AttentionConfig(hidden_size=128, num_attention_heads=2, num_key_value_heads=2,
                             max_position_embeddings=16)
    attn = nq.Attention(cfg).to(DEV).eval()
    with torch.no_grad(), pytest.raises(IndexError):
        attn(torch.randn(1, 17, 128, device=DEV))
    with torch.no_grad():
        attn.rope_positions = "cache"
        cache = nq.KVCache()
        attn(torch.randn(1, 16, 128, device=DEV), kv_cache=cache)
        with pytest.raises(IndexError):
            attn(torch.randn(1, 1, 128, device=DEV), kv_cache=cache)


def test_out_of_range_device_positions_give_nan_rows():
    """Device positions cannot be read back without a sync: the rows they touch are NaN."""
    say("positions out of range (device)")
    B, S, Hq, Hkv, D = 1, 8, 2, 2, 64
    cos, sin = (t.to(DEV) for t in rope_tables(D, 16, 1e6))
    q = randn(B, Hq, S, D, seed=3311, dtype=torch.bfloat16).to(DEV)
    pos = torch.arange(S, device=DEV).view(1, S).clone()
    pos[0, 3] = 40
    qo = nq.qk_norm_rope(q=q, cos=cos, sin=sin, position_ids=pos)[0].float().cpu()
    assert torch.isnan(qo[0, :, 3]).all() and torch.isfinite(qo[0, :, [0, 1, 2, 4, 5, 6, 7]]).all()
    o = nq.attention_prefill(q, q, q, cos=cos, sin=sin, position_ids=pos, causal=True).float().cpu()
    assert torch.isnan(o[0, :, 3]).all() and torch.isfinite(o[0, :, :3]).all()
    dec = nq.attention_decode(q[:, :, 0], q, q, None, max_len=S, cos=cos, sin=sin,
                              q_pos=torch.tensor([99], device=DEV)).float().cpu()
    assert torch.isnan(dec).all()


@pytest.mark.parametrize("Hq,Hkv", [(2, 2), (8, 2)])
def test_pos_base_past_the_tables_gives_nan_rows(Hq, Hkv):
    """Per-sequence position bases (device tensor) run the prefill's staged cos/sin rows:
    the rows whose position lies past the tables are NaN, every other row matches the
    oracle at its own position."""
    say(f"prefill pos_base past the tables {Hq}/{Hkv}")
    B, S, D, max_pos = 2, 8, 64, 16
    cos, sin = rope_tables(D, max_pos, 1e6)
    q = randn(B, Hq, S, D, seed=3321, dtype=torch.bfloat16)
    k = randn(B, Hkv, S, D, seed=3322, dtype=torch.bfloat16)
    v = randn(B, Hkv, S, D, seed=3323, dtype=torch.bfloat16)
    w = torch.ones(D)
    base = torch.tensor([3, max_pos - 4], dtype=torch.int32)
    o = nq.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), q_weight=w.to(DEV), eps=1e-6, cos=cos.to(DEV),
                             sin=sin.to(DEV), pos_base=base.to(DEV), causal=True).float().cpu()
    assert torch.isnan(o[1, :, 4:]).all() and torch.isfinite(o[1, :, :4]).all() and torch.isfinite(o[0]).all()
    from oracle import rms_norm, rotate_half
    for bi in range(B):
        pos = torch.arange(S) + int(base[bi])
        ok = pos < max_pos
        qh = rms_norm(q[bi:bi + 1].float(), w, 1e-6)
        qh = rotate_half(qh, cos[pos.clamp(max=max_pos - 1)][None, None], sin[pos.clamp(max=max_pos - 1)][None, None])
        ref = attention(qh, k[bi:bi + 1].float(), v[bi:bi + 1].float(), causal=True)[0]
        assert_bf16_close(o[bi][:, ok], ref[:, ok], f"pos_base row {bi}")


# ------------------------------------------------------------------ RMSNorm mirror

@pytest.mark.parametrize("width", [32, 128, 256, 2048])
@pytest.mark.parametrize("xdt,wdt", [(torch.bfloat16, torch.float32), (torch.float32, torch.float32),
                                     (torch.bfloat16, torch.bfloat16)])
def test_rmsnorm_mirror_promotion_and_widths(width, xdt, wdt):
    say(f"RMSNorm width={width} x={xdt} w={wdt}")
    x = randn(3, 5, width, seed=3321, dtype=xdt)
    norm = nq.RMSNorm(width, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * randn(width, seed=3322))
    norm = norm.to(DEV, wdt)
    with torch.no_grad():
        y = norm(x.to(DEV))
    ref = rms_norm(x, norm.weight.detach().cpu(), 1e-6)  # the reference's cast order (norm.py:21-22)
    assert y.dtype == ref.dtype == torch.promote_types(xdt, wdt)
    tol = 1e-5 if ref.dtype == torch.float32 and xdt == torch.float32 else 1e-2
    torch.testing.assert_close(y.float().cpu(), ref.float(), rtol=tol, atol=tol)


@pytest.mark.parametrize("width", [64, 256, 2048])
@pytest.mark.parametrize("xdt,wdt", [(torch.bfloat16, torch.float32), (torch.float32, torch.float32)])
def test_rmsnorm_mirror_autograd_any_width(width, xdt, wdt):
    """RMSNorm under autograd at QK-Norm widths and hidden-size widths: the
    gradients of the reference's composition (norm.py:17-22, autograd on the
    CPU with the same casts), dw reduced from the fp32 incoming gradient."""
    say(f"RMSNorm autograd width={width} x={xdt} w={wdt}")
    x = randn(4, 7, width, seed=3331, dtype=xdt)
    w0 = 1 + 0.1 * randn(width, seed=3332)
    dy = randn(4, 7, width, seed=3333)
    norm = nq.RMSNorm(width, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w0)
    norm = norm.to(DEV, wdt)
    xd = x.to(DEV).requires_grad_(True)
    y = norm(xd)
    y.backward(dy.to(DEV, y.dtype))
    xr = x.clone().requires_grad_(True)
    wr = w0.to(wdt).clone().requires_grad_(True)
    yr = rms_norm(xr, wr, 1e-6)
    yr.backward(dy.to(yr.dtype))
    assert y.dtype == yr.dtype
    tol = 1e-5 if xdt == torch.float32 else 2e-2
    torch.testing.assert_close(y.detach().float().cpu(), yr.detach().float(), rtol=tol, atol=tol)
    torch.testing.assert_close(xd.grad.float().cpu(), xr.grad.float(), rtol=tol, atol=tol)
    sc = float(wr.grad.abs().max())
    torch.testing.assert_close(norm.weight.grad.float().cpu(), wr.grad.float(), rtol=0, atol=1e-4 * sc)


# ------------------------------------------------------------------ decode positions, overflow

def test_decode_position_ids_broadcast():
    """position_ids of shape (1, 1) with B > 1 broadcast over the batch, as cos_cached[position_ids]."""
    say("decode position_ids (1,1) broadcast")
    cfg = nq.AttentionConfig(hidden_size=256, num_attention_heads=4, num_key_value_heads=2,
                             max_position_embeddings=512)
    torch.manual_seed(3331)
    attn = nq.Attention(cfg).to(DEV).eval()
    B = 3
    with torch.no_grad():
        cache_a, cache_b = nq.KVCache(), nq.KVCache()
        h = torch.randn(B, 20, 256, device=DEV)
        attn(h, kv_cache=cache_a)
        attn(h, kv_cache=cache_b)
        x = torch.randn(B, 1, 256, device=DEV)
        a = attn(x, position_ids=torch.tensor([[20]], device=DEV), kv_cache=cache_a)
        b = attn(x, position_ids=torch.full((B, 1), 20, device=DEV), kv_cache=cache_b)
    assert torch.equal(a, b)


def test_fused_append_overflow_rows_are_nan_and_untouched():
    say("fused append overflow rows")
    B, Hq, Hkv, D, P = 3, 4, 2, 64, 32
    dt = torch.bfloat16
    kpool = randn(B, Hkv, P, D, seed=3341, dtype=dt).to(DEV)
    vpool = randn(B, Hkv, P, D, seed=3342, dtype=dt).to(DEV)
    k0, v0 = kpool.clone(), vpool.clone()
    bt = torch.arange(B, dtype=torch.int32, device=DEV).view(B, 1)
    lens = torch.tensor([5, 32, 31], dtype=torch.int32, device=DEV)  # row 1 is full
    lens_out = torch.empty_like(lens)
    q = randn(B, Hq, D, seed=3343, dtype=dt).to(DEV)
    kn = randn(B, Hkv, D, seed=3344, dtype=dt).to(DEV)
    vn = randn(B, Hkv, D, seed=3345, dtype=dt).to(DEV)
    o = nq.attention_decode_paged(q, kpool, vpool, bt, lens, max_len=32, k_new=kn, v_new=vn,
                                  lens_out=lens_out).float().cpu()
    assert lens_out.cpu().tolist() == [6, 32, 32]
    assert torch.isnan(o[1]).all() and torch.isfinite(o[[0, 2]]).all()
    assert torch.equal(kpool[1], k0[1]) and torch.equal(vpool[1], v0[1])
    assert torch.equal(vpool[2, :, 31], vn[2]) and torch.equal(vpool[0, :, 5], vn[0])


# ------------------------------------------------------------------ wide groups, many rows

@pytest.mark.parametrize("Hq,Hkv", [(32, 1), (64, 1)])
def test_prefill_widest_groups(Hq, Hkv):
    say(f"prefill G={Hq // Hkv}")
    for S in (5, 130):
        o, ref = _prefill_case(1, S, Hq, Hkv, 64, torch.bfloat16, seed=3350 + S, theta=1e6)
        assert_bf16_close(o, ref, f"G={Hq // Hkv} S={S}")


@pytest.mark.parametrize("paged", [False, True])
def test_decode_batch_past_64_rows(paged):
    """B = 100: lens read from memory (not a register) and the multi-window prefix scan."""
    say(f"decode B=100 paged={paged}")
    B, Hq, Hkv, D, Tcap = 100, 8, 2, 64, 640
    g = torch.Generator().manual_seed(3361)
    lens = torch.randint(1, Tcap, (B,), generator=g, dtype=torch.int32)
    lens[::17] = 0 if not paged else lens[::17]
    kc = randn(B, Hkv, Tcap, D, seed=3362, dtype=torch.bfloat16)
    vc = randn(B, Hkv, Tcap, D, seed=3363, dtype=torch.bfloat16)
    q = randn(B, Hq, D, seed=3364, dtype=torch.bfloat16)
    cos, sin = rope_tables(D, Tcap + 1, 1e6)
    if not paged:
        o = nq.attention_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), max_len=Tcap,
                                cos=cos.to(DEV), sin=sin.to(DEV)).float().cpu()
        for b in range(B):
            if lens[b] == 0:
                assert (o[b] == 0).all()
                continue
            ref = decode_path(q[b:b + 1].float(), kc[b:b + 1].float(), vc[b:b + 1].float(), lens[b:b + 1],
                              q_weight=None, eps=1e-6, cos=cos, sin=sin, q_pos=lens[b:b + 1].long() - 1)
            assert_bf16_close(o[b:b + 1], ref, f"row {b}")
        return
    kn = randn(B, Hkv, D, seed=3365, dtype=torch.bfloat16)
    vn = randn(B, Hkv, D, seed=3366, dtype=torch.bfloat16)
    bt = torch.arange(B, dtype=torch.int32).view(B, 1)
    kd, vd, ld = kc.to(DEV), vc.to(DEV), lens.to(DEV)
    lens_out = torch.empty_like(ld)
    o = nq.attention_decode_paged(q.to(DEV), kd, vd, bt.to(DEV), ld, max_len=Tcap, k_new=kn.to(DEV),
                                  v_new=vn.to(DEV), lens_out=lens_out, cos=cos.to(DEV),
                                  sin=sin.to(DEV)).float().cpu()
    assert lens_out.cpu().tolist() == (lens + 1).tolist()
    for b in range(B):
        t = int(lens[b])
        kc[b, :, t] = rotate_half(kn[b].float(), cos[t], sin[t]).to(torch.bfloat16)
        vc[b, :, t] = vn[b]
        ref = decode_path(q[b:b + 1].float(), kc[b:b + 1].float(), vc[b:b + 1].float(), lens[b:b + 1] + 1,
                          q_weight=None, eps=1e-6, cos=cos, sin=sin, q_pos=lens[b:b + 1].long())
        assert_bf16_close(o[b:b + 1], ref, f"row {b}")


# ------------------------------------------------------------------ plain KVCache one-token step

@torch.no_grad()
def test_plain_cache_step_is_one_fused_call_and_bit_equal():
    """The unragged KVCache's one-token step runs one nq_attn_decode_paged_fwd call (two
    kernels: stream + merge) and gives the same bits as the row-kernel append + decode."""
    say("plain KVCache fused step")
    cfg = nq.AttentionConfig(hidden_size=512, num_attention_heads=8, num_key_value_heads=4,
                             max_position_embeddings=1024)
    torch.manual_seed(3371)
    attn = nq.Attention(cfg).to(DEV, torch.bfloat16).eval()
    B = 2
    h = torch.randn(B, 50, 512, device=DEV, dtype=torch.bfloat16)
    cache = nq.KVCache()
    attn(h, kv_cache=cache)
    kc0, vc0 = (t.clone() for t in cache.storage())
    x = torch.randn(B, 1, 512, device=DEV, dtype=torch.bfloat16)
    calls = []
    lib = nq._lib.load()
    orig = {n: getattr(lib, n) for n in ("nq_attn_decode_paged_fwd", "nq_qk_norm_rope", "nq_attn_decode_fwd")}
    try:
        for n, fn in orig.items():
            setattr(lib, n, (lambda f, name: (lambda *a: (calls.append(name), f(*a))[1]))(fn, n))
        out = attn(x, kv_cache=cache)
    finally:
        for n, fn in orig.items():
            setattr(lib, n, fn)
    assert calls == ["nq_attn_decode_paged_fwd"]
    # the same step the row-kernel way: append K-hat/V rows, then decode
    H, Hkv, D = 8, 4, 64
    q4 = attn.q_proj(x).view(B, 1, H, D).transpose(1, 2)
    k4 = attn.k_proj(x).view(B, 1, Hkv, D).transpose(1, 2)
    v4 = attn.v_proj(x).view(B, 1, Hkv, D).transpose(1, 2)
    cos, sin = attn.rotary_emb.tables_f32()
    nq.qk_norm_rope(k=k4, v=v4, k_out=kc0, v_out=vc0, k_weight=attn.k_norm.weight, eps=1e-6, cos=cos, sin=sin,
                    kv_row_offset=50)
    o = nq.attention_decode(q4, kc0, vc0, None, max_len=51, q_weight=attn.q_norm.weight, eps=1e-6, cos=cos,
                            sin=sin, q_pos0=0)
    kc, vc = cache.storage()
    assert torch.equal(kc[:, :, :51], kc0[:, :, :51]) and torch.equal(vc[:, :, :51], vc0[:, :, :51])
    assert torch.equal(out, attn.o_proj(o.reshape(B, 1, H * D)))
    assert cache.seq_len == 51


# ------------------------------------------------------------------ use_triton keyword

@torch.no_grad()
def test_use_triton_keyword_selects_nothing():
    """kernels/flash_attn.py:136 and kernels/rope.py:104 take use_triton; the
    mirrors accept it and give the same bits for True and False."""
    say("use_triton keyword: flash_attention / apply_rope")
    B, S, H, D = 2, 200, 4, 128
    q = randn(B, H, S, D, seed=4101, dtype=torch.bfloat16).to(DEV)
    k = randn(B, H, S, D, seed=4102, dtype=torch.bfloat16).to(DEV)
    v = randn(B, H, S, D, seed=4103, dtype=torch.bfloat16).to(DEV)
    outs = [nq.flash_attention(q, k, v, causal=True, use_triton=ut) for ut in (True, False)]
    outs.append(nq.flash_attention(q, k, v, True, None, False))  # positional, as the reference allows
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    ref = attention(q.float().cpu(), k.float().cpu(), v.float().cpu(), causal=True)
    assert_bf16_close(outs[0], ref, "flash_attention")
    cos, sin = rope_tables(D, S, 1e6)
    cos, sin = cos.to(DEV), sin.to(DEV)
    rot = []
    for ut in (True, False):
        qq, kk = q.clone(), k.clone()
        r = nq.apply_rope(qq, kk, cos, sin, use_triton=ut)
        assert r[0] is qq and r[1] is kk  # in place, as kernels/rope.py does
        rot.append((qq, kk))
    assert torch.equal(rot[0][0], rot[1][0]) and torch.equal(rot[0][1], rot[1][1])
    c, s = cos.cpu()[None, None], sin.cpu()[None, None]
    assert_bf16_close(rot[0][0], rotate_half(q.float().cpu(), c, s), "apply_rope q")
