"""Key-padding masks on the kernels (model/attention.py:110-114 with attn_mask,
the reward model's padded batches, training/reward_model.py:45).

A mask that keeps, for every head and query, the same prefix [0, L_b) of each
sequence's keys runs the prefill (and, under autograd, the backward) kernels
with per-sequence key counts; any other mask takes SDPA.  References: the
oracle's attention with key_lens / the mask (fp32 math, fp64 for gradients).
Padded K/V rows are poisoned with NaN: the kernels must never read them.
"""

import pytest
import torch

import nano_qwen_amd as nq
from nano_qwen_amd import ops
from oracle import attention, attention_module_forward, rope_tables
from tests.helpers import assert_bf16_close, assert_close_for, randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _poison(t, lens):
    t = t.clone()
    for b, L in enumerate(lens.tolist()):
        t[b, :, L:] = float("nan")
    return t


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("Hq,Hkv", [(8, 2), (4, 4)])
def test_prefill_key_lens(dtype, D, Hq, Hkv):
    say(f"prefill key_lens {dtype} D={D} {Hq}/{Hkv}")
    B, S = 3, 150
    lens = torch.tensor([150, 1, 77], dtype=torch.int32)
    q = randn(B, Hq, S, D, seed=701, dtype=dtype)
    k = _poison(randn(B, Hkv, S, D, seed=702, dtype=dtype), lens)
    v = _poison(randn(B, Hkv, S, D, seed=703, dtype=dtype), lens)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=False, key_lens=lens.to(DEV),
                                   return_lse=True)
    ref = attention(q.float(), k.float().nan_to_num(), v.float().nan_to_num(), key_lens=lens)
    assert torch.isfinite(o.float()).all()
    assert_close_for(dtype, o, ref, "key_lens")
    s = torch.matmul(q.float(), k.float().nan_to_num().repeat_interleave(Hq // Hkv, 1).transpose(-1, -2))
    s = (s / D ** 0.5).masked_fill(torch.arange(S)[None, None, None, :] >= lens.view(B, 1, 1, 1), float("-inf"))
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(lse.cpu(), torch.logsumexp(s, -1), rtol=0, atol=tol)


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (8, 2)])
def test_prefill_key_lens_zero_and_out_of_range(Hq, Hkv):
    """0 keys: zero rows; a count outside [0, T]: NaN rows (lse -inf), for every
    head of the group."""
    say(f"prefill key_lens edge values {Hq}/{Hkv}")
    B, S, D = 3, 40, 64
    lens = torch.tensor([0, 41, 40], dtype=torch.int32)
    q = randn(B, Hq, S, D, seed=710, dtype=torch.bfloat16).to(DEV)
    k, v = (randn(B, Hkv, S, D, seed=711 + i, dtype=torch.bfloat16).to(DEV) for i in range(2))
    o, lse = ops.attention_prefill(q, k, v, causal=False, key_lens=lens.to(DEV), return_lse=True)
    o = o.float().cpu()
    assert not o[0].abs().any() and torch.isnan(o[1]).all() and torch.isfinite(o[2]).all()
    assert torch.isinf(lse[:2].cpu()).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_backward_key_lens(dtype, D):
    """Gradients of attention over each sequence's unpadded keys; padded keys get zero dK, dV."""
    say(f"backward key_lens {dtype} D={D}")
    B, Hq, Hkv, S = 3, 8, 2, 100
    lens = torch.tensor([100, 37, 1], dtype=torch.int32)
    q = randn(B, Hq, S, D, seed=721, dtype=dtype)
    k = _poison(randn(B, Hkv, S, D, seed=722, dtype=dtype), lens)
    v = _poison(randn(B, Hkv, S, D, seed=723, dtype=dtype), lens)
    do = randn(B, Hq, S, D, seed=724, dtype=dtype)
    kl = lens.to(DEV)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=False, key_lens=kl, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=False,
                                        key_lens=kl)
    qd, kd, vd = (t.double().nan_to_num().requires_grad_(True) for t in (q, k, v))
    attention(qd, kd, vd, key_lens=lens, compute_dtype=torch.float64).backward(do.double())
    mx_tol, mean_tol = (1e-5, 1e-6) if dtype == torch.float32 else (2e-2, 2e-3)
    for got, ref, name in ((dq, qd.grad, "dq"), (dk, kd.grad, "dk"), (dv, vd.grad, "dv")):
        got = got.double().cpu()
        assert torch.isfinite(got).all(), name
        sc = float(ref.abs().max())
        d = (got - ref).abs()
        assert float(d.max()) <= mx_tol * sc and float(d.mean()) <= mean_tol * sc, \
            f"{name}: max-abs {float(d.max()):.3e} mean-abs {float(d.mean()):.3e} (ref max {sc:.3e})"
    for b, L in enumerate(lens.tolist()):
        assert not dk[b, :, L:].float().abs().any() and not dv[b, :, L:].float().abs().any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("T", [130, 161])
def test_causal_with_key_lens_forward_and_backward(dtype, D, T):
    """Causal attention with per-sequence key counts: the frontier is
    bottom-right against the launch's T (query i keeps keys j <= i + T - S) and
    key_lens only shortens the key range, in the fp32 and bf16 kernels alike,
    forward and backward.  Rows before a short sequence's first key are the
    case an offset taken from key_lens instead of T would turn into NaN."""
    say(f"causal + key_lens {dtype} D={D} T={T}")
    B, Hq, Hkv, S = 3, 8, 2, 130
    lens = torch.tensor([T, 3, 90], dtype=torch.int32)
    q = randn(B, Hq, S, D, seed=741, dtype=dtype)
    k = _poison(randn(B, Hkv, T, D, seed=742, dtype=dtype), lens)
    v = _poison(randn(B, Hkv, T, D, seed=743, dtype=dtype), lens)
    do = randn(B, Hq, S, D, seed=744, dtype=dtype)
    kl = lens.to(DEV)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, key_lens=kl, return_lse=True)
    assert torch.isfinite(o.float()).all() and torch.isfinite(lse).all()
    ref = attention(q.float(), k.float().nan_to_num(), v.float().nan_to_num(), causal=True,
                    causal_offset=T - S, key_lens=lens)
    assert_close_for(dtype, o, ref, "causal + key_lens forward")
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=True,
                                        key_lens=kl)
    qd, kd, vd = (t.double().nan_to_num().requires_grad_(True) for t in (q, k, v))
    attention(qd, kd, vd, causal=True, causal_offset=T - S, key_lens=lens,
              compute_dtype=torch.float64).backward(do.double())
    mx_tol, mean_tol = (1e-5, 1e-6) if dtype == torch.float32 else (2e-2, 2e-3)
    for got, want, name in ((dq, qd.grad, "dq"), (dk, kd.grad, "dk"), (dv, vd.grad, "dv")):
        got = got.double().cpu()
        assert torch.isfinite(got).all(), name
        sc = float(want.abs().max())
        d = (got - want).abs()
        assert float(d.max()) <= mx_tol * sc and float(d.mean()) <= mean_tol * sc, \
            f"{name}: max-abs {float(d.max()):.3e} mean-abs {float(d.mean()):.3e} (ref max {sc:.3e})"


def _module(dtype, seed=731):
    cfg = nq.AttentionConfig(hidden_size=256, num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                             max_position_embeddings=512)
    torch.manual_seed(seed)
    attn = nq.Attention(cfg)
    with torch.no_grad():
        attn.q_norm.weight.add_(0.1 * torch.randn(64))
        attn.k_norm.weight.add_(0.1 * torch.randn(64))
    attn = attn.to(DEV, dtype)
    names = ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm")
    return attn, {n: getattr(attn, n).weight.detach().cpu() for n in names}


def _masks(kind, lens, S):
    B = lens.numel()
    keep = torch.arange(S)[None, :] < lens[:, None]
    if kind == "bool4d":
        return keep[:, None, None, :]
    if kind == "float4d":
        return torch.zeros(B, 1, 1, S).masked_fill(~keep[:, None, None, :], float("-inf"))
    if kind == "bool2d":  # (1, T): SDPA broadcasts it over the batch as a key mask
        return keep[:1]
    raise ValueError(kind)


@torch.no_grad()
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["bool4d", "float4d", "bool2d"])
def test_module_key_padding_mask_runs_the_kernels(dtype, kind):
    say(f"module key-padding mask {kind} {dtype}")
    attn, w = _module(dtype)
    S = 96
    lens = torch.tensor([96, 60, 1]) if kind != "bool2d" else torch.tensor([70])
    B = lens.numel()
    mask = _masks(kind, lens, S)
    if mask.is_floating_point():
        mask = mask.to(dtype)
    h = randn(B, S, 256, seed=732, dtype=dtype)
    before = nq.stats["kernel_forward"]
    out = attn(h.to(DEV), attention_mask=mask.to(DEV))
    assert nq.stats["kernel_forward"] == before + 1, "the key-padding mask did not take the kernels"
    cos, sin = rope_tables(64, 512, 1e6)
    ref, _ = attention_module_forward(h, {n: t.to(dtype) for n, t in w.items()}, num_heads=8, num_kv_heads=2,
                                      head_dim=64, eps=1e-6, cos_table=cos, sin_table=sin, attention_mask=mask)
    if dtype == torch.float32:
        assert_close_for(dtype, out, ref, f"mask {kind}")
    else:  # the bf16 module's projections round too (the bf16 module gate)
        assert_bf16_close(out, ref, f"mask {kind}", max_abs=3e-2)


@torch.no_grad()
def test_module_other_masks_take_sdpa():
    """Left padding (a hole before the kept keys), a query-dependent mask and an
    additive bias are not key-padding prefixes: they run SDPA, as the reference."""
    say("module non-prefix masks -> SDPA")
    attn, w = _module(torch.float32)
    B, S = 2, 32
    h = randn(B, S, 256, seed=741)
    cos, sin = rope_tables(64, 512, 1e6)
    left = (torch.arange(S)[None, :] >= torch.tensor([0, 5])[:, None])[:, None, None, :]
    causal = torch.ones(S, S, dtype=torch.bool).tril()
    bias = 0.1 * randn(1, 1, 1, S, seed=742)
    for mask in (left, causal, bias):
        before = nq.stats["torch_forward"]
        out = attn(h.to(DEV), attention_mask=mask.to(DEV))
        assert nq.stats["torch_forward"] == before + 1
        ref, _ = attention_module_forward(h, w, num_heads=8, num_kv_heads=2, head_dim=64, eps=1e-6,
                                          cos_table=cos, sin_table=sin, attention_mask=mask)
        assert_close_for(torch.float32, out, ref, "sdpa path")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_training_with_key_padding(dtype):
    """A reward-model-style padded batch under autograd: forward and backward on the
    kernels, every weight gradient against fp64 autograd of the oracle module."""
    say(f"module training with key padding {dtype}")
    attn, w = _module(dtype, seed=751)
    attn.train()
    B, S = 3, 80
    lens = torch.tensor([80, 33, 5])
    mask = _masks("bool4d", lens, S)
    h = randn(B, S, 256, seed=752, dtype=dtype)
    g = randn(B, S, 256, seed=753, dtype=dtype)
    before = nq.stats["kernel_train_forward"]
    out = attn(h.to(DEV), attention_mask=mask.to(DEV))
    out.backward(g.to(DEV))
    assert nq.stats["kernel_train_forward"] == before + 1
    cos, sin = rope_tables(64, 512, 1e6)
    wd = {n: t.double().requires_grad_(True) for n, t in w.items()}
    ref, _ = attention_module_forward(h.double(), wd, num_heads=8, num_kv_heads=2, head_dim=64, eps=1e-6,
                                      cos_table=cos.double(), sin_table=sin.double(), attention_mask=mask)
    ref.backward(g.double())
    mx_tol, mean_tol = (1e-5, 1e-6) if dtype == torch.float32 else (5e-2, 5e-3)
    for n, t in wd.items():
        got = getattr(attn, n).weight.grad.double().cpu()
        sc = float(t.grad.abs().max())
        d = (got - t.grad).abs()
        assert float(d.max()) <= mx_tol * sc and float(d.mean()) <= mean_tol * sc, \
            f"grad {n}: max-abs {float(d.max()):.3e} mean-abs {float(d.mean()):.3e} (ref max {sc:.3e})"
