"""Attention masks on the kernels (model/attention.py:110-114 with attn_mask,
the reward model's padded batches, training/reward_model.py:45).

A mask that keeps, for every head and query, the same prefix [0, L_b) of each
sequence's keys runs the prefill (and, under autograd, the backward) kernels
with per-sequence key counts; any other bool or float mask runs them with an
additive bias read per tile (ops.AttnBias).  No mask takes a torch path.
References: the oracle's attention with key_lens / the mask (fp32 math, fp64
for gradients; a row with every key masked gives zeros, as SDPA does, pinned
against SDPA in the oracle tests).  Padded K/V rows are poisoned with NaN: the
kernels must never read them.
"""

import pytest
import torch

import nano_qwen_amd as nq
from nano_qwen_amd import ops
from oracle import OracleKVCache, attention, attention_module_forward, rope_tables
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
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_other_masks_run_the_bias_kernels(dtype):
    """Left padding (a hole before the kept keys), a query-dependent mask, an
    additive bias and a per-head mask are not key-padding prefixes: they run the
    kernels with the mask as a per-tile bias, and match the oracle module."""
    say(f"module non-prefix masks -> bias kernels {dtype}")
    attn, w = _module(dtype)
    B, S = 2, 32
    h = randn(B, S, 256, seed=741, dtype=dtype)
    cos, sin = rope_tables(64, 512, 1e6)
    left = (torch.arange(S)[None, :] >= torch.tensor([0, 5])[:, None])[:, None, None, :]
    causal = torch.ones(S, S, dtype=torch.bool).tril()
    bias = (0.1 * randn(1, 1, 1, S, seed=742)).to(dtype)
    heads = torch.rand(1, 8, S, S, generator=torch.Generator().manual_seed(743)) > 0.5
    heads[..., 0] = True
    for mask in (left, causal, bias, heads):
        before = dict(nq.stats)
        out = attn(h.to(DEV), attention_mask=mask.to(DEV))
        assert nq.stats["torch_forward"] == before["torch_forward"] == 0
        assert nq.stats["kernel_forward"] == before["kernel_forward"] + 1
        ref, _ = attention_module_forward(h, {k: v.to(dtype) for k, v in w.items()}, num_heads=8, num_kv_heads=2,
                                          head_dim=64, eps=1e-6, cos_table=cos, sin_table=sin, attention_mask=mask)
        if dtype == torch.float32:
            assert_close_for(dtype, out, ref, "bias kernels")
        else:
            assert_bf16_close(out, ref, "bias kernels", max_abs=3e-2)


def _bias_masks(kind, B, Hq, S, T, dtype, seed):
    """Masks broadcastable to (B, Hq, S, T): bool keep-masks (with fully masked rows)
    and float biases (with -inf entries and large finite offsets)."""
    g = torch.Generator().manual_seed(seed)
    if kind == "bool":
        m = torch.rand(B, 1, S, T, generator=g) > 0.35
        m[0, 0, 5] = False                                   # a row with no key at all
        m[-1, 0, :, :70] = False                             # rows whose first tile(s) are all masked
        return m
    if kind == "float":
        m = 0.5 * torch.randn(B, 1, S, T, generator=g)
        m = m.masked_fill(torch.rand(B, 1, S, T, generator=g) < 0.3, float("-inf"))
        m[0, 0, 7] = float("-inf")
        return m.to(dtype)
    if kind == "heads":                                      # per-head, broadcast over the batch
        m = torch.rand(1, Hq, S, T, generator=g) > 0.5
        m[0, 1, :, :] = False
        return m
    if kind == "far":
        # the first 64+ keys masked, the rest far below zero: the running max
        # must start from the first finite tile, not from a placeholder
        m = torch.full((B, 1, S, T), -30000.0) + torch.randn(B, 1, S, T, generator=g)
        m[..., :80] = float("-inf")
        return m.to(dtype)
    raise ValueError(kind)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("kind", ["bool", "float", "heads", "far"])
def test_prefill_bias(dtype, D, kind):
    say(f"prefill bias {kind} {dtype} D={D}")
    B, Hq, Hkv, S, T = 2, 8, 2, 150, 150
    q = randn(B, Hq, S, D, seed=761, dtype=dtype)
    k = randn(B, Hkv, T, D, seed=762, dtype=dtype)
    v = randn(B, Hkv, T, D, seed=763, dtype=dtype)
    mask = _bias_masks(kind, B, Hq, S, T, dtype, 764)
    bias = ops.AttnBias(mask.to(DEV), B, Hq, S, T, dtype, DEV)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=False, bias=bias, return_lse=True)
    assert torch.isfinite(o.float()).all()
    if kind == "far" and dtype == torch.float32:
        # every finite logit is about -4.3e4 in log2 units, where fp32 spacing is
        # 2^-8: any fp32 evaluation (the reference's too) moves P by ~0.5%, so the
        # gate is against fp64 at that level (a wrong running max gives zeros)
        ref = attention(q.double(), k.double(), v.double(), mask=mask.double(), compute_dtype=torch.float64)
        d = (o.double().cpu() - ref).abs()
        assert float(d.max()) <= 1e-2 and float(d.mean()) <= 1e-3, (float(d.max()), float(d.mean()))
    else:
        ref = attention(q.float(), k.float(), v.float(), mask=mask if mask.dtype == torch.bool else mask.float())
        assert_close_for(dtype, o, ref, f"bias {kind}")
    sc = torch.matmul(q.float(), k.float().repeat_interleave(Hq // Hkv, 1).transpose(-1, -2)) / D ** 0.5
    sc = sc.masked_fill(~mask, float("-inf")) if mask.dtype == torch.bool else sc + mask.float()
    want = torch.logsumexp(sc, -1)
    got = lse.cpu()
    assert torch.equal(torch.isneginf(got), torch.isneginf(want))
    fin = torch.isfinite(want)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(got[fin], want[fin], rtol=1e-5, atol=tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prefill_bias_with_causal_and_key_lens(dtype):
    """A bias together with the causal frontier (T > S, bottom-right) and key padding."""
    say(f"prefill bias + causal + key_lens {dtype}")
    B, Hq, Hkv, S, T, D = 3, 8, 4, 100, 140, 128
    lens = torch.tensor([140, 60, 121], dtype=torch.int32)
    q = randn(B, Hq, S, D, seed=771, dtype=dtype)
    k = _poison(randn(B, Hkv, T, D, seed=772, dtype=dtype), lens)
    v = _poison(randn(B, Hkv, T, D, seed=773, dtype=dtype), lens)
    mask = (0.3 * randn(B, 1, S, T, seed=774)).to(dtype)
    bias = ops.AttnBias(mask.to(DEV), B, Hq, S, T, dtype, DEV)
    o = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, bias=bias, key_lens=lens.to(DEV))
    ref = attention(q.float(), k.float().nan_to_num(), v.float().nan_to_num(), causal=True, causal_offset=T - S,
                    key_lens=lens, mask=mask.float())
    assert_close_for(dtype, o, ref, "bias + causal + key_lens")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kind", ["bool", "float"])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_bias(dtype, kind, causal):
    """Gradients with a general mask against fp64 autograd of the oracle (rows whose keys
    are all masked get zero dQ and contribute nothing to dK, dV)."""
    say(f"backward bias {kind} {dtype} causal={causal}")
    B, Hq, Hkv, S, D = 2, 8, 2, 130, 128
    q = randn(B, Hq, S, D, seed=781, dtype=dtype)
    k = randn(B, Hkv, S, D, seed=782, dtype=dtype)
    v = randn(B, Hkv, S, D, seed=783, dtype=dtype)
    do = randn(B, Hq, S, D, seed=784, dtype=dtype)
    mask = _bias_masks(kind, B, Hq, S, S, dtype, 785)
    bias = ops.AttnBias(mask.to(DEV), B, Hq, S, S, dtype, DEV, transpose=True)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, bias=bias, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=causal,
                                        bias=bias)
    qd, kd, vd = (t.double().requires_grad_(True) for t in (q, k, v))
    md = mask if mask.dtype == torch.bool else mask.double()
    attention(qd, kd, vd, causal=causal, mask=md, compute_dtype=torch.float64).backward(do.double())
    mx_tol, mean_tol = (1e-5, 1e-6) if dtype == torch.float32 else (2e-2, 2e-3)
    for got, ref, name in ((dq, qd.grad, "dq"), (dk, kd.grad, "dk"), (dv, vd.grad, "dv")):
        got = got.double().cpu()
        assert torch.isfinite(got).all(), name
        sc = float(ref.abs().max())
        d = (got - ref).abs()
        assert float(d.max()) <= mx_tol * sc and float(d.mean()) <= mean_tol * sc, \
            f"{name}: max-abs {float(d.max()):.3e} mean-abs {float(d.mean()):.3e} (ref max {sc:.3e})"


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


def _grad_close(got, ref, name, dtype):
    """fp64-autograd comparison, relative to the reference's largest magnitude: the
    fp32 gate 1e-5 / 1e-6 (max / mean), the bf16 module's 5e-2 / 5e-3."""
    mx_tol, mean_tol = (1e-5, 1e-6) if dtype == torch.float32 else (5e-2, 5e-3)
    got = got.double().cpu()
    assert torch.isfinite(got).all(), name
    sc = float(ref.abs().max())
    d = (got - ref).abs()
    assert float(d.max()) <= mx_tol * sc and float(d.mean()) <= mean_tol * sc, \
        f"{name}: max-abs {float(d.max()):.3e} mean-abs {float(d.mean()):.3e} (ref max {sc:.3e})"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_training_with_general_mask(dtype):
    """A non-prefix mask under autograd: forward and backward on the bias kernels,
    every weight gradient against fp64 autograd of the oracle module."""
    say(f"module training with a general mask {dtype}")
    attn, w = _module(dtype, seed=791)
    attn.train()
    B, S = 2, 70
    g = torch.Generator().manual_seed(792)
    mask = torch.rand(B, 1, S, S, generator=g) > 0.3
    mask |= torch.eye(S, dtype=torch.bool)
    h = randn(B, S, 256, seed=793, dtype=dtype)
    gout = randn(B, S, 256, seed=794, dtype=dtype)
    before = dict(nq.stats)
    out = attn(h.to(DEV), attention_mask=mask.to(DEV))
    out.backward(gout.to(DEV))
    assert nq.stats["kernel_train_forward"] == before["kernel_train_forward"] + 1
    assert nq.stats["torch_forward"] == 0
    cos, sin = rope_tables(64, 512, 1e6)
    wd = {k: v.double().requires_grad_(True) for k, v in w.items()}
    ref, _ = attention_module_forward(h.double(), wd, num_heads=8, num_kv_heads=2, head_dim=64, eps=1e-6,
                                      cos_table=cos.double(), sin_table=sin.double(), attention_mask=mask)
    ref.backward(gout.double())
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
        _grad_close(getattr(attn, name).weight.grad, wd[name].grad, name, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_autograd_through_a_kv_cache(dtype):
    """Autograd with a KVCache (attention.py:102-115): a prompt cached without grad, then a
    continuation under autograd that appends its rows and attends every cached row.  The
    forward matches the oracle module with the reference's concatenating cache, and so do
    the gradients of every weight and of the continuation's hidden states."""
    say(f"module autograd through a KV cache {dtype}")
    attn, w = _module(dtype, seed=801)
    attn.train()
    B, S0, S1 = 2, 40, 17
    h0 = randn(B, S0, 256, seed=802, dtype=dtype)
    h1 = randn(B, S1, 256, seed=803, dtype=dtype)
    gout = randn(B, S1, 256, seed=804, dtype=dtype)
    cache = nq.KVCache()
    with torch.no_grad():
        attn(h0.to(DEV), kv_cache=cache)
    x1 = h1.to(DEV).requires_grad_(True)
    before = dict(nq.stats)
    out = attn(x1, kv_cache=cache)
    out.backward(gout.to(DEV))
    assert nq.stats["kernel_train_forward"] == before["kernel_train_forward"] + 1
    assert nq.stats["torch_forward"] == 0
    assert cache.seq_len == S0 + S1
    cos, sin = rope_tables(64, 512, 1e6)
    wd = {k: v.double().requires_grad_(True) for k, v in w.items()}
    oc = OracleKVCache()
    with torch.no_grad():
        attention_module_forward(h0.double(), {k: v.detach() for k, v in wd.items()}, num_heads=8,
                                 num_kv_heads=2, head_dim=64, eps=1e-6, cos_table=cos.double(),
                                 sin_table=sin.double(), kv_cache=oc)
    x1r = h1.double().requires_grad_(True)
    ref, _ = attention_module_forward(x1r, wd, num_heads=8, num_kv_heads=2, head_dim=64, eps=1e-6,
                                      cos_table=cos.double(), sin_table=sin.double(), kv_cache=oc)
    ref.backward(gout.double())
    _grad_close(out.detach(), ref.detach(), "output", dtype)
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
        _grad_close(getattr(attn, name).weight.grad, wd[name].grad, name, dtype)
    _grad_close(x1.grad, x1r.grad, "hidden", dtype)


def test_attention_dropout_raises_while_training():
    """attention.py:114 applies dropout_p while training; the kernels have none, so a
    config with attention_dropout > 0 is refused in training mode (no reference config
    sets it) and runs the kernels in eval mode."""
    say("attention dropout: refused while training")
    cfg = nq.AttentionConfig(hidden_size=256, num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                             max_position_embeddings=512, attention_dropout=0.1)
    attn = nq.Attention(cfg).to(DEV)
    h = randn(2, 16, 256, seed=811).to(DEV)
    attn.train()
    with pytest.raises(NotImplementedError, match="dropout"):
        attn(h)
    attn.eval()
    before = dict(nq.stats)
    with torch.no_grad():
        out = attn(h)
    assert torch.isfinite(out).all()
    assert nq.stats["kernel_forward"] == before["kernel_forward"] + 1 and nq.stats["torch_forward"] == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D,Hq,Hkv", [(32, 8, 1), (64, 16, 1), (128, 4, 4)])
@pytest.mark.parametrize("causal", [False, True])
def test_prefill_bias_shapes(dtype, D, Hq, Hkv, causal):
    """The bias kernels at head_dim 32/64/128 and GQA groups 1, 8 and 16, with S < T
    (a continuation over cached keys, bottom-right causal) and a per-head float bias
    with -inf entries; a query-independent bias broadcast over heads too."""
    say(f"prefill bias shapes {dtype} D={D} {Hq}/{Hkv} causal={causal}")
    B, S, T = 2, 70, 201
    q = randn(B, Hq, S, D, seed=911, dtype=dtype)
    k = randn(B, Hkv, T, D, seed=912, dtype=dtype)
    v = randn(B, Hkv, T, D, seed=913, dtype=dtype)
    mask = 0.5 * randn(B, Hq, S, T, seed=914)
    drop = torch.rand(B, Hq, S, T, generator=torch.Generator().manual_seed(915)) < 0.3
    drop[..., 0] = False  # key 0 always kept: no row is masked entirely
    mask = mask.masked_fill(drop, float("-inf")).to(dtype)
    for m in (mask, mask[:, :1, :1].expand(B, 1, 1, T).contiguous()):
        bias = ops.AttnBias(m.to(DEV), B, Hq, S, T, dtype, DEV)
        o = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, bias=bias)
        ref = attention(q.float(), k.float(), v.float(), causal=causal, causal_offset=T - S, mask=m.float())
        assert_close_for(dtype, o, ref, f"bias {tuple(m.shape)}")
