"""The drop-in Attention / KVCache on the GPU against the reference's own outputs.

The golden fixtures were recorded from nano-qwen's Attention.forward (see
tests/golden/make_golden.py); here the same seeded weights are loaded into the
drop-in module and run through the HIP kernels.  The fp32 module keeps fp32
arithmetic end to end, so its outputs are held to the fp32 gate; the bf16
module to the bf16 one.
"""

import os

import numpy as np
import pytest
import torch

import nano_qwen_amd as nq
from tests.conftest import GOLDEN
from tests.golden.make_golden import SHAPE, make_weights
from tests.helpers import assert_bf16_close, assert_fp32_close, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def fx():
    return np.load(os.path.join(GOLDEN, "attention_forward.npz"), allow_pickle=False)


def _module(dtype=torch.float32):
    s = SHAPE
    cfg = nq.AttentionConfig(hidden_size=s["hidden"], num_attention_heads=s["heads"],
                             num_key_value_heads=s["kv_heads"], head_dim=s["head_dim"],
                             max_position_embeddings=s["max_pos"], rope_theta=s["theta"],
                             rms_norm_eps=s["eps"])
    w, hidden = make_weights()
    attn = nq.Attention(cfg).eval()
    with torch.no_grad():
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            getattr(attn, name).weight.copy_(w[name])
        attn.q_norm.weight.copy_(w["q_norm"])
        attn.k_norm.weight.copy_(w["k_norm"])
    return attn.to(device=DEV, dtype=dtype), hidden.to(device=DEV, dtype=dtype)


def _capture(attn):
    box = {}
    attn.o_proj.register_forward_pre_hook(lambda m, a: box.__setitem__("attn", a[0].detach()))
    return box


@torch.no_grad()
def test_forward_nocache_matches_reference(fx):
    say("module no cache")
    attn, h = _module()
    box = _capture(attn)
    before = nq.stats["kernel_forward"]
    out = attn(h)
    assert nq.stats["kernel_forward"] == before + 1
    assert_fp32_close(box["attn"], torch.from_numpy(fx["nocache_attn"]), "attn")
    assert_fp32_close(out, torch.from_numpy(fx["nocache_out"]), "out")


@torch.no_grad()
def test_forward_position_ids_matches_reference(fx):
    say("module position_ids")
    attn, h = _module()
    box = _capture(attn)
    out = attn(h, position_ids=torch.from_numpy(fx["posids_pos"]).to(DEV))
    assert_fp32_close(box["attn"], torch.from_numpy(fx["posids_attn"]), "attn")
    assert_fp32_close(out, torch.from_numpy(fx["posids_out"]), "out")


@torch.no_grad()
def test_cache_protocol_matches_reference(fx):
    """Prefill with a cache (bidirectional) + 3 decode steps at position 0, as generate.py."""
    say("module cache protocol")
    attn, h = _module()
    box = _capture(attn)
    cache = nq.KVCache()
    P = 12
    out = attn(h[:, :P], kv_cache=cache)
    assert_fp32_close(box["attn"], torch.from_numpy(fx["cache_prefill_attn"]), "prefill attn")
    assert_fp32_close(out, torch.from_numpy(fx["cache_prefill_out"]), "prefill out")
    for step in range(3):
        out = attn(h[:, P + step:P + step + 1], kv_cache=cache)
        assert_fp32_close(box["attn"], torch.from_numpy(fx[f"cache_step{step}_attn"]), f"step{step}")
        assert_fp32_close(out, torch.from_numpy(fx[f"cache_step{step}_out"]), f"step{step} out")
    assert cache.seq_len == P + 3
    assert_fp32_close(cache.key, torch.from_numpy(fx["cache_k"]), "cache K")
    assert_fp32_close(cache.value, torch.from_numpy(fx["cache_v"]), "cache V")


@torch.no_grad()
def test_bf16_module_matches_reference(fx):
    say("module bf16")
    attn, h = _module(torch.bfloat16)
    box = _capture(attn)
    out = attn(h)
    assert out.dtype == torch.bfloat16
    assert_bf16_close(box["attn"], torch.from_numpy(fx["bf16_attn"]), "bf16 attn")
    assert_bf16_close(out, torch.from_numpy(fx["bf16_out"]), "bf16 out", max_abs=3e-2)


@torch.no_grad()
def test_mask_runs_the_bias_kernels_and_matches(fx):
    """The reference's own outputs for a random (B, 1, S, S) bool mask: the kernels
    with the mask as a per-tile bias."""
    say("module mask (bias kernels)")
    attn, h = _module()
    box = _capture(attn)
    before = dict(nq.stats)
    out = attn(h, attention_mask=torch.from_numpy(fx["mask_mask"]).to(DEV))
    assert nq.stats["kernel_forward"] == before["kernel_forward"] + 1 and nq.stats["torch_forward"] == 0
    np.testing.assert_allclose(box["attn"].cpu().numpy(), fx["mask_attn"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(out.cpu().numpy(), fx["mask_out"], rtol=1e-4, atol=1e-4)


def test_autograd_runs_on_the_kernels():
    say("module autograd (kernel path)")
    attn, h = _module()
    before = dict(nq.stats)
    out = attn(h)
    out.float().pow(2).mean().backward()
    assert nq.stats["kernel_train_forward"] == before["kernel_train_forward"] + 1
    assert nq.stats["torch_forward"] == before["torch_forward"]
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
        g = getattr(attn, name).weight.grad
        assert g is not None and torch.isfinite(g).all(), name


@torch.no_grad()
def test_opt_in_cache_positions_equal_full_causal_prefill():
    """With rope_positions='cache' + causal cached prefill, token-by-token decode
    reproduces the one-shot causal forward (the generate loop without quirks)."""
    say("module opt-in cache positions")
    attn, h = _module(torch.bfloat16)
    full = attn(h)
    attn.rope_positions = "cache"
    attn.cache_prefill_causal = True
    cache = nq.KVCache(max_seq_len=64)
    outs = [attn(h[:, :5], kv_cache=cache)]
    for t in range(5, h.shape[1]):
        outs.append(attn(h[:, t:t + 1], kv_cache=cache))
    assert_bf16_close(torch.cat(outs, 1), full, "decode loop vs full", max_abs=3e-2)


@torch.no_grad()
def test_empty_inputs_give_empty_outputs():
    """Zero batch rows or zero tokens: empty outputs (as the reference's SDPA), the cache
    untouched, no kernel launched."""
    say("module empty inputs")
    attn, h = _module()
    before = dict(nq.stats)
    for shape in ((0, 5, h.shape[-1]), (h.shape[0], 0, h.shape[-1])):
        out = attn(h.new_zeros(shape))
        assert tuple(out.shape) == shape
    cache = nq.KVCache()
    out = attn(h[:, :0], kv_cache=cache)
    assert out.shape[1] == 0 and cache.seq_len == 0
    assert nq.stats == before
    q = torch.zeros(2, 4, 0, 64, device=DEV, dtype=torch.bfloat16)
    assert nq.flash_attention(q, q, q).shape == q.shape
