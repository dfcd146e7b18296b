"""Pin the oracle against golden vectors recorded from the reference itself.

The fixtures under tests/golden/ were written by tests/golden/make_golden.py
from nano-qwen's model/attention.py, model/rope.py and model/norm.py.
"""

import os

import numpy as np
import pytest
import torch

from oracle import (OracleKVCache, attention_module_forward, rms_norm, rope_inv_freq,
                    rope_tables, yarn_inv_freq)
from tests.conftest import GOLDEN
from tests.golden.make_golden import SHAPE, checksums, make_weights


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


@pytest.fixture(scope="module")
def fwd():
    return _load("attention_forward.npz")


@pytest.fixture(scope="module")
def weights(fwd):
    w, hidden = make_weights()
    np.testing.assert_allclose(checksums(w), fwd["weight_checksums"], rtol=0, atol=1e-9)
    np.testing.assert_array_equal(hidden.numpy(), fwd["hidden"])
    return w


def _module(w, hidden, dtype=torch.float32, **kw):
    s = SHAPE
    cos, sin = rope_tables(s["head_dim"], s["max_pos"], s["theta"])
    ww = {k: v.to(dtype) for k, v in w.items()}
    return attention_module_forward(hidden.to(dtype), ww, num_heads=s["heads"],
                                    num_kv_heads=s["kv_heads"], head_dim=s["head_dim"],
                                    eps=s["eps"], cos_table=cos, sin_table=sin, **kw)


def test_forward_nocache_causal(fwd, weights):
    out, attn = _module(weights, torch.from_numpy(fwd["hidden"]))
    np.testing.assert_allclose(attn.numpy(), fwd["nocache_attn"], rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(out.numpy(), fwd["nocache_out"], rtol=1e-5, atol=2e-6)


def test_forward_position_ids(fwd, weights):
    pos = torch.from_numpy(fwd["posids_pos"])
    out, attn = _module(weights, torch.from_numpy(fwd["hidden"]), position_ids=pos)
    np.testing.assert_allclose(attn.numpy(), fwd["posids_attn"], rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(out.numpy(), fwd["posids_out"], rtol=1e-5, atol=2e-6)


def test_forward_bool_mask(fwd, weights):
    mask = torch.from_numpy(fwd["mask_mask"])
    out, attn = _module(weights, torch.from_numpy(fwd["hidden"]), attention_mask=mask)
    np.testing.assert_allclose(attn.numpy(), fwd["mask_attn"], rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(out.numpy(), fwd["mask_out"], rtol=1e-5, atol=2e-6)


def test_forward_cache_protocol(fwd, weights):
    """Prefill with a cache is bidirectional; S=1 steps without position_ids
    rotate at position 0 (eval/generate.py:75-136 driving attention.py:99-113)."""
    hidden = torch.from_numpy(fwd["hidden"])
    cache = OracleKVCache()
    P = 12
    out, attn = _module(weights, hidden[:, :P], kv_cache=cache)
    np.testing.assert_allclose(attn.numpy(), fwd["cache_prefill_attn"], rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(out.numpy(), fwd["cache_prefill_out"], rtol=1e-5, atol=2e-6)
    for step in range(3):
        out, attn = _module(weights, hidden[:, P + step:P + step + 1], kv_cache=cache)
        np.testing.assert_allclose(attn.numpy(), fwd[f"cache_step{step}_attn"], rtol=1e-5, atol=2e-6)
        np.testing.assert_allclose(out.numpy(), fwd[f"cache_step{step}_out"], rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(cache.key.numpy(), fwd["cache_k"], rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(cache.value.numpy(), fwd["cache_v"], rtol=1e-5, atol=2e-6)


def test_forward_bf16_module(fwd, weights):
    out, attn = _module(weights, torch.from_numpy(fwd["hidden"]), dtype=torch.bfloat16)
    a, ref = attn.float().numpy(), fwd["bf16_attn"]
    # bf16 rounding of the softmax/PV path differs between SDPA and the oracle's
    # fp32 evaluation by at most a couple of bf16 ulps.
    assert np.abs(a - ref).max() <= 2e-2
    assert np.abs(a - ref).mean() <= 2e-3
    o = out.float().numpy()
    assert np.abs(o - fwd["bf16_out"]).max() <= 2e-2


def test_rope_tables_golden():
    fr = _load("rope_tables.npz")
    rows = torch.from_numpy(fr["rows"])
    cos, sin = rope_tables(128, 131072, 1e6, {"type": "yarn", "factor": 4.0,
                                               "original_max_position_embeddings": 32768})
    np.testing.assert_array_equal(cos[rows].numpy(), fr["yarn128_cos"])
    np.testing.assert_array_equal(sin[rows].numpy(), fr["yarn128_sin"])
    cos, sin = rope_tables(128, 131072, 1e6)
    np.testing.assert_array_equal(cos[rows].numpy(), fr["plain128_cos"])
    np.testing.assert_array_equal(sin[rows].numpy(), fr["plain128_sin"])
    r64 = torch.from_numpy(fr["plain64_rows"])
    cos, sin = rope_tables(64, 256, 1e6)
    np.testing.assert_array_equal(cos[r64].numpy(), fr["plain64_cos"])
    np.testing.assert_array_equal(sin[r64].numpy(), fr["plain64_sin"])
    np.testing.assert_array_equal(yarn_inv_freq(128, 1e6, 4.0, 32768).numpy(), fr["yarn128_inv_freq"])
    np.testing.assert_array_equal(rope_inv_freq(128, 1e6).numpy(), fr["plain128_inv_freq"])
    np.testing.assert_array_equal(yarn_inv_freq(64, 1e4, 2.0, 2048).numpy(), fr["yarn64_f2_inv_freq"])


def test_rmsnorm_cast_order_golden():
    nf = _load("rmsnorm.npz")
    x = torch.from_numpy(nf["x_bf16"]).to(torch.bfloat16)
    w = torch.from_numpy(nf["w_fp32"])
    y = rms_norm(x, w, 1e-6)
    assert str(y.dtype) == str(nf["y_bf16in_fp32w_dtype"])
    np.testing.assert_array_equal(y.numpy(), nf["y_bf16in_fp32w"])
    y = rms_norm(x, w.to(torch.bfloat16), 1e-6)
    assert str(y.dtype) == str(nf["y_bf16in_bf16w_dtype"])
    np.testing.assert_array_equal(y.float().numpy(), nf["y_bf16in_bf16w"])
