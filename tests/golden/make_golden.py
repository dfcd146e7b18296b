"""Write the golden fixtures under tests/golden/ from the nano-qwen reference.

Run once, in a container that holds the reference source tree (default
/root/reference, or $NANO_QWEN_REF):

    python tests/golden/make_golden.py

It imports the reference's ``model.attention``, ``model.rope``, ``model.norm``
and ``model.config`` (pure PyTorch, CPU) and records inputs/outputs of:
  * Attention.forward (model/attention.py:82-118) at a small GQA shape
    (B=2, S=16, hidden=64, Hq=8, Hkv=2, D=64, theta=1e6, eps=1e-6) in fp32:
    no cache (causal), explicit position_ids, a bool attention mask, and the
    eval/generate.py:75-136 cache protocol (prefill with a KVCache, then three
    S=1 steps with no position_ids); plus the same module cast to bf16;
  * RotaryEmbedding tables (model/rope.py:78-130): plain RoPE and YaRN
    (D=128, theta=1e6, factor 4, L0=32768, max_pos 131072) at selected rows,
    and the inverse-frequency rows;
  * RMSNorm (model/norm.py:11-22) cast order for bf16 input with fp32 and
    bf16 weights.

Weights are drawn from a seeded CPU torch.Generator; the tests regenerate them
from the same seed and check the stored checksums before comparing.  The
fixtures are data only (inputs and expected outputs); no reference source is
copied.  Bytecode writing is disabled so nothing is written into the
reference tree.
"""

from __future__ import annotations

import os
import sys

sys.dont_write_bytecode = True

import numpy as np
import torch

REF = os.environ.get("NANO_QWEN_REF", "/root/reference")
OUT = os.path.dirname(os.path.abspath(__file__))

SHAPE = dict(batch=2, seq=16, hidden=64, heads=8, kv_heads=2, head_dim=64,
             theta=1e6, eps=1e-6, max_pos=256)
SEED = 20261201


def make_weights(shape=SHAPE, seed=SEED):
    """Seeded weights shared by the generator script and the tests."""
    g = torch.Generator().manual_seed(seed)
    H, Hkv, D, hid = shape["heads"], shape["kv_heads"], shape["head_dim"], shape["hidden"]
    w = {
        "q_proj": torch.randn(H * D, hid, generator=g) * 0.05,
        "k_proj": torch.randn(Hkv * D, hid, generator=g) * 0.05,
        "v_proj": torch.randn(Hkv * D, hid, generator=g) * 0.05,
        "o_proj": torch.randn(hid, H * D, generator=g) * 0.05,
        "q_norm": 1.0 + 0.02 * torch.randn(D, generator=g),
        "k_norm": 1.0 + 0.02 * torch.randn(D, generator=g),
    }
    hidden = torch.randn(shape["batch"], shape["seq"], hid, generator=g)
    return w, hidden


def checksums(w):
    return np.array([float(w[k].double().sum()) for k in sorted(w)], dtype=np.float64)


def main():
    sys.path.insert(0, REF)
    from model.config import ModelConfig            # noqa: E402
    from model.attention import Attention, KVCache  # noqa: E402
    from model.rope import RotaryEmbedding, compute_yarn_freqs, _compute_freqs  # noqa: E402
    from model.norm import RMSNorm                  # noqa: E402

    s = SHAPE
    cfg = ModelConfig(hidden_size=s["hidden"], num_attention_heads=s["heads"],
                      num_key_value_heads=s["kv_heads"], head_dim=s["head_dim"],
                      max_position_embeddings=s["max_pos"], rope_theta=s["theta"],
                      rms_norm_eps=s["eps"], qk_norm=True)
    w, hidden = make_weights()
    attn = Attention(cfg, 0).eval()
    with torch.no_grad():
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            getattr(attn, name).weight.copy_(w[name])
        attn.q_norm.weight.copy_(w["q_norm"])
        attn.k_norm.weight.copy_(w["k_norm"])

    captured = {}

    def pre_o(_m, args):
        captured["attn"] = args[0].detach().clone()

    attn.o_proj.register_forward_pre_hook(pre_o)
    fx = {"weight_checksums": checksums(w), "hidden": hidden.numpy()}
    B, S = s["batch"], s["seq"]
    with torch.no_grad():
        out = attn(hidden)
        fx["nocache_out"], fx["nocache_attn"] = out.numpy(), captured["attn"].numpy()

        pos = (torch.arange(S)[None, :] + torch.tensor([[3], [40]])).long()
        out = attn(hidden, position_ids=pos)
        fx["posids_pos"] = pos.numpy()
        fx["posids_out"], fx["posids_attn"] = out.numpy(), captured["attn"].numpy()

        g = torch.Generator().manual_seed(SEED + 1)
        mask = torch.rand(B, 1, S, S, generator=g) > 0.3
        mask |= torch.eye(S, dtype=torch.bool)[None, None]
        out = attn(hidden, attention_mask=mask)
        fx["mask_mask"] = mask.numpy()
        fx["mask_out"], fx["mask_attn"] = out.numpy(), captured["attn"].numpy()

        P = 12
        cache = KVCache()
        out = attn(hidden[:, :P], kv_cache=cache)
        fx["cache_prefill_out"], fx["cache_prefill_attn"] = out.numpy(), captured["attn"].numpy()
        for step in range(3):
            out = attn(hidden[:, P + step:P + step + 1], kv_cache=cache)
            fx[f"cache_step{step}_out"] = out.numpy()
            fx[f"cache_step{step}_attn"] = captured["attn"].numpy()
        fx["cache_k"], fx["cache_v"] = cache.key.numpy(), cache.value.numpy()

        attn_bf = attn.to(torch.bfloat16)
        out = attn_bf(hidden.to(torch.bfloat16))
        fx["bf16_out"] = out.float().numpy()
        fx["bf16_attn"] = captured["attn"].float().numpy()
    np.savez_compressed(os.path.join(OUT, "attention_forward.npz"), **fx)

    rows = np.array([0, 1, 2, 1000, 32767, 32768, 65536, 131071], dtype=np.int64)
    yarn = {"type": "yarn", "factor": 4.0, "original_max_position_embeddings": 32768}
    re_yarn = RotaryEmbedding(128, 131072, 1e6, rope_scaling=yarn)
    re_plain128 = RotaryEmbedding(128, 131072, 1e6)
    re_plain64 = RotaryEmbedding(64, 256, 1e6)
    fr = {
        "rows": rows,
        "yarn128_cos": re_yarn.cos_cached[rows].numpy(),
        "yarn128_sin": re_yarn.sin_cached[rows].numpy(),
        "plain128_cos": re_plain128.cos_cached[rows].numpy(),
        "plain128_sin": re_plain128.sin_cached[rows].numpy(),
        "plain64_rows": np.array([0, 1, 17, 255], dtype=np.int64),
        "yarn128_inv_freq": compute_yarn_freqs(128, 2, 1e6, 4.0, 32768)[1].numpy(),
        "plain128_inv_freq": _compute_freqs(128, 2, 1e6)[1].numpy(),
        "yarn64_f2_inv_freq": compute_yarn_freqs(64, 2, 1e4, 2.0, 2048)[1].numpy(),
    }
    fr["plain64_cos"] = re_plain64.cos_cached[fr["plain64_rows"]].numpy()
    fr["plain64_sin"] = re_plain64.sin_cached[fr["plain64_rows"]].numpy()
    np.savez_compressed(os.path.join(OUT, "rope_tables.npz"), **fr)

    g = torch.Generator().manual_seed(SEED + 2)
    x = (torch.randn(4, 64, generator=g) * 3).to(torch.bfloat16)
    w32 = 1.0 + 0.1 * torch.randn(64, generator=g)
    nf = {"x_bf16": x.float().numpy(), "w_fp32": w32.numpy()}
    with torch.no_grad():
        n32 = RMSNorm(64, eps=1e-6)
        n32.weight.copy_(w32)
        y = n32(x)
        nf["y_bf16in_fp32w"] = y.numpy()
        nf["y_bf16in_fp32w_dtype"] = np.array(str(y.dtype))
        nbf = RMSNorm(64, eps=1e-6).to(torch.bfloat16)
        nbf.weight.copy_(w32.to(torch.bfloat16))
        y = nbf(x)
        nf["y_bf16in_bf16w"] = y.float().numpy()
        nf["y_bf16in_bf16w_dtype"] = np.array(str(y.dtype))
    np.savez_compressed(os.path.join(OUT, "rmsnorm.npz"), **nf)
    for f in ("attention_forward.npz", "rope_tables.npz", "rmsnorm.npz"):
        print(f, os.path.getsize(os.path.join(OUT, f)), "bytes")


if __name__ == "__main__":
    main()
