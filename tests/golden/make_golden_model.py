"""Write tests/golden/model_forward.npz from the nano-qwen reference's model and generator.

Run once, in a container that holds the reference source tree (default
/root/reference, or $NANO_QWEN_REF):

    python tests/golden/make_golden_model.py

It imports the reference's ``model.transformer.Qwen3Model`` (transformer.py:78-162,
built from model/attention.py, model/ffn.py, model/embedding.py, model/norm.py,
model/rope.py) and ``eval.generate.TextGenerator`` (eval/generate.py:20-138), all
pure PyTorch on the CPU, and records for a small dense GQA model (2 layers,
hidden 128, 4 query / 2 kv heads of 64, SwiGLU 256, vocab 160, fp32):
  * ``Qwen3Model.forward`` logits with no cache (causal) for a (2, 12) batch;
  * the same with explicit ``position_ids``;
  * greedy generation (temperature 0) through the reference's cache protocol
    (eval/generate.py:75-136: a fresh KVCache per layer, the prompt prefilled
    with the caches, then one token per step with no position_ids), for two
    prompts of different lengths, with the logits of every step.  The greedy
    tokens are cross-checked against ``TextGenerator.generate`` itself (with a
    pass-through tokenizer) before they are written.

Weights come from a seeded CPU torch.Generator (``make_model_weights``), keyed by
the reference's state-dict names; the tests regenerate them from the same seed.
The fixture is data only.  Bytecode writing is disabled so nothing is written
into the reference tree.
"""

from __future__ import annotations

import os
import sys

sys.dont_write_bytecode = True

import numpy as np
import torch

REF = os.environ.get("NANO_QWEN_REF", "/root/reference")
OUT = os.path.dirname(os.path.abspath(__file__))

MODEL = dict(vocab_size=160, hidden_size=128, num_hidden_layers=2, num_attention_heads=4,
             num_key_value_heads=2, head_dim=64, intermediate_size=256,
             max_position_embeddings=512, rope_theta=1e6, rms_norm_eps=1e-6)
SEED = 20261202
PROMPTS = [[3, 17, 42, 99, 7], [150, 2, 9, 33, 61, 80, 120, 5, 44, 12, 77]]
NEW_TOKENS = 10


def make_model_weights(cfg=MODEL, seed=SEED):
    """Seeded weights with the reference's state-dict names (fan-in scaled, so the
    greedy choices are decisive)."""
    g = torch.Generator().manual_seed(seed)
    V, hid, L = cfg["vocab_size"], cfg["hidden_size"], cfg["num_hidden_layers"]
    H, Hkv, D, F = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"], cfg["intermediate_size"]

    def lin(out_f, in_f, gain=1.0):
        return torch.randn(out_f, in_f, generator=g) * (gain / in_f ** 0.5)

    w = {"embed.embed_tokens.weight": torch.randn(V, hid, generator=g)}
    for i in range(L):
        p = f"layers.{i}."
        w[p + "input_layernorm.weight"] = 1.0 + 0.1 * torch.randn(hid, generator=g)
        w[p + "attention.q_proj.weight"] = lin(H * D, hid)
        w[p + "attention.k_proj.weight"] = lin(Hkv * D, hid)
        w[p + "attention.v_proj.weight"] = lin(Hkv * D, hid)
        w[p + "attention.o_proj.weight"] = lin(hid, H * D)
        w[p + "attention.q_norm.weight"] = 1.0 + 0.1 * torch.randn(D, generator=g)
        w[p + "attention.k_norm.weight"] = 1.0 + 0.1 * torch.randn(D, generator=g)
        w[p + "post_attention_layernorm.weight"] = 1.0 + 0.1 * torch.randn(hid, generator=g)
        w[p + "feed_forward.gate_proj.weight"] = lin(F, hid)
        w[p + "feed_forward.up_proj.weight"] = lin(F, hid)
        w[p + "feed_forward.down_proj.weight"] = lin(hid, F)
    w["norm.weight"] = 1.0 + 0.1 * torch.randn(hid, generator=g)
    w["lm_head.weight"] = lin(V, hid, gain=4.0)
    return w


def make_inputs(cfg=MODEL, seed=SEED + 1):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, cfg["vocab_size"], (2, 12), generator=g)
    pos = torch.stack([torch.arange(12) + 5, torch.arange(12) * 3 + 1])
    return ids, pos


def checksums(w):
    return np.array([float(w[k].double().sum()) for k in sorted(w)], dtype=np.float64)


class _PassThroughTokenizer:
    """Token ids travel as a space-separated string."""

    eos_id = None

    def encode(self, text, allowed_special=None):
        return [int(t) for t in text.split()]

    def decode(self, ids):
        return " ".join(str(int(t)) for t in ids)


def main():
    sys.path.insert(0, REF)
    from model.config import ModelConfig            # noqa: E402
    from model.transformer import Qwen3Model        # noqa: E402
    from model.attention import KVCache             # noqa: E402
    from eval.generate import TextGenerator         # noqa: E402

    cfg = ModelConfig(**MODEL, qk_norm=True, tie_word_embeddings=False)
    torch.manual_seed(0)
    model = Qwen3Model(cfg).eval()
    w = make_model_weights()
    missing, unexpected = model.load_state_dict(w, strict=False)
    assert not unexpected, unexpected
    assert all("rotary_emb" in m for m in missing), missing

    ids, pos = make_inputs()
    out = {"weights_checksums": checksums(w), "input_ids": ids.numpy(), "position_ids": pos.numpy()}
    with torch.no_grad():
        out["logits_nocache"] = model(input_ids=ids)["logits"].numpy()
        out["logits_position_ids"] = model(input_ids=ids, position_ids=pos)["logits"].numpy()

        gen = TextGenerator(model, _PassThroughTokenizer())
        for n, prompt in enumerate(PROMPTS):
            # the protocol of eval/generate.py:75-136 at temperature 0, step by step
            caches = [KVCache() for _ in range(len(model.layers))]
            logits = model(input_ids=torch.tensor([prompt]), kv_caches=caches)["logits"][:, -1, :]
            toks, steps = [], []
            for _ in range(NEW_TOKENS):
                steps.append(logits[0].numpy().copy())
                t = int(logits.argmax(dim=-1))
                toks.append(t)
                logits = model(input_ids=torch.tensor([[t]]), kv_caches=caches)["logits"][:, -1, :]
            text = gen.generate(" ".join(map(str, prompt)), max_new_tokens=NEW_TOKENS, temperature=0.0)
            assert [int(t) for t in text.split()] == toks, (text, toks)
            out[f"prompt{n}"] = np.array(prompt, dtype=np.int64)
            out[f"greedy_tokens{n}"] = np.array(toks, dtype=np.int64)
            out[f"greedy_logits{n}"] = np.stack(steps)
    np.savez_compressed(os.path.join(OUT, "model_forward.npz"), **out)
    print("wrote model_forward.npz:", {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
