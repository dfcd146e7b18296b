"""End-to-end parity of the model and generators on the attention kernels.

The model is nano-qwen's dense Qwen3 (2 layers, hidden 128, 4 query / 2 kv
heads of 64) with the seeded weights of tests/golden/make_golden_model.py, run
in bf16 on the GPU.  References:
  * the reference's own fp32 logits and greedy tokens (model_forward.npz);
  * the oracle model (fp32, CPU), pinned to those goldens, for the ragged
    batch with causal prefill and true positions, by teacher forcing: the
    oracle is evaluated on the token sequence the GPU produced.

Tolerances (on logits of magnitude up to ~16): max-abs 0.3, mean-abs 0.05.
The oracle itself run in bf16 on the CPU lands at max 0.13 / mean 0.028 from
the fp32 goldens.  A greedy token must equal the reference's wherever the
reference's top-2 margin exceeds twice the max-abs tolerance.
"""

import os

import numpy as np
import pytest
import torch

from nano_qwen_amd import (KVCache, ModelConfig, Qwen3Model, TextGenerator, generate_greedy_batch,
                           stats)
from oracle import greedy_reference_protocol, model_forward
from tests.conftest import GOLDEN
from tests.golden.make_golden_model import MODEL, NEW_TOKENS, make_model_weights
from tests.helpers import say

pytestmark = pytest.mark.gpu

MAX_ABS = 0.3
MEAN_ABS = 0.05


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLDEN, "model_forward.npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def weights():
    return make_model_weights()


@pytest.fixture(scope="module")
def model(weights):
    torch.manual_seed(0)
    m = Qwen3Model(ModelConfig(**MODEL)).eval()
    m.load_state_dict(weights, strict=True)
    return m.to(device="cuda", dtype=torch.bfloat16)


@pytest.fixture
def reference_semantics(model):
    model.set_cache_semantics(False)
    yield model


def _close(got, ref, what):
    got = torch.as_tensor(got).float().cpu()
    ref = torch.as_tensor(ref).float().cpu()
    d = (got - ref).abs()
    assert float(d.max()) <= MAX_ABS and float(d.mean()) <= MEAN_ABS, \
        f"{what}: max-abs {float(d.max()):.3f} mean-abs {float(d.mean()):.4f}"


def _margins(logits):
    top2 = torch.as_tensor(logits).float().topk(2, dim=-1).values
    return top2[..., 0] - top2[..., 1]


def _tokens_agree(toks, ref_logits, what):
    """Each chosen token is the reference's argmax where its margin is decisive."""
    ref_logits = torch.as_tensor(ref_logits).float()
    ref_arg = ref_logits.argmax(-1).tolist()
    marg = _margins(ref_logits).tolist()
    for i, (t, r, m) in enumerate(zip(toks, ref_arg, marg)):
        if m > 2 * MAX_ABS:
            assert t == r, f"{what}: step {i} chose {t}, reference {r} (margin {m:.3f})"


def test_nocache_logits(gold, model):
    say("e2e no-cache logits (2,12)")
    ids = torch.from_numpy(gold["input_ids"]).cuda()
    before = dict(stats)
    with torch.no_grad():
        out = model(input_ids=ids)
    assert stats["kernel_forward"] - before["kernel_forward"] == MODEL["num_hidden_layers"]
    assert stats["torch_forward"] == before["torch_forward"]
    _close(out["logits"], gold["logits_nocache"], "no-cache logits")
    assert out["loss"] is None and out["aux_loss"] is None


def test_position_ids_logits(gold, model):
    say("e2e position_ids logits (2,12)")
    ids = torch.from_numpy(gold["input_ids"]).cuda()
    pos = torch.from_numpy(gold["position_ids"]).cuda()
    with torch.no_grad():
        out = model(input_ids=ids, position_ids=pos)
    _close(out["logits"], gold["logits_position_ids"], "position_ids logits")


def _replay(model, prompt, n):
    """eval/generate.py:75-136 at temperature 0, keeping every step's logits."""
    caches = [KVCache() for _ in model.layers]
    with torch.no_grad():
        logits = model(input_ids=torch.tensor([prompt], device="cuda"), kv_caches=caches)["logits"][0, -1]
        toks, steps = [], []
        for _ in range(n):
            steps.append(logits.float().cpu())
            t = int(logits.argmax())
            toks.append(t)
            logits = model(input_ids=torch.tensor([[t]], device="cuda"), kv_caches=caches)["logits"][0, -1]
    return toks, torch.stack(steps)


@pytest.mark.parametrize("n", [0, 1])
def test_reference_protocol_greedy(gold, weights, reference_semantics, n):
    model = reference_semantics
    prompt = gold[f"prompt{n}"].tolist()
    say(f"e2e reference-protocol greedy prompt{n} (len {len(prompt)})")
    toks, logits = _replay(model, prompt, NEW_TOKENS)
    gtoks, glogits = gold[f"greedy_tokens{n}"].tolist(), gold[f"greedy_logits{n}"]
    # against the reference itself, up to the first step both runs could split at
    agree = 0
    while agree < NEW_TOKENS and toks[agree] == gtoks[agree]:
        agree += 1
    if agree < NEW_TOKENS:
        assert float(_margins(glogits[agree])) <= 2 * MAX_ABS, \
            f"diverged from the reference at a decisive step {agree}: {toks} vs {gtoks}"
    _close(logits[:agree + (agree < NEW_TOKENS)], glogits[:agree + (agree < NEW_TOKENS)],
           "greedy logits vs reference")
    # the whole GPU sequence, teacher-forced through the pinned oracle
    _, ologits = greedy_reference_protocol(weights, MODEL, prompt, NEW_TOKENS, forced=toks)
    _close(logits, ologits, "greedy logits vs oracle (forced)")
    _tokens_agree(toks, ologits, "greedy tokens vs oracle")


class _Ids:
    eos_id = None

    def encode(self, text, allowed_special=None):
        return [int(t) for t in text.split()]

    def decode(self, ids):
        return " ".join(str(int(t)) for t in ids)


def test_text_generator_matches_replay(gold, reference_semantics):
    model = reference_semantics
    prompt = gold["prompt1"].tolist()
    say("e2e TextGenerator greedy prompt1")
    toks, _ = _replay(model, prompt, NEW_TOKENS)
    gen = TextGenerator(model, _Ids())
    text = gen.generate(" ".join(map(str, prompt)), max_new_tokens=NEW_TOKENS, temperature=0.0)
    assert [int(t) for t in text.split()] == toks
    # a stop token ends generation before it is emitted
    text = gen.generate(" ".join(map(str, prompt)), max_new_tokens=NEW_TOKENS, temperature=0.0,
                        stop_tokens=[toks[3]])
    assert [int(t) for t in text.split()] == toks[:toks.index(toks[3])]


def test_text_generator_sampling_runs(gold, reference_semantics):
    say("e2e TextGenerator sampling")
    gen = TextGenerator(reference_semantics, _Ids())
    torch.manual_seed(1)
    text = gen.generate("1 2 3", max_new_tokens=6, temperature=0.8, top_k=20, top_p=0.9,
                        repetition_penalty=1.1)
    toks = [int(t) for t in text.split()]
    assert len(toks) == 6 and all(0 <= t < MODEL["vocab_size"] for t in toks)


def _check_ragged(model, weights, prompts, n, what):
    toks, logits = generate_greedy_batch(model, prompts, n, return_logits=True)
    for b, p in enumerate(prompts):
        assert len(toks[b]) == n
        full = model_forward(weights, MODEL, torch.tensor([list(p) + toks[b]]))[0]
        ref = full[len(p) - 1:len(p) - 1 + n]
        _close(logits[b], ref, f"{what} row {b} (prompt len {len(p)})")
        _tokens_agree(toks[b], ref, f"{what} row {b}")
    return toks


def test_ragged_batch_true_positions(gold, weights, model):
    prompts = [gold["prompt0"].tolist(), gold["prompt1"].tolist(), [77], [5, 9, 13, 21, 34, 55, 89]]
    say(f"e2e ragged greedy batch lens {[len(p) for p in prompts]}")
    _check_ragged(model, weights, prompts, 12, "ragged")
    # the model's own setting is left as it was
    assert all(l.attention.rope_positions == "reference" for l in model.layers)


def test_ragged_batch_long_prompts(weights, model):
    g = torch.Generator().manual_seed(7)
    lens = [200, 77, 130, 3]
    prompts = [torch.randint(0, MODEL["vocab_size"], (L,), generator=g).tolist() for L in lens]
    say(f"e2e ragged greedy batch lens {lens}")
    _check_ragged(model, weights, prompts, 16, "ragged long")


def test_ragged_batch_stop_tokens(gold, model):
    prompts = [gold["prompt0"].tolist(), gold["prompt1"].tolist(), [77]]
    say("e2e ragged greedy batch with stop tokens")
    toks, _ = generate_greedy_batch(model, prompts, 10)
    stop = toks[0][2]
    cut, _ = generate_greedy_batch(model, prompts, 10, stop_tokens=[stop])
    for b in range(len(prompts)):
        want = toks[b][:toks[b].index(stop)] if stop in toks[b] else toks[b]
        assert cut[b] == want, (b, cut[b], want)


def test_fixed_semantics_cache_matches_nocache(gold, model):
    """With causal cached prefill and true positions, prefill + decode through
    the cache gives the no-cache logits of the whole sequence."""
    prompt = gold["prompt1"].tolist()
    say("e2e fixed-semantics cache vs no-cache")
    model.set_cache_semantics(True)
    try:
        caches = [KVCache() for _ in model.layers]
        with torch.no_grad():
            pre = model(input_ids=torch.tensor([prompt], device="cuda"), kv_caches=caches)["logits"][0]
            dec = model(input_ids=torch.tensor([[42]], device="cuda"), kv_caches=caches)["logits"][0, -1]
            full = model(input_ids=torch.tensor([prompt + [42]], device="cuda"))["logits"][0]
    finally:
        model.set_cache_semantics(False)
    torch.testing.assert_close(pre.float(), full[:-1].float(), atol=0.05, rtol=0)
    # The last row comes from the decode kernel (fp32 P against bf16 V) on one
    # side and the prefill kernel (bf16 P on the MFMA) on the other; through the
    # bf16 model's layers their logits differ by a few bf16 steps (0.0625 at
    # |logit| >= 8).  A cache or position mistake moves logits by O(1).
    torch.testing.assert_close(dec.float(), full[-1].float(), atol=0.1, rtol=0)


def test_training_step_gradients_against_oracle(weights):
    """One cross-entropy training step of the fp32 model on the kernels (attention
    forward and backward: prefill with LSE, the FlashAttention-2 backward, the
    QK-Norm + RoPE backward), every parameter gradient against fp64 autograd
    through the oracle model.  The fp32 model's attention runs its products on
    fp32 MFMA, so the gate is fp32-level: loss within 1e-5 relative, and per
    tensor, relative to its largest reference magnitude, max-abs <= 1e-4 and
    mean-abs <= 1e-5 (a few layers of fp32 rounding against fp64)."""
    say("training step gradients (kernels vs oracle fp64 autograd)")
    torch.manual_seed(0)
    m = Qwen3Model(ModelConfig(**MODEL)).train()
    m.load_state_dict(weights, strict=True)
    m = m.to("cuda")
    g = torch.Generator().manual_seed(601)
    ids = torch.randint(0, MODEL["vocab_size"], (2, 96), generator=g)
    before = stats["kernel_train_forward"]
    out = m(ids.cuda(), labels=ids.cuda())
    out["loss"].backward()
    assert stats["kernel_train_forward"] == before + MODEL["num_hidden_layers"]

    ref_w = {n: t.detach().double().clone().requires_grad_(True) for n, t in weights.items()}
    logits = model_forward(ref_w, MODEL, ids)
    loss = torch.nn.functional.cross_entropy(logits[:, :-1].reshape(-1, logits.shape[-1]),
                                             ids[:, 1:].reshape(-1))
    loss.backward()
    got_loss, ref_loss = out["loss"].detach().item(), loss.detach().item()
    assert abs(got_loss - ref_loss) <= 1e-5 * ref_loss, (got_loss, ref_loss)
    grads = dict(m.named_parameters())
    worst = 0.0
    for name, ref in ref_w.items():
        got = grads[name].grad
        assert got is not None, name
        got = got.double().cpu()
        r = ref.grad
        scale = float(r.abs().max())
        d = (got - r).abs()
        worst = max(worst, float(d.max()) / scale)
        assert float(d.max()) <= 1e-4 * scale and float(d.mean()) <= 1e-5 * scale, \
            f"{name}: max-abs {float(d.max()):.3e} mean-abs {float(d.mean()):.3e} (ref max {scale:.3e})"
    say(f"training step: loss rel err {abs(got_loss - ref_loss) / ref_loss:.2e}, worst grad rel err {worst:.2e}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gradient_checkpointing_gradients_bit_equal(weights, dtype):
    """transformer.py:92,121-127: with gradient_checkpointing each block's forward
    (the attention kernels' autograd Function included) runs again inside the
    backward; the kernels are deterministic, so every parameter gradient equals
    the one without recompute bit for bit."""
    say(f"gradient checkpointing {dtype}")
    g = torch.Generator().manual_seed(611)
    ids = torch.randint(0, MODEL["vocab_size"], (2, 80), generator=g).cuda()
    grads = {}
    for ckpt in (False, True):
        torch.manual_seed(0)
        m = Qwen3Model(ModelConfig(**MODEL, gradient_checkpointing=ckpt)).train()
        m.load_state_dict(weights, strict=True)
        m = m.to("cuda", dtype)
        assert m.gradient_checkpointing is ckpt
        before = stats["kernel_train_forward"]
        m(ids, labels=ids)["loss"].backward()
        # the attention forward runs once per layer, and once more per layer under recompute
        assert stats["kernel_train_forward"] == before + MODEL["num_hidden_layers"] * (2 if ckpt else 1)
        grads[ckpt] = {n: p.grad.clone() for n, p in m.named_parameters()}
    for n, gr in grads[False].items():
        assert torch.equal(gr, grads[True][n]), n
