"""Pin the oracle model against the reference's own Qwen3Model / TextGenerator.

tests/golden/model_forward.npz was written by tests/golden/make_golden_model.py
from nano-qwen's model/transformer.py and eval/generate.py (fp32, CPU).
"""

import os

import numpy as np
import pytest
import torch

from oracle import (OracleKVCache, greedy_full_recompute, greedy_reference_protocol,
                    model_forward)
from tests.conftest import GOLDEN
from tests.golden.make_golden_model import MODEL, NEW_TOKENS, checksums, make_inputs, make_model_weights


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLDEN, "model_forward.npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def weights(gold):
    w = make_model_weights()
    np.testing.assert_allclose(checksums(w), gold["weights_checksums"], rtol=0, atol=1e-9)
    ids, pos = make_inputs()
    np.testing.assert_array_equal(ids.numpy(), gold["input_ids"])
    np.testing.assert_array_equal(pos.numpy(), gold["position_ids"])
    return w


def test_forward_nocache(gold, weights):
    got = model_forward(weights, MODEL, torch.from_numpy(gold["input_ids"]))
    np.testing.assert_allclose(got.numpy(), gold["logits_nocache"], rtol=1e-4, atol=1e-4)


def test_forward_position_ids(gold, weights):
    got = model_forward(weights, MODEL, torch.from_numpy(gold["input_ids"]),
                        position_ids=torch.from_numpy(gold["position_ids"]))
    np.testing.assert_allclose(got.numpy(), gold["logits_position_ids"], rtol=1e-4, atol=1e-4)
    # positions matter: the explicit ones give different logits from 0..S-1
    assert np.abs(gold["logits_position_ids"] - gold["logits_nocache"]).max() > 1e-2


@pytest.mark.parametrize("n", [0, 1])
def test_greedy_reference_protocol(gold, weights, n):
    toks, logits = greedy_reference_protocol(weights, MODEL, gold[f"prompt{n}"].tolist(), NEW_TOKENS)
    assert toks == gold[f"greedy_tokens{n}"].tolist()
    np.testing.assert_allclose(logits.numpy(), gold[f"greedy_logits{n}"], rtol=1e-4, atol=2e-4)


@pytest.mark.parametrize("n", [0, 1])
def test_full_recompute_is_causal_forward(gold, weights, n):
    prompt = gold[f"prompt{n}"].tolist()
    toks, logits = greedy_full_recompute(weights, MODEL, prompt, 6)
    full = model_forward(weights, MODEL, torch.tensor([prompt + toks]))[0]
    P = len(prompt)
    # step t was chosen from row P-1+t of one causal forward over the final sequence
    torch.testing.assert_close(logits, full[P - 1:P - 1 + 6], rtol=1e-5, atol=1e-5)
    assert toks == full[P - 1:P - 1 + 6].argmax(-1).tolist()


def test_reference_protocol_differs_from_causal(gold, weights):
    """The reference's cache protocol (bidirectional cached prefill, decode
    rotated at position 0) is not the causal model: the goldens show it."""
    prompt = gold["prompt1"].tolist()
    _, causal = greedy_full_recompute(weights, MODEL, prompt, 1)
    assert (causal[0] - torch.from_numpy(gold["greedy_logits1"][0])).abs().max() > 1e-2


def test_oracle_cache_prefill_then_decode_shapes(weights):
    caches = [OracleKVCache() for _ in range(MODEL["num_hidden_layers"])]
    model_forward(weights, MODEL, torch.tensor([[1, 2, 3]]), kv_caches=caches)
    model_forward(weights, MODEL, torch.tensor([[4]]), kv_caches=caches)
    assert all(c.seq_len == 4 for c in caches)
