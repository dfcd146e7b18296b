"""Host-side checks of the model mirror and the ragged cache (no GPU needed)."""

import pytest
import torch

from nano_qwen_amd import KVCache, ModelConfig, Qwen3Model, generate_greedy_batch
from tests.golden.make_golden_model import MODEL, make_model_weights


def _model():
    torch.manual_seed(0)
    return Qwen3Model(ModelConfig(**MODEL)).eval()


def test_reference_state_dict_loads_strict():
    """The reference's state-dict names load with no missing or extra keys
    (the rotary tables are non-persistent buffers, as in the reference)."""
    m = _model()
    w = make_model_weights()
    m.load_state_dict(w, strict=True)
    assert set(m.state_dict()) == set(w)
    assert m.count_parameters()["total"] == sum(v.numel() for v in w.values())


def test_forward_on_cpu_fails_loudly():
    m = _model()
    with pytest.raises(RuntimeError, match="HIP devices only"):
        m(torch.tensor([[1, 2, 3]]))


def test_cache_semantics_switch():
    m = _model()
    m.set_cache_semantics(True)
    assert all(l.attention.rope_positions == "cache" and l.attention.cache_prefill_causal
               for l in m.layers)
    m.set_cache_semantics(False)
    assert all(l.attention.rope_positions == "reference" and not l.attention.cache_prefill_causal
               for l in m.layers)


def test_moe_config_refused():
    class Cfg(ModelConfig):
        is_moe = True
    with pytest.raises(NotImplementedError):
        Qwen3Model(Cfg(**MODEL))


def test_generate_batch_rejects_empty_prompt():
    with pytest.raises(ValueError):
        generate_greedy_batch(_model(), [[1, 2], []], 4)


def _filled_cache(B=3, H=2, T=6, D=8):
    c = KVCache(max_seq_len=16)
    c.reserve(B, H, T, D, torch.float32, "cpu")
    c.advance(T)
    return c


def test_ragged_cache_lengths():
    c = _filled_cache()
    c.set_lengths(torch.tensor([6, 1, 4]))
    assert c.lens.dtype == torch.int32 and c.lens.tolist() == [6, 1, 4]
    with pytest.raises(NotImplementedError):
        c.update(torch.zeros(3, 2, 1, 8), torch.zeros(3, 2, 1, 8))
    c.reset()
    assert c.lens is None and c.seq_len == 0


@pytest.mark.parametrize("lens", [[7, 1, 1], [0, 2, 3], [1, 2]])
def test_ragged_cache_rejects_bad_lengths(lens):
    c = _filled_cache()
    with pytest.raises(ValueError):
        c.set_lengths(torch.tensor(lens))


def test_set_lengths_needs_storage():
    with pytest.raises(ValueError):
        KVCache().set_lengths(torch.tensor([1]))
