"""Host-side checks of the ring-attention pieces (no GPU)."""

import ctypes

import pytest
import torch

import nano_qwen_amd as nq
from nano_qwen_amd import _lib


def test_split_sequence_chunks():
    h = torch.arange(2 * 12 * 3).view(2, 12, 3)
    parts = [nq.split_sequence(h, r, 4) for r in range(4)]
    assert all(p.shape == (2, 3, 3) for p in parts)
    assert torch.equal(torch.cat(parts, dim=1), h)
    with pytest.raises(ValueError):
        nq.split_sequence(h, 0, 5)


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8])
def test_ring_schedule_visits_every_chunk_once_starting_with_its_own(n):
    for r in range(n):
        order = nq.ring_schedule(r, n)
        assert order[0] == r and sorted(order) == list(range(n))
        # what rank r holds at step s+1 is what rank r-1 held at step s (one hop per step)
        for s in range(n - 1):
            assert order[s + 1] == nq.ring_schedule((r - 1) % n, n)[s]


def test_ring_module_refuses_cpu_and_merge_arguments_are_checked():
    q = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP device"):
        nq.RingAttention()(q, q, q)
    lib = _lib.load()
    st = _lib.strides3((0, 0, 0))
    assert lib.nq_attn_merge(None, st, None, None, st, None, 1, 1, 1, 96, 0, None) == _lib.NQ_ERR_UNSUPPORTED
    assert lib.nq_attn_merge(None, st, None, None, st, None, 1, 1, 1, 64, 0, None) == _lib.NQ_ERR_INVALID
    fake = ctypes.c_void_p(4096)  # never dereferenced: the stride check fails first
    bad = _lib.strides3((4, 4, 4))  # 8 bytes in bf16
    assert lib.nq_attn_merge(fake, bad, fake, fake, bad, fake, 1, 1, 1, 64, 0, None) == _lib.NQ_ERR_INVALID
    assert b"16 bytes" in lib.nq_last_error()
