"""The kernels launch on the caller's current stream (torch.cuda.current_stream()).

Every op is run once on the default stream, then again under
``torch.cuda.stream(s)`` for a second (default-priority) stream, and a planned
call is relaunched on a third stream; after synchronizing only those streams the
results must equal the default-stream ones bit for bit (same kernels, same inputs).
"""

import pytest
import torch

import nano_qwen_amd as nq
from nano_qwen_amd import ops
from tests.helpers import randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs():
    B, S, Hq, Hkv, D = 2, 300, 8, 2, 128
    q = randn(B, Hq, S, D, seed=901, dtype=torch.bfloat16).to(DEV)
    k = randn(B, Hkv, S, D, seed=902, dtype=torch.bfloat16).to(DEV)
    v = randn(B, Hkv, S, D, seed=903, dtype=torch.bfloat16).to(DEV)
    do = randn(B, Hq, S, D, seed=904, dtype=torch.bfloat16).to(DEV)
    lens = torch.tensor([300, 123], dtype=torch.int32, device=DEV)
    cos, sin = (t.to(DEV) for t in nq.build_tables(D, 512, 1e6))
    return q, k, v, do, lens, cos, sin


def _run(q, k, v, do, lens, cos, sin):
    o, lse = ops.attention_prefill(q, k, v, causal=True, return_lse=True)
    dq, dk, dv = ops.attention_backward(q, k, v, o, do, lse, causal=True)
    dec = ops.attention_decode(q[:, :, -1], k, v, lens, max_len=300, cos=cos, sin=sin)
    return o, lse, dq, dk, dv, dec


def test_ops_follow_the_current_stream():
    say("ops on a side stream")
    args = _inputs()
    ref = _run(*args)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        got = _run(*args)
    s.synchronize()
    for name, a, b in zip(("o", "lse", "dq", "dk", "dv", "decode"), got, ref):
        assert torch.equal(a, b), name


def test_planned_call_relaunches_on_another_stream():
    say("planned prefill on another stream")
    q, k, v, _, _, cos, sin = _inputs()
    ref = ops.attention_prefill(q, k, v, causal=True, cos=cos, sin=sin)
    torch.cuda.synchronize()
    out = torch.full_like(ref, float("nan"))
    call = ops.attention_prefill(q, k, v, causal=True, cos=cos, sin=sin, out=out, plan=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    call.launch(s)
    s.synchronize()
    assert torch.equal(out, ref)
