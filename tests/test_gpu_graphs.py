"""A decode step (K-hat/V append, split-K decode, merge) captured in a HIP graph.

Serving loops capture the per-token launches once and replay them.  The library
allocates nothing and records no memset, so planned calls capture as plain
kernel nodes.  The graph is replayed three times with eager torch work (new
inputs) and device synchronizations between the replays; after every replay the
output and the cache must equal an eager run of the same step on copies of the
same buffers, bit for bit.
"""

import pytest
import torch

import nano_qwen_amd as nq
from tests.helpers import randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_decode_step_replays_from_a_hip_graph():
    say("decode step in a HIP graph")
    B, Hq, Hkv, D, T = 4, 16, 2, 128, 1024
    lens = torch.tensor([1000, 17, 512, 1024], dtype=torch.int32, device=DEV)
    row = lens - 1                                   # slot of the new token
    kc = randn(B, Hkv, T, D, seed=951, dtype=torch.bfloat16).to(DEV)
    vc = randn(B, Hkv, T, D, seed=952, dtype=torch.bfloat16).to(DEV)
    q = torch.empty(B, Hq, 1, D, dtype=torch.bfloat16, device=DEV)
    kn = torch.empty(B, Hkv, 1, D, dtype=torch.bfloat16, device=DEV)
    vn = torch.empty_like(kn)
    qw = (1 + 0.02 * randn(D, seed=953)).to(DEV)
    kw = (1 + 0.02 * randn(D, seed=954)).to(DEV)
    cos, sin = (t.to(DEV) for t in nq.build_tables(D, T, 1e6))
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(nq.decode_workspace_bytes(B, Hq, Hkv, D, T), dtype=torch.uint8, device=DEV)
    append = nq.qk_norm_rope(k=kn, v=vn, k_out=kc, v_out=vc, k_weight=kw, cos=cos, sin=sin,
                             pos_base=row, kv_row_base=row, plan=True)
    decode = nq.attention_decode(q, kc, vc, lens, max_len=T, q_weight=qw, cos=cos, sin=sin,
                                 out=out, workspace=ws, plan=True)

    def fill(i):
        q.copy_(randn(B, Hq, 1, D, seed=960 + i, dtype=torch.bfloat16))
        kn.copy_(randn(B, Hkv, 1, D, seed=970 + i, dtype=torch.bfloat16))
        vn.copy_(randn(B, Hkv, 1, D, seed=980 + i, dtype=torch.bfloat16))

    fill(0)
    side = torch.cuda.Stream()                       # warm-up launches off the default stream
    side.wait_stream(torch.cuda.current_stream())
    append.launch(side)
    decode.launch(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cs = torch.cuda.current_stream()
        append.launch(cs)
        decode.launch(cs)
    torch.cuda.synchronize()
    for i in range(1, 4):
        fill(i)
        kc0, vc0 = kc.clone(), vc.clone()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        # the same step, eager, on copies of the buffers as they were before the replay
        nq.qk_norm_rope(k=kn, v=vn, k_out=kc0, v_out=vc0, k_weight=kw, cos=cos, sin=sin,
                        pos_base=row, kv_row_base=row)
        ref = nq.attention_decode(q, kc0, vc0, lens, max_len=T, q_weight=qw, cos=cos, sin=sin)
        torch.cuda.synchronize()
        assert torch.equal(kc, kc0) and torch.equal(vc, vc0), f"replay {i}: cache rows differ"
        assert torch.equal(out, ref), f"replay {i}: max diff {float((out.float() - ref.float()).abs().max())}"
        assert not torch.equal(ref, torch.zeros_like(ref))
