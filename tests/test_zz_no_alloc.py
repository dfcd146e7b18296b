"""nq_attn_decode_paged_fwd_noalloc (workspace in a static device array) against
nq_attn_decode_paged_fwd (caller-owned workspace), both through the C ABI:
two calls in a row, the second with smaller sizes, each with the new token's
append fused in.  Same kernels and schedule, so outputs, appended cache rows and
lens_out must be bit-identical."""

import ctypes

import pytest
import torch

from nano_qwen_amd import _lib
from oracle import rope_tables
from tests.helpers import randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _i64(*vals):
    return (ctypes.c_int64 * len(vals))(*vals)


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _case(B, Hq, Hkv, D, P, pages_per_seq, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    npages = B * pages_per_seq + 3
    table = torch.randperm(npages, generator=g)[:B * pages_per_seq].to(torch.int32).view(B, pages_per_seq)
    max_len = P * pages_per_seq
    lens = torch.randint(0, max_len, (B,), generator=g, dtype=torch.int32)
    return dict(
        q=randn(B, Hq, D, seed=seed + 1, dtype=dtype).to(DEV),
        kn=randn(B, Hkv, D, seed=seed + 2, dtype=dtype).to(DEV),
        vn=randn(B, Hkv, D, seed=seed + 3, dtype=dtype).to(DEV),
        kpool=randn(npages, Hkv, P, D, seed=seed + 4, dtype=dtype).to(DEV),
        vpool=randn(npages, Hkv, P, D, seed=seed + 5, dtype=dtype).to(DEV),
        table=table.to(DEV), lens=lens.to(DEV), max_len=max_len,
        qw=(1 + 0.02 * randn(D, seed=seed + 6)).to(DEV), kw=(1 + 0.02 * randn(D, seed=seed + 7)).to(DEV),
        B=B, Hq=Hq, Hkv=Hkv, D=D, P=P, dtype=dtype)


def _run(c, noalloc, cos, sin):
    lib = _lib.load()
    kp, vp = c["kpool"].clone(), c["vpool"].clone()
    out = torch.empty(c["B"], c["Hq"], c["D"], dtype=c["dtype"], device=DEV)
    lens_out = torch.empty_like(c["lens"])
    q, kn, vn = c["q"], c["kn"], c["vn"]
    head = (_p(q), _i64(q.stride(0), q.stride(1)), _p(kn), _i64(kn.stride(0), kn.stride(1)), _p(vn),
            _i64(vn.stride(0), vn.stride(1)), _p(c["kw"]), _p(kp), _i64(*kp.stride()[:3]), _p(vp),
            _i64(*vp.stride()[:3]), _p(c["table"]), c["table"].stride(0), c["P"], _p(c["lens"]), _p(lens_out),
            _p(out), _i64(out.stride(0), out.stride(1)))
    code = _lib.NQ_DTYPE_F32 if c["dtype"] == torch.float32 else _lib.NQ_DTYPE_BF16
    tail = (c["B"], c["Hq"], c["Hkv"], c["D"], c["max_len"], c.get("chunk", 0), code, _p(c["qw"]), 1e-6,
            _p(cos), _p(sin), cos.shape[0], None, -1, 0.0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    if noalloc:
        rc = lib.nq_attn_decode_paged_fwd_noalloc(*head, *tail)
        _lib.check(rc, "nq_attn_decode_paged_fwd_noalloc")
    else:
        need = lib.nq_attn_decode_workspace_bytes(c["B"], c["Hq"], c["Hkv"], c["D"], c["max_len"], c.get("chunk", 0))
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        rc = lib.nq_attn_decode_paged_fwd(*head, _p(ws), need, *tail)
        _lib.check(rc, "nq_attn_decode_paged_fwd")
    torch.cuda.synchronize()
    return out, kp, vp, lens_out


def test_noalloc_decode_equals_workspace_decode():
    cos, sin = (t.to(DEV) for t in rope_tables(128, 4096, 1e6))
    # two calls in a row on the shared scratch, the second smaller
    for name, args in (("B48 64/4 D128 P64", (48, 64, 4, 128, 64, 40, 9100)),
                       ("B5 16/8 D128 P32", (5, 16, 8, 128, 32, 7, 9200))):
        say(f"no-alloc decode {name}")
        c = _case(*args)
        want = _run(c, False, cos, sin)
        got = _run(c, True, cos, sin)
        for w, g_, what in zip(want, got, ("out", "k_pool", "v_pool", "lens_out")):
            assert torch.equal(w, g_), f"{name}: {what} differs"
        assert torch.isfinite(got[0].float()).all()


def test_noalloc_refuses_sizes_beyond_the_scratch():
    say("no-alloc decode: oversized")
    lib = _lib.load()
    need = lib.nq_attn_decode_workspace_bytes(512, 64, 8, 128, 1024, 32)
    assert need > (16 << 20)
    z = _i64(0, 0, 0)
    rc = lib.nq_attn_decode_paged_fwd_noalloc(
        None, z, None, None, None, None, None, None, z, None, z, None, 1, 32, None, None, None, z,
        512, 64, 8, 128, 1024, 32, _lib.NQ_DTYPE_BF16, None, 1e-6, None, None, 0, None, -1, 0.0, None)
    assert rc == _lib.NQ_ERR_WORKSPACE
    assert b"static scratch" in lib.nq_last_error()


def test_noalloc_fp32_needs_no_scratch():
    """fp32 caches keep no partials, so sizes whose bf16 workspace would exceed
    the static scratch are served, with the workspace path's bits."""
    say("no-alloc decode: fp32 beyond the bf16 scratch size")
    lib = _lib.load()
    c = _case(16, 64, 4, 128, 64, 64, 9300, dtype=torch.float32)
    c["chunk"] = 32
    assert lib.nq_attn_decode_workspace_bytes(16, 64, 4, 128, c["max_len"], 32) > (16 << 20)
    cos, sin = (t.to(DEV) for t in rope_tables(128, 4096, 1e6))
    want = _run(c, False, cos, sin)
    got = _run(c, True, cos, sin)
    for w, g_, what in zip(want, got, ("out", "k_pool", "v_pool", "lens_out")):
        assert torch.equal(w, g_), f"fp32: {what} differs"
    assert torch.isfinite(got[0]).all()
