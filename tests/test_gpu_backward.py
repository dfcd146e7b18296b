"""GPU parity of the attention backward and the QK-Norm + RoPE backward.

References are torch autograd in fp64 on the CPU through the oracle's
functions (``attention``, ``rms_norm``, ``rotate_half``, pinned by the
oracle tests), on the same bf16-valued (or fp32) inputs.

Tolerance for gradients, relative to the largest reference magnitude of the
same tensor: bf16 storage max-abs <= 2e-2 * max|ref| and mean-abs <=
2e-3 * max|ref| (the bf16 gate of the forward, scaled to the tensor); fp32
storage, whose products run on fp32 MFMA, max-abs <= 1e-5 * max|ref| and
mean-abs <= 1e-6 * max|ref|.
"""

import pytest
import torch

import nano_qwen_amd as nq
from nano_qwen_amd import ops
from oracle import attention, attention_module_forward, rms_norm, rope_tables, rotate_half
from tests.helpers import randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close_rel(got, ref, what, dtype=torch.bfloat16):
    assert got.dtype == dtype, f"{what}: {got.dtype} result for {dtype} inputs"
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    scale = float(ref.abs().max())
    mx_tol, mean_tol = (1e-5, 1e-6) if dtype == torch.float32 else (2e-2, 2e-3)
    d = (got - ref).abs()
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    assert float(d.max()) <= mx_tol * scale and float(d.mean()) <= mean_tol * scale, \
        f"{what}: max-abs {float(d.max()):.3e} mean-abs {float(d.mean()):.3e} (ref max {scale:.3e})"


def _ref_grads(q, k, v, do, causal, scale=None):
    qd, kd, vd = (t.detach().double().cpu().requires_grad_(True) for t in (q, k, v))
    S, T = q.shape[2], k.shape[2]
    o = attention(qd, kd, vd, causal=causal, causal_offset=T - S, scale=scale,
                  compute_dtype=torch.float64)
    o.backward(do.double().cpu())
    return o.detach(), qd.grad, kd.grad, vd.grad


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (8, 2), (16, 1)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_backward_against_fp64_autograd(D, Hq, Hkv, causal):
    say(f"bwd D={D} {Hq}/{Hkv} causal={causal}")
    B, S = 2, 200
    q = randn(B, Hq, S, D, seed=501, dtype=torch.bfloat16)
    k = randn(B, Hkv, S, D, seed=502, dtype=torch.bfloat16)
    v = randn(B, Hkv, S, D, seed=503, dtype=torch.bfloat16)
    do = randn(B, Hq, S, D, seed=504, dtype=torch.bfloat16)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=causal)
    _, rq, rk, rv = _ref_grads(q, k, v, do, causal)
    _close_rel(dq, rq, "dq")
    _close_rel(dk, rk, "dk")
    _close_rel(dv, rv, "dv")


@pytest.mark.parametrize("S,T,Hq,Hkv,causal", [
    (2, 2, 2, 2, True), (17, 17, 2, 2, True), (32, 32, 2, 2, True), (33, 33, 2, 2, True),
    (64, 64, 2, 2, True), (96, 96, 2, 2, True), (129, 129, 2, 1, True), (250, 250, 4, 1, True),
    (40, 300, 2, 1, True), (96, 96, 2, 2, False), (33, 200, 4, 2, False)])
def test_dkdv_steps_per_block_and_partial_tiles(S, T, Hq, Hkv, causal):
    """head_dim 128: key blocks that walk one, two, three or many query steps, a top
    tile that runs past S, keys past the last query (bottom-right causal) and keys
    of a block past T (every wave of the dK/dV kernel masked or partly masked)."""
    say(f"bwd steps S={S} T={T} {Hq}/{Hkv} causal={causal}")
    B, D = 2, 128
    q = randn(B, Hq, S, D, seed=531, dtype=torch.bfloat16)
    k = randn(B, Hkv, T, D, seed=532, dtype=torch.bfloat16)
    v = randn(B, Hkv, T, D, seed=533, dtype=torch.bfloat16)
    do = randn(B, Hq, S, D, seed=534, dtype=torch.bfloat16)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=causal)
    _, rq, rk, rv = _ref_grads(q, k, v, do, causal)
    _close_rel(dq, rq, "dq")
    _close_rel(dk, rk, "dk")
    _close_rel(dv, rv, "dv")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attention_backward_bottom_right_causal_and_dtypes(dtype):
    """S < T (queries are the last S positions), ragged sizes, fp32 storage too."""
    say(f"bwd S<T {dtype}")
    B, Hq, Hkv, S, T, D = 1, 8, 4, 77, 301, 128
    q = randn(B, Hq, S, D, seed=511, dtype=dtype)
    k = randn(B, Hkv, T, D, seed=512, dtype=dtype)
    v = randn(B, Hkv, T, D, seed=513, dtype=dtype)
    do = randn(B, Hq, S, D, seed=514, dtype=dtype)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=True)
    _, rq, rk, rv = _ref_grads(q, k, v, do, True)
    for got, ref, name in ((dq, rq, "dq"), (dk, rk, "dk"), (dv, rv, "dv")):
        _close_rel(got, ref, name, dtype)


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("Hq,Hkv,S,T,causal", [(4, 4, 200, 200, True), (8, 2, 77, 301, True),
                                                (16, 1, 130, 130, False), (8, 8, 257, 64, False)])
def test_fp32_attention_backward(D, Hq, Hkv, S, T, causal):
    """fp32 storage runs the fp32 MFMA backward: every gradient at the fp32 gate
    against fp64 autograd, the forward's O and LSE from the fp32 prefill."""
    say(f"bwd fp32 D={D} {Hq}/{Hkv} S={S} T={T} causal={causal}")
    B = 2
    q = randn(B, Hq, S, D, seed=581 + D)
    k = randn(B, Hkv, T, D, seed=582 + D)
    v = randn(B, Hkv, T, D, seed=583 + D)
    do = randn(B, Hq, S, D, seed=584 + D)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=causal)
    ro, rq, rk, rv = _ref_grads(q, k, v, do, causal)
    _close_rel(o, ro, "o", torch.float32)
    for got, ref, name in ((dq, rq, "dq"), (dk, rk, "dk"), (dv, rv, "dv")):
        _close_rel(got, ref, name, torch.float32)


def test_attention_backward_long_sequence():
    """B1 S2048 16/8 D128 causal, every gradient element against fp64 autograd."""
    say("bwd S=2048")
    B, Hq, Hkv, S, D = 1, 16, 8, 2048, 128
    q = randn(B, Hq, S, D, seed=521, dtype=torch.bfloat16)
    k = randn(B, Hkv, S, D, seed=522, dtype=torch.bfloat16)
    v = randn(B, Hkv, S, D, seed=523, dtype=torch.bfloat16)
    do = randn(B, Hq, S, D, seed=524, dtype=torch.bfloat16)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=True)
    _, rq, rk, rv = _ref_grads(q, k, v, do, True)
    _close_rel(dq, rq, "dq S=2048")
    _close_rel(dk, rk, "dk S=2048")
    _close_rel(dv, rv, "dv S=2048")


@pytest.mark.parametrize("S,T", [(100, 333), (257, 64)])
def test_attention_backward_non_causal_cross_lengths(S, T):
    """Non-causal with S != T (more keys than queries and fewer), ragged sizes."""
    say(f"bwd non-causal S={S} T={T}")
    B, Hq, Hkv, D = 2, 8, 2, 128
    q = randn(B, Hq, S, D, seed=571, dtype=torch.bfloat16)
    k = randn(B, Hkv, T, D, seed=572, dtype=torch.bfloat16)
    v = randn(B, Hkv, T, D, seed=573, dtype=torch.bfloat16)
    do = randn(B, Hq, S, D, seed=574, dtype=torch.bfloat16)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=False, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=False)
    _, rq, rk, rv = _ref_grads(q, k, v, do, False)
    _close_rel(dq, rq, "dq")
    _close_rel(dk, rk, "dk")
    _close_rel(dv, rv, "dv")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_norm_rope_backward_against_fp64_autograd(dtype, D):
    say(f"norm+rope bwd D={D} {dtype}")
    B, H, S = 2, 3, 50
    x = randn(B, H, S, D, seed=531, dtype=dtype, scale=2.0)
    dy = randn(B, H, S, D, seed=532, dtype=dtype)
    w = 1 + 0.1 * randn(D, seed=533)
    cos, sin = rope_tables(D, 512, 1e6)
    pos = torch.randint(0, 512, (B, S), generator=torch.Generator().manual_seed(534))
    dx, dw = ops.qk_norm_rope_backward(x.to(DEV), dy.to(DEV), weight=w.to(DEV), eps=1e-6,
                                       cos=cos.to(DEV), sin=sin.to(DEV), position_ids=pos.to(DEV))
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    y = rotate_half(rms_norm(xd, wd, 1e-6, compute_dtype=torch.float64),
                    cos.double()[pos][:, None], sin.double()[pos][:, None])
    y.backward(dy.double())
    _close_rel(dx, xd.grad, "dx", dtype)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    torch.testing.assert_close(dw.double().cpu(), wd.grad, rtol=tol, atol=tol * float(wd.grad.abs().max()))


def test_flash_attention_mirror_autograd():
    say("flash_attention autograd")
    B, H, S, D = 2, 4, 96, 64
    q = randn(B, H, S, D, seed=541, dtype=torch.bfloat16).to(DEV).requires_grad_(True)
    k = randn(B, H, S, D, seed=542, dtype=torch.bfloat16).to(DEV).requires_grad_(True)
    v = randn(B, H, S, D, seed=543, dtype=torch.bfloat16).to(DEV).requires_grad_(True)
    do = randn(B, H, S, D, seed=544, dtype=torch.bfloat16)
    o = nq.flash_attention(q, k, v, causal=True)
    assert o.is_contiguous()
    o.backward(do.to(DEV))
    _, rq, rk, rv = _ref_grads(q, k, v, do, True)
    _close_rel(q.grad, rq, "flash dq")
    _close_rel(k.grad, rk, "flash dk")
    _close_rel(v.grad, rv, "flash dv")


@pytest.mark.parametrize("causal", [True, False])
def test_flash_attention_head_dim_16(causal):
    """head_dim 16, which the reference's kernel accepts (kernels/flash_attn.py:106),
    runs on the head_dim-32 kernels with zero padding: the output and the
    gradients against fp64 autograd at D = 16 (default scale 1/4), and a
    contiguous (B, H, N, 16) result."""
    say(f"flash_attention D=16 causal={causal}")
    B, H, S, D = 2, 4, 150, 16
    q = randn(B, H, S, D, seed=551, dtype=torch.bfloat16).to(DEV).requires_grad_(True)
    k = randn(B, H, S, D, seed=552, dtype=torch.bfloat16).to(DEV).requires_grad_(True)
    v = randn(B, H, S, D, seed=553, dtype=torch.bfloat16).to(DEV).requires_grad_(True)
    do = randn(B, H, S, D, seed=554, dtype=torch.bfloat16)
    o = nq.flash_attention(q, k, v, causal=causal)
    assert o.shape == (B, H, S, D) and o.is_contiguous()
    ro, rq, rk, rv = _ref_grads(q, k, v, do, causal)
    _close_rel(o, ro, "D16 out")
    o.backward(do.to(DEV))
    _close_rel(q.grad, rq, "D16 dq")
    _close_rel(k.grad, rk, "D16 dk")
    _close_rel(v.grad, rv, "D16 dv")
    with torch.no_grad():  # the inference path, with an explicit scale
        o2 = nq.flash_attention(q.detach(), k.detach(), v.detach(), causal=causal, sm_scale=0.1)
    ro2, _, _, _ = _ref_grads(q, k, v, do, causal, scale=0.1)
    _close_rel(o2, ro2, "D16 scale")


@pytest.mark.parametrize("Hq,Hkv,S,T,causal", [(4, 4, 150, 150, True), (8, 2, 77, 301, True), (2, 1, 20, 20, True),
                                                (4, 2, 130, 130, False), (4, 4, 257, 64, False)])
def test_attention_backward_head_dim_256(Hq, Hkv, S, T, causal):
    """head_dim 256 on its own backward kernels: dq, dk, dv against fp64 autograd;
    GQA sums over the group, S < T and S > T, and a sequence shorter than one
    64-row query block (its scratch holds a single 32-row tile)."""
    say(f"bwd D=256 {Hq}/{Hkv} S={S} T={T} causal={causal}")
    B, D = 2, 256
    q = randn(B, Hq, S, D, seed=591, dtype=torch.bfloat16)
    k = randn(B, Hkv, T, D, seed=592, dtype=torch.bfloat16)
    v = randn(B, Hkv, T, D, seed=593, dtype=torch.bfloat16)
    do = randn(B, Hq, S, D, seed=594, dtype=torch.bfloat16)
    o, lse = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, return_lse=True)
    dq, dk, dv = ops.attention_backward(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), lse, causal=causal)
    _, rq, rk, rv = _ref_grads(q, k, v, do, causal)
    _close_rel(dq, rq, "dq D=256")
    _close_rel(dk, rk, "dk D=256")
    _close_rel(dv, rv, "dv D=256")


def test_flash_attention_head_dim_256_autograd():
    say("flash_attention D=256 autograd")
    B, H, S, D = 2, 4, 100, 256
    q = randn(B, H, S, D, seed=601, dtype=torch.bfloat16).to(DEV).requires_grad_(True)
    k = randn(B, H, S, D, seed=602, dtype=torch.bfloat16).to(DEV).requires_grad_(True)
    v = randn(B, H, S, D, seed=603, dtype=torch.bfloat16).to(DEV).requires_grad_(True)
    do = randn(B, H, S, D, seed=604, dtype=torch.bfloat16)
    o = nq.flash_attention(q, k, v, causal=True)
    o.backward(do.to(DEV))
    ro, rq, rk, rv = _ref_grads(q, k, v, do, True)
    _close_rel(o, ro, "D256 out")
    _close_rel(q.grad, rq, "D256 dq")
    _close_rel(k.grad, rk, "D256 dk")
    _close_rel(v.grad, rv, "D256 dv")


def _module_grads(weights, h, g, pos, cos, sin, dtype, H, Hkv, D):
    """Oracle module forward + backward on the CPU in ``dtype`` (the reference's dtype flow)."""
    w = {n: t.detach().to(dtype).clone().requires_grad_(True) for n, t in weights.items()}
    out, _ = attention_module_forward(h.to(dtype), w, num_heads=H, num_kv_heads=Hkv, head_dim=D, eps=1e-6,
                                      cos_table=cos.to(dtype), sin_table=sin.to(dtype), position_ids=pos)
    out.backward(g.to(dtype))
    return out.detach().double(), {n: t.grad.double() for n, t in w.items()}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_training_gradients_against_oracle(dtype):
    """Attention.forward + backward on the kernels against the oracle module under autograd.

    fp32 module: within the relative bound above of fp64 autograd.  bf16
    module: no further from fp64 autograd than the reference's own arithmetic
    run in bf16 (the oracle module in bf16 on the CPU, the dtype flow of
    model/attention.py under SDPA autograd) is, within a factor 1.5.
    """
    say(f"module train grads {dtype}")
    hidden, H, Hkv, D, B, S = 256, 8, 2, 64, 2, 80
    cfg = nq.AttentionConfig(hidden_size=hidden, num_attention_heads=H, num_key_value_heads=Hkv,
                             head_dim=D, max_position_embeddings=256)
    torch.manual_seed(0)
    attn = nq.Attention(cfg)
    with torch.no_grad():
        attn.q_norm.weight.add_(0.1 * torch.randn(D))
        attn.k_norm.weight.add_(0.1 * torch.randn(D))
    attn = attn.to(DEV, dtype).train()
    # the references take the module's own (possibly bf16-rounded) weights
    names = ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm")
    weights = {n: getattr(attn, n).weight.detach().cpu() for n in names}
    h = randn(B, S, hidden, seed=551, dtype=dtype)
    g = randn(B, S, hidden, seed=552, dtype=dtype)
    pos = torch.stack([torch.arange(S) + 3, torch.arange(S) * 2])
    out = attn(h.to(DEV), position_ids=pos.to(DEV))
    out.backward(g.to(DEV))
    cos, sin = rope_tables(D, 256, 1e6)
    ref_out, ref_g = _module_grads(weights, h, g, pos, cos, sin, torch.float64, H, Hkv, D)
    if dtype == torch.float32:
        _close_rel(out, ref_out, "module out", dtype)
        for n in names:
            _close_rel(getattr(attn, n).weight.grad, ref_g[n], f"grad {n}", dtype)
        return
    _, bf_g = _module_grads(weights, h, g, pos, cos, sin, torch.bfloat16, H, Hkv, D)
    for n in names:
        got = getattr(attn, n).weight.grad.double().cpu()
        e_k = (got - ref_g[n]).abs()
        e_r = (bf_g[n] - ref_g[n]).abs()
        floor = 1e-3 * float(ref_g[n].abs().max())
        assert float(e_k.mean()) <= 1.5 * float(e_r.mean()) + floor, \
            f"grad {n}: mean error {float(e_k.mean()):.3e}, reference bf16 autograd {float(e_r.mean()):.3e}"
        assert float(e_k.max()) <= 1.5 * float(e_r.max()) + floor, \
            f"grad {n}: max error {float(e_k.max()):.3e}, reference bf16 autograd {float(e_r.max()):.3e}"


def test_attention_backward_wide_dq_workgroups_bit_equal():
    """B8 S4096 16/8 D128 causal: enough dQ work for the 8-wave (256-row) workgroups.
    Each row's dQ accumulates over the same key tiles in the same order in the 4-wave
    workgroups that a one-sequence launch uses, and tiles past a row's frontier add
    exact zeros, so the batched call equals the per-sequence calls bit for bit."""
    say("bwd wide dQ workgroups vs per-sequence launches")
    B, Hq, Hkv, S, D = 8, 16, 8, 4096, 128
    q = randn(B, S, Hq, D, seed=561, dtype=torch.bfloat16).to(DEV).transpose(1, 2)
    k = randn(B, S, Hkv, D, seed=562, dtype=torch.bfloat16).to(DEV).transpose(1, 2)
    v = randn(B, S, Hkv, D, seed=563, dtype=torch.bfloat16).to(DEV).transpose(1, 2)
    do = randn(B, S, Hq, D, seed=564, dtype=torch.bfloat16).to(DEV).transpose(1, 2)
    o, lse = ops.attention_prefill(q, k, v, causal=True, return_lse=True)
    dq, dk, dv = ops.attention_backward(q, k, v, o, do, lse, causal=True)
    for b in (0, 5):
        sl = slice(b, b + 1)
        dq1, dk1, dv1 = ops.attention_backward(q[sl], k[sl], v[sl], o[sl], do[sl], lse[sl], causal=True)
        for got, ref, name in ((dq[sl], dq1, "dq"), (dk[sl], dk1, "dk"), (dv[sl], dv1, "dv")):
            assert torch.equal(got, ref), f"{name} batch {b}: max diff {float((got.float() - ref.float()).abs().max())}"
    # and one sequence against fp64 autograd on its last 256 queries (all keys)
    b, q0 = 3, S - 256
    qs = q[b:b + 1, :, q0:].cpu()
    _, rq, _, _ = _ref_grads(qs, k[b:b + 1].cpu(), v[b:b + 1].cpu(), do[b:b + 1, :, q0:].cpu(), True)
    _close_rel(dq[b:b + 1, :, q0:], rq, "dq (wide workgroups, last 256 rows)")


def _fp32_grads_on_device(q, k, v, do, causal=True):
    """fp32 autograd on the device for one (batch, kv head) slice.

    q, do: (G, S, D); k, v: (T, D).  The oracle's math (softmax(q k^T / sqrt(D)) v, key j
    kept for query i iff j <= i + T - S) with fp32 torch matmuls on the GPU, for shapes
    where fp64 autograd on the CPU would take minutes.  Returns dq, dk, dv in fp32.
    """
    qd, kd, vd = (t.detach().to(DEV).float().requires_grad_(True) for t in (q, k, v))
    S, T, D = qd.shape[1], kd.shape[0], qd.shape[2]
    sc = torch.matmul(qd, kd.t().contiguous()) * D ** -0.5
    if causal:
        past = torch.arange(T, device=DEV)[None, :] > torch.arange(S, device=DEV)[:, None] + (T - S)
        sc = sc.masked_fill(past, float("-inf"))
    o = torch.matmul(torch.softmax(sc, dim=-1), vd)
    o.backward(do.to(DEV).float())
    return qd.grad, kd.grad, vd.grad


def test_device_fp32_gradients_match_fp64_autograd():
    """The device reference of the full-size backward test against fp64 autograd on the CPU."""
    say("bwd device fp32 reference vs fp64 autograd")
    G, S, T, D = 4, 300, 333, 128
    q = randn(1, G, S, D, seed=571, dtype=torch.bfloat16)
    k = randn(1, 1, T, D, seed=572, dtype=torch.bfloat16)
    v = randn(1, 1, T, D, seed=573, dtype=torch.bfloat16)
    do = randn(1, G, S, D, seed=574, dtype=torch.bfloat16)
    for causal in (True, False):
        _, rq, rk, rv = _ref_grads(q, k, v, do, causal)
        gq, gk, gv = _fp32_grads_on_device(q[0], k[0, 0], v[0, 0], do[0], causal)
        for got, ref, name in ((gq, rq[0], "dq"), (gk, rk[0, 0], "dk"), (gv, rv[0, 0], "dv")):
            torch.testing.assert_close(got.double().cpu(), ref, rtol=1e-4, atol=1e-4 * float(ref.abs().max()),
                                       msg=lambda m: f"{name} causal={causal}: {m}")


@pytest.mark.parametrize("B,Hq,Hkv,S", [(8, 16, 8, 2048), (4, 32, 8, 8192)])
def test_attention_backward_full_size(B, Hq, Hkv, S):
    """The two benchmarked backward shapes (Qwen3-1.7B-like and 8B-like, D128 causal bf16)
    in one launch each; every (batch, kv head) slice's dq, dk, dv against fp32 autograd on
    the device."""
    say(f"bwd full size B{B} S{S} {Hq}/{Hkv}")
    D, G = 128, Hq // Hkv
    q = randn(B, S, Hq, D, seed=581, dtype=torch.bfloat16).to(DEV).transpose(1, 2)
    k = randn(B, S, Hkv, D, seed=582, dtype=torch.bfloat16).to(DEV).transpose(1, 2)
    v = randn(B, S, Hkv, D, seed=583, dtype=torch.bfloat16).to(DEV).transpose(1, 2)
    do = randn(B, S, Hq, D, seed=584, dtype=torch.bfloat16).to(DEV).transpose(1, 2)
    o, lse = ops.attention_prefill(q, k, v, causal=True, return_lse=True)
    dq, dk, dv = ops.attention_backward(q, k, v, o, do, lse, causal=True)
    torch.cuda.synchronize()
    for b in range(B):
        for kvh in range(Hkv):
            hs = slice(kvh * G, (kvh + 1) * G)
            rq, rk, rv = _fp32_grads_on_device(q[b, hs], k[b, kvh], v[b, kvh], do[b, hs])
            for got, ref, name in ((dq[b, hs], rq, "dq"), (dk[b, kvh], rk, "dk"), (dv[b, kvh], rv, "dv")):
                _close_rel(got, ref, f"{name} b={b} kvh={kvh}")
