"""GPU parity of the prefill attention kernel against the oracle (fp32 reference math)."""

import pytest
import torch

import nano_qwen_amd as nq
from oracle import attention, attention_path, rms_norm, rope_tables, rotate_half
from tests.helpers import assert_bf16_close, assert_close_for, assert_fp32_close, randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def gpu_attention(q, k, v, qw, kw, eps, cos, sin, causal=True, position_ids=None, pos_offset=0):
    """The drop-in's prefill sequence: K-Norm+RoPE row kernel, then the fused prefill kernel."""
    kh = nq.qk_norm_rope(k=k, k_weight=kw, eps=eps, cos=cos, sin=sin, position_ids=position_ids,
                         pos_offset=pos_offset)[1]
    return nq.attention_prefill(q, kh, v, q_weight=qw, eps=eps, cos=cos, sin=sin,
                                position_ids=position_ids, pos_offset=pos_offset, causal=causal)


def make(B, S, Hq, Hkv, D, dtype, seed, model_layout=True, wscale=0.02):
    if model_layout:  # (B, S, H, D) storage viewed as (B, H, S, D), as q_proj(...).view().transpose()
        q = randn(B, S, Hq, D, seed=seed, dtype=dtype).transpose(1, 2)
        k = randn(B, S, Hkv, D, seed=seed + 1, dtype=dtype).transpose(1, 2)
        v = randn(B, S, Hkv, D, seed=seed + 2, dtype=dtype).transpose(1, 2)
    else:
        q = randn(B, Hq, S, D, seed=seed, dtype=dtype)
        k = randn(B, Hkv, S, D, seed=seed + 1, dtype=dtype)
        v = randn(B, Hkv, S, D, seed=seed + 2, dtype=dtype)
    qw = 1 + wscale * randn(D, seed=seed + 3)
    kw = 1 + wscale * randn(D, seed=seed + 4)
    return q, k, v, qw, kw


def run_case(B, S, Hq, Hkv, D, dtype, seed, causal=True, rope_scaling=None, max_pos=None,
             pos_offset=0, model_layout=True):
    q, k, v, qw, kw = make(B, S, Hq, Hkv, D, dtype, seed, model_layout)
    max_pos = max_pos or (S + pos_offset)
    cos, sin = rope_tables(D, max_pos, 1e6, rope_scaling)
    o = gpu_attention(q.to(DEV), k.to(DEV), v.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6,
                      cos.to(DEV), sin.to(DEV), causal=causal, pos_offset=pos_offset)
    torch.cuda.synchronize()
    pos = torch.arange(pos_offset, pos_offset + S)
    ref = attention_path(q.float(), k.float(), v.float(), q_weight=qw, k_weight=kw, eps=1e-6,
                         cos=cos, sin=sin, q_pos=pos, causal=causal)
    return o.cpu(), ref


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_debug_scale_config(dtype):
    """B2 S256 Hq8 Hkv2 D64 causal, norm weights 1, theta 1e6 (the CPU-runnable config)."""
    say(f"prefill debug config {dtype}")
    q, k, v, _, _ = make(2, 256, 8, 2, 64, dtype, seed=1000)
    ones = torch.ones(64)
    cos, sin = rope_tables(64, 256, 1e6)
    o = gpu_attention(q.to(DEV), k.to(DEV), v.to(DEV), ones.to(DEV), ones.to(DEV), 1e-6,
                      cos.to(DEV), sin.to(DEV))
    ref = attention_path(q.float(), k.float(), v.float(), q_weight=ones, k_weight=ones, eps=1e-6,
                         cos=cos, sin=sin, q_pos=torch.arange(256), causal=True)
    assert o.dtype == dtype
    assert_close_for(dtype, o, ref, "debug config")


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("Hq,Hkv,S,causal", [(8, 2, 256, True), (4, 4, 77, True), (16, 1, 130, False),
                                              (32, 4, 33, True), (8, 8, 1, True)])
def test_fp32_prefill(D, Hq, Hkv, S, causal):
    """fp32 inputs run the fp32 MFMA kernel: QK-Norm + RoPE + GQA attention at the fp32 gate."""
    say(f"prefill fp32 D={D} Hq={Hq} Hkv={Hkv} S={S} causal={causal}")
    o, ref = run_case(2, S, Hq, Hkv, D, torch.float32, seed=300 + D + S, causal=causal)
    assert_fp32_close(o, ref, f"fp32 D={D} G={Hq // Hkv} S={S}")


def test_fp32_queries_after_cached_keys_and_lse():
    """fp32, S < T (bottom-right causal) with the log-sum-exp output."""
    say("prefill fp32 S<T + lse")
    B, S, T, Hq, Hkv, D = 2, 45, 203, 8, 2, 64
    q = randn(B, Hq, S, D, seed=61)
    k = randn(B, Hkv, T, D, seed=62)
    v = randn(B, Hkv, T, D, seed=63)
    o, lse = nq.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, return_lse=True)
    ref = attention(q.float(), k.float(), v.float(), causal=True, causal_offset=T - S)
    assert_fp32_close(o, ref, "fp32 S<T")
    s = torch.matmul(q, k.repeat_interleave(Hq // Hkv, 1).transpose(-1, -2))
    s = s / D ** 0.5
    keep = torch.ones(S, T, dtype=torch.bool).tril(T - S)
    s = s.masked_fill(~keep, float("-inf"))
    torch.testing.assert_close(lse.cpu(), torch.logsumexp(s, -1), rtol=0, atol=1e-5)


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (16, 8), (32, 8), (32, 4), (32, 2)])
@pytest.mark.parametrize("S", [1, 77, 300])
def test_gqa_group_sizes(Hq, Hkv, S):
    say(f"prefill G={Hq // Hkv} S={S}")
    o, ref = run_case(2, S, Hq, Hkv, 128, torch.bfloat16, seed=7 + S)
    assert_bf16_close(o, ref, f"G={Hq // Hkv} S={S}")


@pytest.mark.parametrize("D", [64, 128])
def test_non_causal(D):
    say(f"prefill non-causal D={D}")
    o, ref = run_case(2, 150, 8, 2, D, torch.bfloat16, seed=21, causal=False)
    assert_bf16_close(o, ref, "non-causal")


def test_contiguous_bhsd_inputs():
    say("prefill BHSD inputs")
    o, ref = run_case(1, 200, 16, 8, 128, torch.bfloat16, seed=23, model_layout=False)
    assert_bf16_close(o, ref, "bhsd")


@pytest.mark.parametrize("causal", [True, False])
def test_queries_after_cached_keys(causal):
    """S < T: queries are the last S of T positions (causal is bottom-right aligned)."""
    say(f"prefill S<T causal={causal}")
    B, S, T, Hq, Hkv, D = 2, 45, 203, 8, 2, 128
    q = randn(B, Hq, S, D, seed=31, dtype=torch.bfloat16)
    k = randn(B, Hkv, T, D, seed=32, dtype=torch.bfloat16)
    v = randn(B, Hkv, T, D, seed=33, dtype=torch.bfloat16)
    o = nq.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal)
    ref = attention(q.float(), k.float(), v.float(), causal=causal, causal_offset=T - S)
    assert_bf16_close(o, ref, "S<T")


def test_flash_attention_mirror_and_lse():
    say("flash_attention mirror + lse")
    B, H, N, D = 2, 4, 190, 64
    q = randn(B, H, N, D, seed=41, dtype=torch.bfloat16)
    k = randn(B, H, N, D, seed=42, dtype=torch.bfloat16)
    v = randn(B, H, N, D, seed=43, dtype=torch.bfloat16)
    o = nq.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True)
    assert o.shape == (B, H, N, D) and o.is_contiguous()
    assert_bf16_close(o, attention(q.float(), k.float(), v.float(), causal=True), "flash")
    scale = 0.3
    o2, lse = nq.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, sm_scale=scale,
                                   return_lse=True)
    assert_bf16_close(o2, attention(q.float(), k.float(), v.float(), causal=True, scale=scale), "scale")
    s = torch.matmul(q.float(), k.float().transpose(-1, -2)) * scale
    s = s.masked_fill(torch.ones(N, N, dtype=torch.bool).triu(1), float("-inf"))
    torch.testing.assert_close(lse.cpu(), torch.logsumexp(s, -1), rtol=1e-3, atol=2e-2)


@pytest.mark.parametrize("Hq,Hkv,S,T,causal", [(4, 4, 150, 150, True), (8, 2, 77, 301, True), (2, 2, 1, 1, True),
                                                (4, 1, 130, 130, False), (4, 2, 257, 64, False)])
def test_head_dim_256_prefill(Hq, Hkv, S, T, causal):
    """head_dim 256 (kernels/flash_attn.py:106 accepts it) runs on a kernel of its
    own: the output against the oracle at the bf16 gate, the LSE against
    logsumexp of the fp32 scores, flash_attention equal to it bit for bit, and
    the fused options refused."""
    say(f"prefill D=256 {Hq}/{Hkv} S={S} T={T} causal={causal}")
    B, D = 2, 256
    q = randn(B, Hq, S, D, seed=91, dtype=torch.bfloat16)
    k = randn(B, Hkv, T, D, seed=92, dtype=torch.bfloat16)
    v = randn(B, Hkv, T, D, seed=93, dtype=torch.bfloat16)
    o, lse = nq.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, return_lse=True)
    assert o.shape == (B, Hq, S, D)
    ref = attention(q.float(), k.float(), v.float(), causal=causal, causal_offset=T - S)
    assert_bf16_close(o, ref, "D=256")
    qf = q.float().reshape(B, Hkv, Hq // Hkv, S, D)
    s = torch.matmul(qf, k.float()[:, :, None].transpose(-1, -2)).reshape(B, Hq, S, T) / 16.0
    if causal:
        s = s.masked_fill(torch.ones(S, T, dtype=torch.bool).triu(T - S + 1), float("-inf"))
    torch.testing.assert_close(lse.cpu(), torch.logsumexp(s, -1), rtol=1e-3, atol=2e-2)
    if S == T and Hq == Hkv:
        f = nq.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal)
        assert f.is_contiguous() and torch.equal(f.cpu(), o.contiguous().cpu())
    with pytest.raises(RuntimeError, match="head_dim 256"):
        nq.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal,
                             q_weight=torch.ones(D, device=DEV), eps=1e-6)


def test_explicit_position_ids_and_yarn_high_positions():
    say("prefill position_ids + YaRN")
    B, S, Hq, Hkv, D = 2, 96, 8, 2, 128
    yarn = {"type": "yarn", "factor": 4.0, "original_max_position_embeddings": 32768}
    q, k, v, qw, kw = make(B, S, Hq, Hkv, D, torch.bfloat16, seed=51)
    cos, sin = rope_tables(D, 131072, 1e6, yarn)
    pos = torch.stack([torch.arange(S) + 131072 - S - 7 * b for b in range(B)])
    o = gpu_attention(q.to(DEV), k.to(DEV), v.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6,
                      cos.to(DEV), sin.to(DEV), position_ids=pos.to(DEV))
    ref = attention_path(q.float(), k.float(), v.float(), q_weight=qw, k_weight=kw, eps=1e-6,
                         cos=cos, sin=sin, q_pos=pos, causal=True)
    assert_bf16_close(o, ref, "yarn positions")


def test_qwen3_1p7b_like_full_size():
    """B8 S2048 Hq16 Hkv8 D128 bf16: CPU oracle on batches 0 and 7 (all heads, all rows),
    and every row of every head of every batch row against the fp32 math on the device."""
    say("prefill Qwen3-1.7B-like B8 S2048")
    B, S, Hq, Hkv, D = 8, 2048, 16, 8, 128
    G = Hq // Hkv
    q, k, v, qw, kw = make(B, S, Hq, Hkv, D, torch.bfloat16, seed=1001)
    cos, sin = rope_tables(D, S, 1e6)
    od = gpu_attention(q.to(DEV), k.to(DEV), v.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6,
                       cos.to(DEV), sin.to(DEV))
    o = od.cpu()
    assert torch.isfinite(o.float()).all()
    for b in (0, 7):
        ref = attention_path(q[b:b + 1].float(), k[b:b + 1].float(), v[b:b + 1].float(),
                             q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin,
                             q_pos=torch.arange(S), causal=True)
        assert_bf16_close(o[b:b + 1], ref, f"1.7B b={b}")
    for b in range(B):
        for kvh in range(Hkv):
            refs = _fp32_blocks_on_device(q, k, v, qw, kw, cos, sin, kvh, G, [0, 1024], 1024, b=b)
            for r0, ref in zip([0, 1024], refs):
                assert_bf16_close(od[b, kvh * G:(kvh + 1) * G, r0:r0 + 1024], ref,
                                  f"1.7B b={b} kvh={kvh} rows={r0}")


def _sampled_blocks(q, k, v, qw, kw, cos, sin, b, kvh, G, rows):
    """Oracle rows [r0, r1) for batch b, the G heads of kv head kvh (causal from 0)."""
    kh = rotate_half(rms_norm(k[b:b + 1, kvh:kvh + 1].float(), kw, 1e-6),
                     cos[None, None], sin[None, None])
    outs = []
    for r0, r1 in rows:
        qs = q[b:b + 1, kvh * G:(kvh + 1) * G, r0:r1].float()
        qh = rotate_half(rms_norm(qs, qw, 1e-6), cos[r0:r1][None, None], sin[r0:r1][None, None])
        outs.append(attention(qh, kh[:, :, :r1], v[b:b + 1, kvh:kvh + 1, :r1].float(),
                              causal=True, causal_offset=r0))
    return outs


def test_qwen3_8b_like_full_size():
    """B4 S8192 Hq32 Hkv8 D128 bf16: CPU oracle on sampled 128-row blocks of two (batch,
    kv head) pairs, and every head of every batch row on 1024-row blocks (the first, the
    last and two seeded random ones) against the fp32 math on the device."""
    say("prefill Qwen3-8B-like B4 S8192")
    B, S, Hq, Hkv, D = 4, 8192, 32, 8, 128
    G = Hq // Hkv
    q, k, v, qw, kw = make(B, S, Hq, Hkv, D, torch.bfloat16, seed=1002)
    cos, sin = rope_tables(D, S, 1e6)
    o = gpu_attention(q.to(DEV), k.to(DEV), v.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6,
                      cos.to(DEV), sin.to(DEV))
    rows = [(0, 128), (4000, 4128), (S - 128, S)]
    for b, kvh in ((0, 0), (3, 7)):
        for (r0, r1), ref in zip(rows, _sampled_blocks(q, k, v, qw, kw, cos, sin, b, kvh, G, rows)):
            assert_bf16_close(o[b:b + 1, kvh * G:(kvh + 1) * G, r0:r1], ref, f"8B b={b} kvh={kvh} rows={r0}")
    n = 1024
    gen = torch.Generator().manual_seed(1006)
    starts = [0, S - n] + torch.randint(1, S - n, (2,), generator=gen).tolist()
    for b in range(B):
        for kvh in range(Hkv):
            refs = _fp32_blocks_on_device(q, k, v, qw, kw, cos, sin, kvh, G, starts, n, b=b)
            for r0, ref in zip(starts, refs):
                assert_bf16_close(o[b, kvh * G:(kvh + 1) * G, r0:r0 + n], ref, f"8B b={b} kvh={kvh} rows={r0}")


def _fp32_blocks_on_device(q, k, v, qw, kw, cos, sin, kvh, G, starts, n, b=0):
    """Causal rows [r0, r0 + n) of batch b, the G heads of kv head kvh, in fp32 on the device.

    The oracle's composition (rms_norm, rotate_half, softmax(q k^T / sqrt(D)) v, all in
    fp32 from the bf16-valued inputs), with the two products as fp32 torch matmuls on the
    GPU: the CPU oracle takes ~9 s per 1024-row block at 131072 keys.  Returns (G, n, D)
    fp32 device tensors.
    """
    D = q.shape[-1]
    cd, sd = cos.to(DEV), sin.to(DEV)
    kh = rotate_half(rms_norm(k[b, kvh].to(DEV).float(), kw.to(DEV), 1e-6), cd, sd)
    vd = v[b, kvh].to(DEV).float()
    outs = []
    for r0 in starts:
        r1 = r0 + n
        qs = q[b, kvh * G:(kvh + 1) * G, r0:r1].to(DEV).float()
        qh = rotate_half(rms_norm(qs, qw.to(DEV), 1e-6), cd[r0:r1], sd[r0:r1])
        sc = torch.matmul(qh, kh[:r1].t().contiguous()) * (D ** -0.5)
        past = torch.arange(r1, device=DEV)[None, :] > torch.arange(r0, r1, device=DEV)[:, None]
        sc.masked_fill_(past, float("-inf"))
        outs.append(torch.matmul(torch.softmax(sc, dim=-1), vd[:r1]))
        del sc, past
    return outs


def test_long_context_yarn_full_size():
    """B1 S131072 Hq32 Hkv4 D128 bf16 YaRN x4, over all 32 heads: the first and last
    1024-row blocks and 6 seeded random ones, against the fp32 math on the device, which
    is first checked against the CPU oracle on a 64-row block."""
    say("prefill YaRN B1 S131072")
    B, S, Hq, Hkv, D = 1, 131072, 32, 4, 128
    G = Hq // Hkv
    yarn = {"type": "yarn", "factor": 4.0, "original_max_position_embeddings": 32768}
    q, k, v, qw, kw = make(B, S, Hq, Hkv, D, torch.bfloat16, seed=1004)
    cos, sin = rope_tables(D, S, 1e6, yarn)
    o = gpu_attention(q.to(DEV), k.to(DEV), v.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6,
                      cos.to(DEV), sin.to(DEV))
    n = 1024
    gen = torch.Generator().manual_seed(1005)
    starts = [0, S - n] + sorted(torch.randint(n, S - 2 * n, (6,), generator=gen).tolist())
    # the device reference against the CPU oracle: 64 rows inside a random block, kv head 1
    r0 = starts[2] + 300
    dev_ref = _fp32_blocks_on_device(q, k, v, qw, kw, cos, sin, 1, G, [r0], 64)[0].cpu()
    cpu_ref = _sampled_blocks(q, k, v, qw, kw, cos, sin, 0, 1, G, [(r0, r0 + 64)])[0][0]
    torch.testing.assert_close(dev_ref, cpu_ref, rtol=1e-3, atol=1e-5)
    worst_rel = 0.0
    for kvh in range(Hkv):
        refs = _fp32_blocks_on_device(q, k, v, qw, kw, cos, sin, kvh, G, starts, n)
        for r0, ref in zip(starts, refs):
            got = o[0, kvh * G:(kvh + 1) * G, r0:r0 + n].float()
            assert_bf16_close(got, ref, f"yarn kvh={kvh} rows={r0}")
            rel = float((got - ref).norm() / ref.norm())
            assert rel <= 1e-2, f"yarn kvh={kvh} rows={r0}: relative error {rel:.3e}"
            worst_rel = max(worst_rel, rel)
    say(f"prefill YaRN B1 S131072: worst relative (Frobenius) error {worst_rel:.3e} over "
        f"{len(starts)} blocks x {Hq} heads")


@pytest.mark.parametrize("D,Hq,Hkv,B,S", [(64, 16, 16, 16, 2048), (128, 128, 8, 2, 4096)])
def test_wide_workgroups(D, Hq, Hkv, B, S):
    """Launches with at least 2048 workgroups of 256 rows run the 8-wave kernel
    (D=64 with G=1, D=128 with G=16); oracle on sampled 128-row blocks."""
    say(f"prefill 8-wave workgroups D={D} G={Hq // Hkv}")
    G = Hq // Hkv
    q, k, v, qw, kw = make(B, S, Hq, Hkv, D, torch.bfloat16, seed=1010 + D)
    cos, sin = rope_tables(D, S, 1e6)
    o = gpu_attention(q.to(DEV), k.to(DEV), v.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6,
                      cos.to(DEV), sin.to(DEV)).cpu()
    rows = [(0, 128), (S // 2 + 40, S // 2 + 168), (S - 128, S)]
    for b, kvh in ((0, 0), (B - 1, Hkv - 1)):
        for (r0, r1), ref in zip(rows, _sampled_blocks(q, k, v, qw, kw, cos, sin, b, kvh, G, rows)):
            assert_bf16_close(o[b:b + 1, kvh * G:(kvh + 1) * G, r0:r1], ref, f"wide b={b} kvh={kvh} rows={r0}")


def test_staged_tables_match_per_token_positions_at_8_waves():
    """At an 8-wave shape (>= 2048 workgroups of 64 positions x 4 heads), the cos/sin rows
    staged in LDS for per-sequence position bases, or for a uniform offset, give the same
    output bits as explicit per-token positions (per-lane table loads): same table
    entries, same arithmetic.  Key lengths (read through the scalar path) are exercised
    alongside: a padded batch row gives the same bits either way too."""
    say("prefill staged tables vs per-token positions, 8 waves")
    B, S, Hq, Hkv, D = 8, 4096, 16, 4, 128
    cos, sin = rope_tables(D, S + 64, 1e6)
    cos, sin = cos.to(DEV), sin.to(DEV)
    q = torch.randn(B, S, Hq, D, device=DEV, generator=torch.Generator(DEV).manual_seed(41),
                    dtype=torch.bfloat16).transpose(1, 2)
    k = torch.randn(B, S, Hkv, D, device=DEV, generator=torch.Generator(DEV).manual_seed(42),
                    dtype=torch.bfloat16).transpose(1, 2)
    v = torch.randn(B, S, Hkv, D, device=DEV, generator=torch.Generator(DEV).manual_seed(43),
                    dtype=torch.bfloat16).transpose(1, 2)
    w = (1 + 0.02 * torch.randn(D, generator=torch.Generator().manual_seed(44))).to(DEV)
    base = torch.tensor([0, 7, 64, 3, 50, 1, 33, 12], dtype=torch.int32, device=DEV)
    lens = torch.tensor([S, S, S - 5, S, 1000, S, S, 17], dtype=torch.int32, device=DEV)
    ids = (base[:, None].long() + torch.arange(S, device=DEV)[None, :])
    kw = dict(q_weight=w, eps=1e-6, cos=cos, sin=sin, causal=False, return_lse=True, key_lens=lens)
    o_base, l_base = nq.attention_prefill(q, k, v, pos_base=base, **kw)
    o_ids, l_ids = nq.attention_prefill(q, k, v, position_ids=ids, **kw)
    assert torch.isfinite(o_base).all()
    assert torch.equal(o_base, o_ids) and torch.equal(l_base, l_ids), \
        f"max |diff| {(o_base.float() - o_ids.float()).abs().max().item():.3e}"
    kw["key_lens"] = None
    kw["causal"] = True
    o_off, _ = nq.attention_prefill(q, k, v, pos_offset=5, **kw)
    o_ids5, _ = nq.attention_prefill(q, k, v, position_ids=torch.arange(S, device=DEV)[None, :].expand(B, S) + 5,
                                     **kw)
    assert torch.equal(o_off, o_ids5), f"max |diff| {(o_off.float() - o_ids5.float()).abs().max().item():.3e}"
