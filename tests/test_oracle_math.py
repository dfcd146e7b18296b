"""Pin the oracle with closed forms, invariants, brute force and the library routine.

None of these re-types the oracle's own formula: each check is a property the
mathematics fixes (and which a dropped term, wrong sign, wrong index or
transposed operand would break), a pure-Python fp64 brute force, or torch's
SDPA, the routine the reference itself calls (model/attention.py:110-115).
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import (attention, attention_path, decode_path, reference_chunk_sdpa, reference_decode_sdpa,
                    reference_path_sdpa,
                    rms_norm, rope_inv_freq, rope_tables, rotate_half, yarn_correction_range,
                    yarn_inv_freq)


def _rand(*shape, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


# ---------------------------------------------------------------- RMSNorm

def test_rmsnorm_unit_rms_and_scale_invariance():
    x = _rand(5, 7, 128, seed=1)
    y = rms_norm(x, None, eps=0.0, compute_dtype=torch.float64)
    rms = y.pow(2).mean(-1).sqrt()
    torch.testing.assert_close(rms, torch.ones_like(rms), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(rms_norm(3.7 * x, None, 0.0, torch.float64), y, rtol=1e-12, atol=1e-12)
    # the weight multiplies per column after normalisation
    w = _rand(128, seed=2)
    torch.testing.assert_close(rms_norm(x, w, 0.0, torch.float64), y * w, rtol=1e-12, atol=1e-12)
    # eps enters under the root: a zero row stays finite and zero
    z = rms_norm(torch.zeros(1, 8, dtype=torch.float64), None, 1e-6, torch.float64)
    assert torch.all(z == 0)


# ---------------------------------------------------------------- RoPE / YaRN

def test_yarn_correction_range_closed_form():
    # D=128, theta=1e6, L0=32768: raw correction dims 23.60 (beta_fast=32) and
    # 39.65 (beta_slow=1), so low=23, high=40.
    assert yarn_correction_range(128, 1e6, 32768) == (23, 40)
    # Meaning of the range, checked from the rotation counts themselves:
    # pair i turns L0*inv_freq_i/(2*pi) times over the original context.
    inv = rope_inv_freq(128, 1e6).double()
    rot = 32768 * inv / (2 * math.pi)
    low, high = 23, 40
    assert rot[low] >= 32 > rot[low + 1]
    assert rot[high - 1] > 1 >= rot[high]


def test_yarn_blend_endpoints_and_identity():
    plain = rope_inv_freq(128, 1e6)
    yarn = yarn_inv_freq(128, 1e6, 4.0, 32768)
    low, high = 23, 40
    # fully extrapolated (original) frequencies below the ramp ...
    torch.testing.assert_close(yarn[:low + 1], plain[:low + 1], rtol=0, atol=0)
    # ... fully interpolated (divided by the factor) above it
    torch.testing.assert_close(yarn[high:], plain[high:] / 4.0, rtol=2e-7, atol=0)
    # strictly between: a convex blend, monotone in the ramp
    mid = slice(low + 1, high)
    lam = (yarn[mid] - plain[mid] / 4) / (plain[mid] - plain[mid] / 4)
    assert torch.all(lam > 0) and torch.all(lam < 1)
    assert torch.all(lam[1:] < lam[:-1])
    # factor 1 reproduces plain RoPE
    torch.testing.assert_close(yarn_inv_freq(128, 1e6, 1.0, 32768), plain, rtol=1e-7, atol=0)


def test_rope_position_zero_is_identity_and_norm_preserving():
    cos, sin = rope_tables(128, 64, 1e6)
    x = _rand(3, 64, 128, seed=3, dtype=torch.float32)
    y0 = rotate_half(x[:, :1], cos[:1], sin[:1])
    torch.testing.assert_close(y0, x[:, :1], rtol=0, atol=0)
    y = rotate_half(x, cos, sin)
    pair_in = x[..., :64] ** 2 + x[..., 64:] ** 2
    pair_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    torch.testing.assert_close(pair_out, pair_in, rtol=1e-5, atol=1e-5)


def test_rope_relative_position_property():
    # <R_m q, R_n k> depends only on m - n (fp64 tables from the fp64 angles)
    D = 64
    inv = rope_inv_freq(D, 1e4).double()
    ang = torch.arange(40, dtype=torch.float64)[:, None] * inv[None]
    cos, sin = ang.cos(), ang.sin()
    q, k = _rand(D, seed=4), _rand(D, seed=5)

    def dot(m, n):
        return float(rotate_half(q, cos[m], sin[m]) @ rotate_half(k, cos[n], sin[n]))

    assert dot(7, 3) == pytest.approx(dot(30, 26), rel=1e-12, abs=1e-12)
    assert dot(3, 7) == pytest.approx(dot(20, 24), rel=1e-12, abs=1e-12)
    assert dot(5, 5) == pytest.approx(float(q @ k), rel=1e-12, abs=1e-12)


def test_rope_d2_is_textbook_rotation():
    th = 0.7
    x = torch.tensor([0.3, -1.1], dtype=torch.float64)
    y = rotate_half(x, torch.tensor([math.cos(th)], dtype=torch.float64),
                    torch.tensor([math.sin(th)], dtype=torch.float64))
    R = torch.tensor([[math.cos(th), -math.sin(th)], [math.sin(th), math.cos(th)]], dtype=torch.float64)
    torch.testing.assert_close(y, R @ x, rtol=1e-15, atol=1e-15)


# ---------------------------------------------------------------- attention

def _brute(q, k, v, causal, offset=0, mask=None, scale=None):
    """Pure-Python fp64 loops: softmax over keys of scaled dot products."""
    B, Hq, S, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    sc = scale if scale is not None else 1.0 / math.sqrt(D)
    out = torch.zeros(B, Hq, S, D, dtype=torch.float64)
    for b in range(B):
        for h in range(Hq):
            kh = h // G
            for i in range(S):
                logits = []
                for j in range(T):
                    keep = (not causal) or j <= i + offset
                    if mask is not None:
                        keep = keep and bool(mask[b, 0, i, j])
                    if keep:
                        s = sum(float(q[b, h, i, d]) * float(k[b, kh, j, d]) for d in range(D)) * sc
                        logits.append((j, s))
                mx = max(s for _, s in logits)
                ws = [(j, math.exp(s - mx)) for j, s in logits]
                tot = sum(w for _, w in ws)
                for d in range(D):
                    out[b, h, i, d] = sum(w * float(v[b, kh, j, d]) for j, w in ws) / tot
    return out


@pytest.mark.parametrize("causal,S,T,offset", [(True, 5, 5, 0), (False, 3, 6, 0), (True, 3, 6, 3)])
def test_attention_matches_bruteforce(causal, S, T, offset):
    q, k, v = _rand(2, 4, S, 4, seed=6), _rand(2, 2, T, 4, seed=7), _rand(2, 2, T, 4, seed=8)
    got = attention(q, k, v, causal=causal, causal_offset=offset, compute_dtype=torch.float64)
    torch.testing.assert_close(got, _brute(q, k, v, causal, offset), rtol=1e-12, atol=1e-12)


def test_attention_mask_matches_bruteforce():
    q, k, v = _rand(1, 2, 4, 4, seed=9), _rand(1, 1, 4, 4, seed=10), _rand(1, 1, 4, 4, seed=11)
    mask = torch.tensor([[1, 0, 1, 1], [0, 1, 0, 0], [1, 1, 1, 0], [0, 0, 1, 1]], dtype=torch.bool)[None, None]
    got = attention(q, k, v, mask=mask, compute_dtype=torch.float64)
    torch.testing.assert_close(got, _brute(q, k, v, False, mask=mask), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_matches_sdpa_gqa(causal):
    q, k, v = _rand(2, 8, 33, 16, seed=12), _rand(2, 2, 33, 16, seed=13), _rand(2, 2, 33, 16, seed=14)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1),
                                         is_causal=causal)
    got = attention(q, k, v, causal=causal, compute_dtype=torch.float64, q_block=7)
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)


def test_attention_special_cases():
    # a single key returns that value row for every query
    q, k, v = _rand(1, 2, 3, 8, seed=15), _rand(1, 1, 1, 8, seed=16), _rand(1, 1, 1, 8, seed=17)
    torch.testing.assert_close(attention(q, k, v, compute_dtype=torch.float64),
                               v.expand(1, 2, 3, 8), rtol=1e-14, atol=1e-14)
    # zero queries -> uniform weights -> causal prefix mean of V
    T = 6
    q0 = torch.zeros(1, 2, T, 8, dtype=torch.float64)
    k, v = _rand(1, 1, T, 8, seed=18), _rand(1, 1, T, 8, seed=19)
    got = attention(q0, k, v, causal=True, compute_dtype=torch.float64)
    prefix = v[0, 0].cumsum(0) / torch.arange(1, T + 1, dtype=torch.float64)[:, None]
    torch.testing.assert_close(got[0, 0], prefix, rtol=1e-13, atol=1e-13)
    torch.testing.assert_close(got[0, 1], prefix, rtol=1e-13, atol=1e-13)
    # causal row 0 sees only key 0
    q = _rand(1, 2, T, 8, seed=20)
    torch.testing.assert_close(attention(q, k, v, causal=True, compute_dtype=torch.float64)[0, :, 0],
                               v[0, 0, 0].expand(2, 8), rtol=1e-14, atol=1e-14)


def test_gqa_head_mapping_is_h_div_G():
    # query head h must read kv head h // G (attention.py:106-108)
    q, k, v = _rand(1, 6, 4, 8, seed=21), _rand(1, 3, 4, 8, seed=22), _rand(1, 3, 4, 8, seed=23)
    full = attention(q, k, v, compute_dtype=torch.float64)
    for h in range(6):
        one = attention(q[:, h:h + 1], k[:, h // 2:h // 2 + 1], v[:, h // 2:h // 2 + 1],
                        compute_dtype=torch.float64)
        torch.testing.assert_close(full[:, h:h + 1], one, rtol=1e-14, atol=1e-14)


# ---------------------------------------------------------------- decode

def test_decode_equals_last_row_of_causal_prefill():
    B, Hq, Hkv, D, T = 3, 8, 2, 32, 21
    q, k, v = _rand(B, Hq, T, D, seed=24), _rand(B, Hkv, T, D, seed=25), _rand(B, Hkv, T, D, seed=26)
    qw, kw = 1 + 0.1 * _rand(D, seed=27), 1 + 0.1 * _rand(D, seed=28)
    cos, sin = rope_tables(D, 64, 1e6)
    pos = torch.arange(T)
    o, kh = attention_path(q, k, v, q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin,
                           q_pos=pos, causal=True, compute_dtype=torch.float64, return_khat=True)
    lens = torch.full((B,), T, dtype=torch.int32)
    od = decode_path(q[:, :, -1], kh, v, lens, q_weight=qw, eps=1e-6, cos=cos, sin=sin,
                     q_pos=torch.full((B,), T - 1), compute_dtype=torch.float64)
    torch.testing.assert_close(od, o[:, :, -1], rtol=1e-12, atol=1e-12)


def test_decode_ragged_rows_equal_their_slices():
    B, Hq, Hkv, D, Tcap = 3, 4, 1, 16, 12
    q = _rand(B, Hq, D, seed=29)
    kc, vc = _rand(B, Hkv, Tcap, D, seed=30), _rand(B, Hkv, Tcap, D, seed=31)
    lens = torch.tensor([5, 12, 1], dtype=torch.int32)
    cos, sin = rope_tables(D, 32, 1e6)
    qpos = lens.long() - 1
    full = decode_path(q, kc, vc, lens, q_weight=None, eps=1e-6, cos=cos, sin=sin, q_pos=qpos,
                       compute_dtype=torch.float64)
    # poison the unused rows: the result must not change
    kc2, vc2 = kc.clone(), vc.clone()
    for b in range(B):
        kc2[b, :, lens[b]:] = float("nan")
        vc2[b, :, lens[b]:] = float("nan")
    again = decode_path(q, kc2, vc2, lens, q_weight=None, eps=1e-6, cos=cos, sin=sin, q_pos=qpos,
                        compute_dtype=torch.float64)
    torch.testing.assert_close(again, full, rtol=0, atol=0)
    # length-1 row returns V[0] for every head
    torch.testing.assert_close(full[2], vc[2, 0, 0].expand(Hq, D), rtol=1e-14, atol=1e-14)


# ---------------------------------------------------------------- the CPU baseline's routine

@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("S,T", [(37, 37), (9, 40)])
def test_reference_path_sdpa_equals_attention_path(causal, S, T):
    """The timed CPU baseline (QK-Norm -> RoPE -> repeat_interleave -> SDPA) computes
    the same function as the golden-pinned attention_path, including bottom-right
    causal alignment when the queries are the last S of T positions."""
    B, Hq, Hkv, D = 2, 8, 2, 32
    q, k, v = _rand(B, Hq, S, D, seed=61), _rand(B, Hkv, T, D, seed=62), _rand(B, Hkv, T, D, seed=63)
    qw, kw = 1 + 0.1 * _rand(D, seed=64), 1 + 0.1 * _rand(D, seed=65)
    cos, sin = rope_tables(D, 64, 1e6)
    cos, sin = cos.double(), sin.double()
    qpos, kpos = torch.arange(T - S, T), torch.arange(T)
    got = reference_path_sdpa(q, k, v, q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin,
                              q_pos=qpos, k_pos=kpos, causal=causal)
    ref = attention_path(q, k, v, q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin, q_pos=qpos,
                         k_pos=kpos, causal=causal, causal_offset=T - S if causal else 0,
                         compute_dtype=torch.float64)
    # QK-Norm upcasts to fp32 as the reference does (norm.py:20), so fp64 inputs
    # differ from the fp64 oracle by fp32 rounding (~3e-7); a wrong term is O(0.1)
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-6)
    # the first query of a causal S < T block still sees T - S + 1 keys, not one
    if causal and S < T:
        one = reference_path_sdpa(q, k[:, :, :1], v[:, :, :1], q_weight=qw, k_weight=kw, eps=1e-6,
                                  cos=cos, sin=sin, q_pos=qpos[:1], k_pos=kpos[:1], causal=True)
        assert not torch.allclose(got[:, :, :1], one[:, :, :1])


def test_reference_decode_sdpa_equals_decode_path():
    """The decode CPU baseline's step (norm + RoPE of the new token, cache concatenation,
    repeat_interleave, SDPA) equals decode_path over the grown cache, and the row it
    appends is attention_path's k-hat at that position."""
    Hq, Hkv, D, T = 8, 2, 32, 23
    q, kn, vn = _rand(1, Hq, 1, D, seed=71), _rand(1, Hkv, 1, D, seed=72), _rand(1, Hkv, 1, D, seed=73)
    kc, vc = _rand(1, Hkv, T - 1, D, seed=74), _rand(1, Hkv, T - 1, D, seed=75)
    qw, kw = 1 + 0.1 * _rand(D, seed=76), 1 + 0.1 * _rand(D, seed=77)
    cos, sin = rope_tables(D, 64, 1e6)
    cos, sin = cos.double(), sin.double()
    o, k_all, v_all = reference_decode_sdpa(q, kn, vn, kc, vc, q_weight=qw, k_weight=kw, eps=1e-6,
                                            cos=cos, sin=sin)
    assert k_all.shape == (1, Hkv, T, D)
    torch.testing.assert_close(k_all[:, :, :T - 1], kc, rtol=0, atol=0)
    torch.testing.assert_close(v_all[:, :, -1:], vn, rtol=0, atol=0)
    _, kh = attention_path(q, kn, vn, q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin,
                           q_pos=torch.tensor([T - 1]), causal=False, compute_dtype=torch.float64,
                           return_khat=True)
    # fp32 QK-Norm as in the reference (norm.py:20): fp32 rounding, a wrong term is O(0.1)
    torch.testing.assert_close(k_all[:, :, -1:], kh, rtol=1e-5, atol=1e-6)
    ref = decode_path(q[:, :, 0], k_all, v_all, torch.tensor([T], dtype=torch.int32), q_weight=qw,
                      eps=1e-6, cos=cos, sin=sin, q_pos=torch.tensor([T - 1]),
                      compute_dtype=torch.float64)
    torch.testing.assert_close(o[:, :, 0], ref, rtol=1e-5, atol=1e-6)
    og, _, _ = reference_decode_sdpa(q, kn, vn, kc, vc, q_weight=qw, k_weight=kw, eps=1e-6, cos=cos,
                                     sin=sin, repeat_kv=False)
    torch.testing.assert_close(og, o, rtol=1e-12, atol=1e-12)


def test_reference_chunk_sdpa_equals_attention_path():
    """The chunked-prefill CPU baseline (norm + RoPE of the chunk, concatenation after the
    cached K-hat, repeat_interleave, SDPA with the bottom-right mask) equals attention_path
    over the whole sequence at the chunk's rows; a top-left mask (a plausible slip) does not."""
    Hq, Hkv, D, T0, S = 8, 2, 32, 19, 7
    q = _rand(1, Hq, T0 + S, D, seed=81)
    k, v = _rand(1, Hkv, T0 + S, D, seed=82), _rand(1, Hkv, T0 + S, D, seed=83)
    qw, kw = 1 + 0.1 * _rand(D, seed=84), 1 + 0.1 * _rand(D, seed=85)
    cos, sin = rope_tables(D, 64, 1e6)
    cos, sin = cos.double(), sin.double()
    full, kh = attention_path(q, k, v, q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin,
                              q_pos=torch.arange(T0 + S), causal=True, compute_dtype=torch.float64,
                              return_khat=True)
    o = reference_chunk_sdpa(q[:, :, T0:], k[:, :, T0:], v[:, :, T0:], kh[:, :, :T0], v[:, :, :T0],
                             q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin)
    torch.testing.assert_close(o, full[:, :, T0:], rtol=1e-5, atol=1e-6)
    kw_args = dict(q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin, q_pos=torch.arange(T0, T0 + S),
                   k_pos=torch.arange(T0 + S), causal=True, compute_dtype=torch.float64)
    br = attention_path(q[:, :, T0:], k, v, causal_offset=T0, **kw_args)  # bottom-right frontier
    torch.testing.assert_close(o, br, rtol=1e-5, atol=1e-6)
    tl = attention_path(q[:, :, T0:], k, v, causal_offset=0, **kw_args)  # top-left frontier
    assert not torch.allclose(tl, o, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("kind", ["bool", "float"])
def test_attention_masks_against_sdpa(kind):
    """The oracle's attn_mask handling (model/attention.py:110-113) against torch's SDPA,
    the library routine the reference calls: a bool keep-mask or an additive float mask,
    broadcast over heads, with rows whose keys are all masked (SDPA returns zeros there),
    in GQA form against SDPA over the repeat_interleave'd heads."""
    import torch.nn.functional as F
    B, Hq, Hkv, S, T, D = 2, 4, 2, 9, 13, 16
    q, k, v = _rand(B, Hq, S, D, seed=91), _rand(B, Hkv, T, D, seed=92), _rand(B, Hkv, T, D, seed=93)
    g = torch.Generator().manual_seed(94)
    keep = torch.rand(B, 1, S, T, generator=g) > 0.4
    keep[0, 0, 3] = False            # a fully masked row
    keep[1, 0, :, 0] = False
    if kind == "bool":
        mask = keep
    else:
        mask = torch.zeros(B, 1, S, T, dtype=torch.float64).masked_fill(~keep, float("-inf"))
        mask = mask + 0.3 * torch.randn(B, 1, S, T, generator=g, dtype=torch.float64)
    got = attention(q, k, v, mask=mask, compute_dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), attn_mask=mask)
    torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-10)
    assert not got[0, :, 3].abs().any()
