"""GPU parity of the paged cache and of the decode with the K/V append fused in.

References:
  * the dense decode kernel (itself checked against the oracle) on the same
    keys: the paged kernel follows the same schedule and arithmetic, so the
    outputs must be bit-identical;
  * the unfused path (row-kernel append, then dense decode) for the fused
    append: identical cache rows, identical outputs;
  * the oracle decode on the keys gathered back from the pages.
Block tables are shuffled page permutations with unmapped pages left NaN, so a
wrong page or a read past a sequence's length shows up.
"""

import pytest
import torch

import nano_qwen_amd as nq
from nano_qwen_amd import ops
from oracle import attention, decode_path, rms_norm, rope_tables, rotate_half
from tests.helpers import assert_bf16_close, assert_close_for, randn, say

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _poison_tail(cache, lens):
    for b, L in enumerate(lens.tolist()):
        cache[b, :, L:] = float("nan")


def _pages(dense_k, dense_v, rows, P, seed, spare=3):
    """Scatter rows [0, rows[b]) of dense (B, H, T, D) caches into shuffled pages.

    Returns (k_pool, v_pool, block_table); pages that hold no row stay NaN.
    """
    B, H, T, D = dense_k.shape
    npg = [-(-int(r) // P) for r in rows]
    total = sum(npg) + spare
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(seed))
    kp = torch.full((total, H, P, D), float("nan"), dtype=dense_k.dtype)
    vp = torch.full((total, H, P, D), float("nan"), dtype=dense_k.dtype)
    bt = torch.zeros(B, max(npg) + 1, dtype=torch.int32)
    i = 0
    for b in range(B):
        for j in range(npg[b]):
            pid = int(perm[i])
            i += 1
            bt[b, j] = pid
            n = min(P, T - j * P)
            kp[pid, :, :n] = dense_k[b, :, j * P:j * P + n]
            vp[pid, :, :n] = dense_v[b, :, j * P:j * P + n]
    return kp, vp, bt


def _gather(pool, bt, b, n, P):
    """Rows [0, n) of sequence b back from the pages, (H, n, D)."""
    pages = [int(x) for x in bt[b, :-(-n // P)]]
    return torch.cat([pool[p] for p in pages], dim=1)[:, :n] if pages else pool[0, :, :0]


@pytest.mark.parametrize("D,P,dtype,chunk", [
    (128, 64, torch.bfloat16, 0), (128, 32, torch.bfloat16, 64), (64, 128, torch.bfloat16, 0),
    (128, 64, torch.float32, 0), (64, 32, torch.float32, 32)])
def test_paged_equals_dense(D, P, dtype, chunk):
    say(f"paged == dense D={D} P={P} {dtype} chunk={chunk}")
    B, Hq, Hkv, T = 5, 16, 2, 700
    lens = torch.tensor([700, 1, 0, 333, 64], dtype=torch.int32)
    q = randn(B, Hq, D, seed=201, dtype=dtype)
    kc = randn(B, Hkv, T, D, seed=202, dtype=dtype)
    vc = randn(B, Hkv, T, D, seed=203, dtype=dtype)
    _poison_tail(kc, lens), _poison_tail(vc, lens)
    kp, vp, bt = _pages(kc, vc, lens, P, seed=204)
    qw = 1 + 0.02 * randn(D, seed=205)
    cos, sin = (t.to(DEV) for t in rope_tables(D, 1024, 1e6))
    kw = dict(q_weight=qw.to(DEV), cos=cos, sin=sin, chunk=chunk)
    dense = nq.attention_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), max_len=T, **kw)
    paged = nq.attention_decode_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV), lens.to(DEV),
                                      max_len=T, **kw)
    torch.cuda.synchronize()
    assert torch.equal(paged, dense), float((paged.float() - dense.float()).abs().max())
    assert not paged[2].float().abs().any()  # no keys -> zeros


def test_paged_long_rows_cross_the_table_window():
    """125-page rows (P = 32): the in-register block-table window reloads."""
    say("paged long rows P=32")
    B, Hq, Hkv, D, T, P = 2, 8, 1, 128, 4000, 32
    lens = torch.tensor([4000, 2113], dtype=torch.int32)
    q = randn(B, Hq, D, seed=211, dtype=torch.bfloat16)
    kc = randn(B, Hkv, T, D, seed=212, dtype=torch.bfloat16)
    vc = randn(B, Hkv, T, D, seed=213, dtype=torch.bfloat16)
    _poison_tail(kc, lens), _poison_tail(vc, lens)
    kp, vp, bt = _pages(kc, vc, lens, P, seed=214)
    cos, sin = rope_tables(D, 4096, 1e6)
    for chunk in (0, 32, 4096):
        o = nq.attention_decode_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV), lens.to(DEV),
                                      max_len=T, cos=cos.to(DEV), sin=sin.to(DEV), chunk=chunk)
        d = nq.attention_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), max_len=T,
                                cos=cos.to(DEV), sin=sin.to(DEV), chunk=chunk)
        assert torch.equal(o, d), (chunk, float((o.float() - d.float()).abs().max()))
    ref = decode_path(q.float(), kc.float(), vc.float(), lens, q_weight=None, eps=1e-6, cos=cos,
                      sin=sin, q_pos=lens.long() - 1)
    assert_bf16_close(o, ref, "paged long rows vs oracle")


def _append_case(B, Hq, Hkv, D, T, lens, dtype, seed):
    q = randn(B, Hq, D, seed=seed, dtype=dtype)
    kn = randn(B, Hkv, D, seed=seed + 1, dtype=dtype)
    vn = randn(B, Hkv, D, seed=seed + 2, dtype=dtype)
    kc = randn(B, Hkv, T, D, seed=seed + 3, dtype=dtype)
    vc = randn(B, Hkv, T, D, seed=seed + 4, dtype=dtype)
    _poison_tail(kc, lens), _poison_tail(vc, lens)  # row lens[b] (the new one) too
    qw = 1 + 0.05 * randn(D, seed=seed + 5)
    kw = 1 + 0.05 * randn(D, seed=seed + 6)
    return q, kn, vn, kc, vc, qw, kw


def _oracle_append(q, kn, vn, kc, vc, lens, qw, kw, cos, sin, pos):
    """Oracle: K-Norm + RoPE of the new key at pos, appended at row lens[b], then decode."""
    kc, vc = kc.float().clone(), vc.float().clone()
    kh = rms_norm(kn.float(), kw, 1e-6)
    for b in range(kc.shape[0]):
        p = int(pos[b])
        kc[b, :, int(lens[b])] = rotate_half(kh[b], cos[p], sin[p])
        vc[b, :, int(lens[b])] = vn[b].float()
    return decode_path(q.float(), kc, vc, lens + 1, q_weight=qw, eps=1e-6, cos=cos, sin=sin,
                       q_pos=pos.long())


@pytest.mark.parametrize("G", [1, 8, 32])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_append_dense_layout(G, dtype):
    say(f"fused append dense G={G} {dtype}")
    B, Hkv, D, T = 4, 2, 128, 320
    Hq = G * Hkv
    lens = torch.tensor([0, 31, 32, 250], dtype=torch.int32)
    q, kn, vn, kc, vc, qw, kw = _append_case(B, Hq, Hkv, D, T, lens, dtype, seed=221)
    cos, sin = rope_tables(D, 512, 1e6)
    dv = lambda t: t.to(DEV)  # noqa: E731
    # unfused: row-kernel append, then the dense decode over lens + 1 keys
    k1, v1 = dv(kc), dv(vc)
    ops.qk_norm_rope(k=dv(kn)[:, :, None], v=dv(vn)[:, :, None], k_out=k1, v_out=v1, k_weight=dv(kw),
                     eps=1e-6, cos=dv(cos), sin=dv(sin), pos_base=dv(lens), kv_row_base=dv(lens))
    o1 = nq.attention_decode(dv(q), k1, v1, dv(lens + 1), max_len=T, q_weight=dv(qw), eps=1e-6,
                             cos=dv(cos), sin=dv(sin))
    # fused, through the identity block table
    k2, v2 = dv(kc), dv(vc)
    lens_d = dv(lens)
    lens_out = torch.full_like(lens_d, -7)
    ident = torch.arange(B, dtype=torch.int32, device=DEV).view(B, 1)
    o2 = nq.attention_decode_paged(dv(q), k2, v2, ident, lens_d, max_len=T, k_new=dv(kn), v_new=dv(vn),
                                   k_weight=dv(kw), lens_out=lens_out, q_weight=dv(qw), eps=1e-6,
                                   cos=dv(cos), sin=dv(sin))
    torch.cuda.synchronize()
    assert lens_out.tolist() == (lens + 1).tolist() and lens_d.tolist() == lens.tolist()
    assert torch.equal(k2.isnan(), k1.isnan()) and torch.equal(v2.isnan(), v1.isnan())
    assert torch.equal(k2.nan_to_num(), k1.nan_to_num()) and torch.equal(v2.nan_to_num(), v1.nan_to_num())
    assert torch.equal(o2, o1), float((o2.float() - o1.float()).abs().max())
    ref = _oracle_append(q, kn, vn, kc, vc, lens, qw, kw, cos, sin, lens)
    assert_close_for(dtype, o2, ref, "fused append vs oracle")


@pytest.mark.parametrize("P", [32, 128])
def test_fused_append_paged_with_positions(P):
    say(f"fused append paged P={P}")
    B, Hq, Hkv, D, T = 3, 64, 4, 128, 3000
    lens = torch.tensor([2999, 0, 1500], dtype=torch.int32)
    q, kn, vn, kc, vc, qw, kw = _append_case(B, Hq, Hkv, D, T, lens, torch.bfloat16, seed=231)
    kp, vp, bt = _pages(kc, vc, lens + 1, P, seed=232)
    cos, sin = rope_tables(D, 8192, 1e6)
    pos = torch.tensor([5000, 3, 1500], dtype=torch.int32)
    dv = lambda t: t.to(DEV)  # noqa: E731
    kpd, vpd, lens_d = dv(kp), dv(vp), dv(lens)
    lens_out = torch.empty_like(lens_d)
    o = nq.attention_decode_paged(dv(q), kpd, vpd, dv(bt), lens_d, max_len=T, k_new=dv(kn),
                                  v_new=dv(vn), k_weight=dv(kw), lens_out=lens_out, q_weight=dv(qw),
                                  eps=1e-6, cos=dv(cos), sin=dv(sin), q_pos=dv(pos))
    torch.cuda.synchronize()
    assert lens_out.tolist() == (lens + 1).tolist()
    ref = _oracle_append(q, kn, vn, kc, vc, lens, qw, kw, cos, sin, pos)
    assert_bf16_close(o, ref, "fused append paged vs oracle")
    # the appended rows in the pages are the row kernel's K-hat/V rows
    kref = torch.empty(B, Hkv, 1, D, dtype=torch.bfloat16, device=DEV)
    vref = torch.empty_like(kref)
    ops.qk_norm_rope(k=dv(kn)[:, :, None], v=dv(vn)[:, :, None], k_out=kref, v_out=vref,
                     k_weight=dv(kw), eps=1e-6, cos=dv(cos), sin=dv(sin),
                     position_ids=dv(pos)[:, None])
    kpc, vpc = kpd.cpu(), vpd.cpu()
    for b in range(B):
        n = int(lens[b]) + 1
        kg, vg = _gather(kpc, bt, b, n, P), _gather(vpc, bt, b, n, P)
        assert torch.equal(kg[:, -1], kref[b, :, 0].cpu())
        assert torch.equal(vg[:, -1], vref[b, :, 0].cpu())
        assert torch.equal(kg[:, :-1], kc[b, :, :n - 1]) and torch.equal(vg[:, :-1], vc[b, :, :n - 1])


def test_kv_append_paged_matches_dense_rows():
    say("kv_append_paged vs qk_norm_rope")
    B, Hkv, D, S, P = 3, 2, 128, 37, 32
    base = torch.tensor([0, 5, 64], dtype=torch.int32)
    k = randn(B, S, Hkv, D, seed=241, dtype=torch.bfloat16).transpose(1, 2)
    v = randn(B, S, Hkv, D, seed=242, dtype=torch.bfloat16).transpose(1, 2)
    kw = 1 + 0.05 * randn(D, seed=243)
    cos, sin = rope_tables(D, 256, 1e6)
    T = int((base + S).max())
    dense_k = torch.full((B, Hkv, T, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    dense_v = torch.full_like(dense_k, float("nan"))
    dv = lambda t: t.to(DEV)  # noqa: E731
    ops.qk_norm_rope(k=dv(k), v=dv(v), k_out=dense_k, v_out=dense_v, k_weight=dv(kw), eps=1e-6,
                     cos=dv(cos), sin=dv(sin), pos_base=dv(base), kv_row_base=dv(base))
    kp, vp, bt = _pages(dense_k.cpu(), dense_v.cpu(), base + S, P, seed=244)
    kp[:], vp[:] = float("nan"), float("nan")
    kpd, vpd = dv(kp), dv(vp)
    ops.kv_append_paged(dv(k), dv(v), kpd, vpd, dv(bt), k_weight=dv(kw), eps=1e-6, cos=dv(cos),
                        sin=dv(sin), pos_base=dv(base), row_base=dv(base))
    kpc, vpc, dk, dvv = kpd.cpu(), vpd.cpu(), dense_k.cpu(), dense_v.cpu()
    for b in range(B):
        lo, hi = int(base[b]), int(base[b]) + S
        assert torch.equal(_gather(kpc, bt, b, hi, P)[:, lo:], dk[b, :, lo:hi])
        assert torch.equal(_gather(vpc, bt, b, hi, P)[:, lo:], dvv[b, :, lo:hi])


def _module(hidden=512, H=8, Hkv=2, D=128, seed=251):
    cfg = nq.AttentionConfig(hidden_size=hidden, num_attention_heads=H, num_key_value_heads=Hkv,
                             head_dim=D, max_position_embeddings=4096)
    torch.manual_seed(seed)
    attn = nq.Attention(cfg)
    with torch.no_grad():
        attn.q_norm.weight.add_(0.05 * torch.randn(D))
        attn.k_norm.weight.add_(0.05 * torch.randn(D))
    attn = attn.to(DEV, torch.bfloat16).eval()
    attn.rope_positions, attn.cache_prefill_causal = "cache", True
    return attn


def test_module_paged_cache_equals_ragged_dense_cache():
    say("Attention with PagedKVCache vs ragged KVCache")
    attn = _module()
    B, S = 3, 20
    h = (0.5 * randn(B, S, 512, seed=252)).to(DEV, torch.bfloat16)
    dense, paged = nq.KVCache(), nq.PagedKVCache(num_pages=32, page_size=32)
    with torch.no_grad():
        od = attn(h, kv_cache=dense)
        op = attn(h, kv_cache=paged)
        torch.testing.assert_close(op.float(), od.float(), rtol=0, atol=1e-2)
        lens = torch.tensor([20, 7, 13], dtype=torch.int32)
        dense.set_lengths(lens.to(DEV))
        paged.set_lengths(lens)
        for t in range(45):  # crosses page boundaries at 32 and 64
            x = (0.5 * randn(B, 1, 512, seed=300 + t)).to(DEV, torch.bfloat16)
            od, op = attn(x, kv_cache=dense), attn(x, kv_cache=paged)
            assert torch.equal(op, od), (t, float((op.float() - od.float()).abs().max()))
    assert paged.host_lens == (lens + 45).tolist() and paged.lens.tolist() == paged.host_lens
    assert dense.lens.tolist() == paged.host_lens
    for b in range(B):
        k, v = paged.gather(b)
        n = paged.host_lens[b]
        assert torch.equal(k, dense.key[b, :, :n]) and torch.equal(v, dense.value[b, :, :n])


def test_module_paged_multi_token_continuation():
    """Prefill 40, then 17 more tokens at once, then one: equals the no-cache causal forward."""
    say("PagedKVCache chunked prefill")
    attn = _module(seed=261)
    B = 2
    h = (0.5 * randn(B, 58, 512, seed=262)).to(DEV, torch.bfloat16)
    cache = nq.PagedKVCache(num_pages=16, page_size=32)
    with torch.no_grad():
        full = attn(h)
        o1 = attn(h[:, :40], kv_cache=cache)
        o2 = attn(h[:, 40:57], kv_cache=cache)
        o3 = attn(h[:, 57:], kv_cache=cache)
    got = torch.cat([o1, o2, o3], dim=1).float()
    assert_bf16_close(got, full, "chunked prefill + decode vs one causal prefill",
                      max_abs=3e-2, mean_abs=3e-3)
    assert cache.host_lens == [58, 58]


def test_generate_greedy_batch_paged_equals_dense():
    from nano_qwen_amd import ModelConfig, Qwen3Model
    from tests.golden.make_golden_model import MODEL, make_model_weights
    say("generate_greedy_batch paged vs dense")
    torch.manual_seed(0)
    m = Qwen3Model(ModelConfig(**MODEL)).eval()
    m.load_state_dict(make_model_weights(), strict=True)
    m = m.to(DEV, torch.bfloat16)
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, MODEL["vocab_size"], (n,), generator=g).tolist() for n in (70, 3, 33, 1)]
    dense, _ = nq.generate_greedy_batch(m, prompts, 40)
    paged, _ = nq.generate_greedy_batch(m, prompts, 40, page_size=32)
    assert paged == dense


def test_fused_append_paged_full_size():
    """The 235B-like decode (B64, Hq64/Hkv4, D128, lengths U[1024, 32768]) on a pool of
    64-row pages dealt in a seeded random order, with the append fused: every row against
    the oracle, and every appended K-hat/V row equal to the row kernel's.  Rows past each
    sequence's keys, the appended row included, start as NaN."""
    say("fused append paged B64 64/4 T_cap 32768")
    B, Hq, Hkv, D, Tcap, P = 64, 64, 4, 128, 32768, 64
    g = torch.Generator().manual_seed(1003)
    lens = torch.randint(1024, Tcap + 1, (B,), generator=g, dtype=torch.int32)
    held = lens - 1                                   # keys before the new token
    npp = Tcap // P
    bt = torch.randperm(B * npp, generator=g).view(B, npp).to(torch.int32)
    gd = torch.Generator(device=DEV).manual_seed(1003)
    kp = torch.randn(B * npp, Hkv, P, D, generator=gd, device=DEV, dtype=torch.bfloat16)
    vp = torch.randn(B * npp, Hkv, P, D, generator=gd, device=DEV, dtype=torch.bfloat16)
    for b in range(B):
        h = int(held[b])
        j0 = h // P
        for pool in (kp, vp):
            pool[int(bt[b, j0]), :, h - j0 * P:] = float("nan")
            pool[bt[b, j0 + 1:].long().to(DEV)] = float("nan")
    q = randn(B, Hq, D, seed=1011, dtype=torch.bfloat16)
    kn = randn(B, Hkv, D, seed=1012, dtype=torch.bfloat16)
    vn = randn(B, Hkv, D, seed=1013, dtype=torch.bfloat16)
    qw = 1 + 0.02 * randn(D, seed=1014)
    kw = 1 + 0.02 * randn(D, seed=1015)
    cos, sin = rope_tables(D, Tcap, 1e6)
    dv = lambda t: t.to(DEV)  # noqa: E731
    lens_out = torch.empty(B, dtype=torch.int32, device=DEV)
    o = nq.attention_decode_paged(dv(q), kp, vp, dv(bt), dv(held), max_len=int(lens.max()),
                                  k_new=dv(kn), v_new=dv(vn), k_weight=dv(kw), lens_out=lens_out,
                                  q_weight=dv(qw), eps=1e-6, cos=dv(cos), sin=dv(sin)).cpu()
    assert lens_out.cpu().tolist() == lens.tolist()
    assert torch.isfinite(o.float()).all()
    # the row kernel's K-hat / V rows of the new tokens, at each sequence's query position
    kref = torch.empty(B, Hkv, 1, D, dtype=torch.bfloat16, device=DEV)
    vref = torch.empty_like(kref)
    ops.qk_norm_rope(k=dv(kn)[:, :, None], v=dv(vn)[:, :, None], k_out=kref, v_out=vref,
                     k_weight=dv(kw), eps=1e-6, cos=dv(cos), sin=dv(sin),
                     position_ids=dv(held)[:, None])
    for b in range(B):
        L = int(lens[b])
        ids = bt[b, :-(-L // P)].long().to(DEV)
        kd = kp[ids].permute(1, 0, 2, 3).reshape(Hkv, -1, D)[:, :L].cpu()
        vd = vp[ids].permute(1, 0, 2, 3).reshape(Hkv, -1, D)[:, :L].cpu()
        assert torch.equal(kd[:, L - 1], kref[b, :, 0].cpu()), f"appended K-hat row, b={b}"
        assert torch.equal(vd[:, L - 1], vref[b, :, 0].cpu()), f"appended V row, b={b}"
        ref = _oracle_append(q[b:b + 1], kn[b:b + 1], vn[b:b + 1], kd[None], vd[None], held[b:b + 1],
                             qw, kw, cos, sin, held[b:b + 1])
        assert_bf16_close(o[b:b + 1], ref, f"fused append paged b={b} len={L}")


def test_paged_chunked_prefill_full_size():
    """An 8B-like sequence set (B4 x 8192, 32/8 heads, D128) prefilled in four
    2048-token chunks into 64-row pages dealt in a seeded random order (unused
    pages NaN): each chunk appends its K-hat/V (norm and rotation fused) and its
    queries attend all keys so far through the block table.  Every chunk's
    output is bit-identical to the dense prefill over the same K-hat/V, and
    sampled query blocks match the oracle."""
    say("paged chunked prefill B4 x 8192 32/8 D128, 4 chunks of 2048, P64")
    B, Hq, Hkv, D, T, C, P = 4, 32, 8, 128, 8192, 2048, 64
    q = randn(B, T, Hq, D, seed=5101, dtype=torch.bfloat16).transpose(1, 2)
    k = randn(B, T, Hkv, D, seed=5102, dtype=torch.bfloat16).transpose(1, 2)
    v = randn(B, T, Hkv, D, seed=5103, dtype=torch.bfloat16).transpose(1, 2)
    qw = 1 + 0.02 * randn(D, seed=5104)
    kw = 1 + 0.02 * randn(D, seed=5105)
    cos, sin = rope_tables(D, T, 1e6)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    qwd, kwd, cd, sd = qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV)
    # dense K-hat of the whole sequence (the row kernel), for the dense reference launches
    khat = nq.qk_norm_rope(k=kd, k_weight=kwd, eps=1e-6, cos=cd, sin=sd)[1]
    npg = T // P
    total = B * npg + 5
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(5106)).to(torch.int32)
    bt = perm[:B * npg].view(B, npg).to(DEV)
    kp = torch.full((total, Hkv, P, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    vp = torch.full_like(kp, float("nan"))
    outs = []
    for c in range(T // C):
        p0 = c * C
        ops.kv_append_paged(kd[:, :, p0:p0 + C], vd[:, :, p0:p0 + C], kp, vp, bt, k_weight=kwd, eps=1e-6,
                            cos=cd, sin=sd, row_offset=p0, pos_offset=p0)
        got = ops.attention_prefill_paged(qd[:, :, p0:p0 + C], kp, vp, bt, T=p0 + C, q_weight=qwd, eps=1e-6,
                                          cos=cd, sin=sd, causal=True, pos_offset=p0)
        want = ops.attention_prefill(qd[:, :, p0:p0 + C], khat[:, :, :p0 + C], vd[:, :, :p0 + C], q_weight=qwd,
                                     eps=1e-6, cos=cd, sin=sd, causal=True, pos_offset=p0)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all(), f"chunk {c}"
        assert torch.equal(got, want), f"chunk {c}: paged differs from dense (max {float((got.float() - want.float()).abs().max()):.3e})"
        outs.append(got.float().cpu())
    # oracle on sampled 64-row query blocks (first chunk's first block, last chunk's first and last)
    kf = rms_norm(k.float(), kw, 1e-6)
    kh = rotate_half(kf, cos[None, None], sin[None, None])
    for c, s0 in ((0, 0), (3, 0), (3, C - 64)):
        p0 = c * C
        rows = torch.arange(p0 + s0, p0 + s0 + 64)
        qh = rotate_half(rms_norm(q[:, :, rows].float(), qw, 1e-6), cos[rows][None, None], sin[rows][None, None])
        ref = attention(qh, kh[:, :, :p0 + C], v[:, :, :p0 + C].float(), causal=True, causal_offset=p0 + s0)
        assert_bf16_close(outs[c][:, :, s0:s0 + 64], ref, f"chunk {c} rows {s0}..{s0 + 63} vs oracle")


@pytest.mark.parametrize("dtype,D,P,Hq,Hkv", [
    (torch.bfloat16, 128, 64, 8, 2), (torch.bfloat16, 128, 32, 16, 1), (torch.bfloat16, 64, 128, 4, 4),
    (torch.bfloat16, 32, 32, 8, 1), (torch.float32, 128, 64, 8, 2), (torch.float32, 64, 32, 4, 1)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_paged_equals_dense(dtype, D, P, Hq, Hkv, causal):
    """A chunk of S queries over T keys held in shuffled pages (T a multiple of neither
    64 nor the page size; unmapped pages NaN): bit-identical to the dense kernel over the
    same K-hat/V rows, and within the gate of the oracle."""
    say(f"paged prefill {dtype} D={D} P={P} {Hq}/{Hkv} causal={causal}")
    B, S, T = 3, 77, 213
    q = randn(B, Hq, S, D, seed=901, dtype=dtype)
    k = randn(B, Hkv, T, D, seed=902, dtype=dtype)
    v = randn(B, Hkv, T, D, seed=903, dtype=dtype)
    qw = 1 + 0.02 * randn(D, seed=904)
    cos, sin = rope_tables(D, 512, 1e6)
    kp, vp, bt = _pages(k, v, [T] * B, P, seed=905)
    kw = dict(q_weight=qw.to(DEV), eps=1e-6, cos=cos.to(DEV), sin=sin.to(DEV), causal=causal, pos_offset=T - S)
    got = ops.attention_prefill_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV), T=T, **kw)
    want = ops.attention_prefill(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, want), float((got.float() - want.float()).abs().max())
    rows = torch.arange(T - S, T)
    qh = rotate_half(rms_norm(q.float(), qw, 1e-6), cos[rows][None, None], sin[rows][None, None])
    ref = attention(qh, k.float(), v.float(), causal=causal, causal_offset=T - S)
    assert_close_for(dtype, got, ref, "paged prefill vs oracle")
