"""Host-side checks of the paged cache: allocator, block table, argument errors (no GPU)."""

import pytest
import torch

import nano_qwen_amd as nq
from nano_qwen_amd import _lib


def _cache(B=3, num_pages=10, P=32, H=2, D=64, max_pages=None):
    c = nq.PagedKVCache(num_pages, page_size=P, max_pages_per_seq=max_pages)
    c._setup(B, H, D, torch.float32, "cpu")
    return c


def test_pages_are_mapped_as_sequences_grow():
    c = _cache()
    c._grow([1, 32, 33])
    pages = [list(p) for p in c._pages]
    assert [len(p) for p in pages] == [1, 1, 2]
    flat = sum(pages, [])
    assert len(set(flat)) == len(flat) == c.num_pages - c.free_pages
    for b, p in enumerate(pages):
        assert c.block_table[b, :len(p)].tolist() == p
    c._grow([64, 32, 33])  # only sequence 0 needs another page
    assert len(c._pages[0]) == 2 and c._pages[1] == pages[1] and c._pages[2] == pages[2]


def test_set_lengths_returns_tail_pages_and_free_drops_a_sequence():
    c = _cache()
    c._grow([96, 96, 10])
    c.host_lens = [96, 96, 10]
    before = c.free_pages
    c.set_lengths([40, 96, 10])
    assert len(c._pages[0]) == 2 and c.free_pages == before + 1
    assert c.lens.tolist() == [40, 96, 10] and c.seq_len == 96
    c.free(1)
    assert c._pages[1] == [] and c.host_lens == [40, 0, 10] and c.free_pages == before + 4
    with pytest.raises(ValueError):
        c.set_lengths([41, 0, 10])  # longer than held


def test_out_of_pages_and_per_sequence_limit():
    c = _cache(num_pages=3, max_pages=2)
    with pytest.raises(ValueError, match="max_pages_per_seq"):
        c._grow([65, 0, 0])
    c._grow([64, 32, 0])
    with pytest.raises(RuntimeError, match="out of pages"):
        c._grow([64, 32, 1])


def test_reused_pages_and_gather_layout():
    c = _cache(B=2, num_pages=6, P=32, H=2, D=64)
    c._grow([70, 5])
    c.host_lens = [70, 5]
    # fill the pages so that gather can be checked against the block table
    for b, pages in enumerate(c._pages):
        for j, pid in enumerate(pages):
            for h in range(2):
                rows = torch.arange(32, dtype=torch.float32) + 32 * j + 1000 * b + 100000 * h
                c.k_pool[pid, h] = rows[:, None].expand(32, 64)
                c.v_pool[pid, h] = -rows[:, None].expand(32, 64)
    k, v = c.gather(0)
    assert k.shape == (2, 70, 64)
    want = torch.arange(70, dtype=torch.float32)
    torch.testing.assert_close(k[0, :, 0], want, rtol=0, atol=0)
    torch.testing.assert_close(k[1, :, 0], want + 100000, rtol=0, atol=0)
    torch.testing.assert_close(v[0, :, 0], -want, rtol=0, atol=0)
    freed = list(c._pages[0])
    c.free(0)
    c._grow([40, 5])
    assert set(c._pages[0]) <= set(freed) | set(range(6))
    assert len(c._pages[0]) == 2


def test_page_size_must_be_a_multiple_of_32():
    with pytest.raises(ValueError):
        nq.PagedKVCache(8, page_size=48)


def test_reset_returns_everything():
    c = _cache()
    c._grow([100, 10, 3])
    c.reset()
    assert c.free_pages == c.num_pages and c.block_table is None and c.lens is None


def test_paged_argument_errors_need_no_gpu():
    """Every call below fails validation before any HIP call: the placeholder
    addresses are never dereferenced."""
    import ctypes
    lib = _lib.load()
    st = _lib.strides3((1024, 64 * 128, 128))
    s2 = (ctypes.c_int64 * 2)(1024, 128)
    fake = ctypes.c_void_p(4096)
    args = dict(q=fake, q_strides=s2, k_new=None, k_new_strides=None, v_new=None, v_new_strides=None,
                k_weight=None, k_pool=None, k_pool_strides=st, v_pool=None, v_pool_strides=st,
                block_table=None, bt_stride=4, page_size=64, lens=None, lens_out=None, o=fake,
                o_strides=s2, workspace=None, workspace_bytes=0, B=2, Hq=8, Hkv=2, D=128,
                max_len=256, chunk=0, dtype=0, q_weight=None, eps=1e-6, cos=None, sin=None,
                max_pos=0, q_pos=None, q_pos0=-1, sm_scale=0.0, stream=None)
    need = lib.nq_attn_decode_workspace_bytes(2, 8, 2, 128, 256, 0)

    def call(**kw):
        a = dict(args, **kw)
        return lib.nq_attn_decode_paged_fwd(*a.values())

    assert call(D=96) == _lib.NQ_ERR_UNSUPPORTED and b"head_dim" in lib.nq_last_error()
    assert call(Hkv=3) == _lib.NQ_ERR_INVALID and b"divisible" in lib.nq_last_error()
    assert call() == _lib.NQ_ERR_WORKSPACE
    ws = dict(workspace=fake, workspace_bytes=need)
    assert call(**ws) == _lib.NQ_ERR_INVALID and b"caches" in lib.nq_last_error()
    pools = dict(ws, k_pool=fake, v_pool=fake)
    assert call(**pools) == _lib.NQ_ERR_INVALID and b"block table" in lib.nq_last_error()
    full = dict(pools, block_table=fake, lens=fake)
    assert call(**full, page_size=48) == _lib.NQ_ERR_UNSUPPORTED and b"multiple of 32" in lib.nq_last_error()
    assert call(**full, bt_stride=3) == _lib.NQ_ERR_INVALID and b"bt_stride" in lib.nq_last_error()
    assert call(**full, k_new=fake, k_new_strides=s2) == _lib.NQ_ERR_INVALID  # v_new missing
    assert call(**full, lens_out=fake) == _lib.NQ_ERR_INVALID and b"lens_out" in lib.nq_last_error()
    assert call(**full, k_new=fake, k_new_strides=s2, v_new=fake, v_new_strides=s2,
                lens_out=fake) == _lib.NQ_ERR_INVALID and b"alias" in lib.nq_last_error()
    assert lib.nq_kv_append_paged(None, st, None, st, None, st, None, st, None, 0, 64, 1, 1, 2,
                                  128, 0, 0, None, 1e-6, None, None, 0, None, None, 0, None, 0,
                                  None) == _lib.NQ_ERR_INVALID
    assert b"block table" in lib.nq_last_error()


def test_paged_decode_refuses_cpu_tensors():
    q = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    pool = torch.zeros(4, 2, 64, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP device"):
        nq.attention_decode_paged(q, pool, pool, torch.zeros(2, 2, dtype=torch.int32),
                                  torch.ones(2, dtype=torch.int32), max_len=64)
