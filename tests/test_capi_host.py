"""CPU-side checks of the boundary: C-ABI exports, host logic, no-CPU-path guarantees."""

import ctypes
import os
import re

import pytest
import torch

import nano_qwen_amd as nq
from nano_qwen_amd import _lib
from nano_qwen_amd.config import AttentionConfig
from tests.conftest import ROOT


def _header_functions():
    text = open(os.path.join(ROOT, "include", "nq_attn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nq_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert _header_functions() == sorted(_lib.SIGNATURES)


def test_library_loads_and_exports_every_header_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libnqattn.so is not built (run python -m nano_qwen_amd.build)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _header_functions():
        assert hasattr(lib, name), name
    loaded = _lib.load()
    assert loaded.nq_version() == 100
    # a call with no jobs succeeds without touching the GPU and clears the error text
    st = _lib.strides3((0, 0, 0))
    assert loaded.nq_qk_norm_rope(None, st, None, st, None, st, None, st, None, st, None, st,
                                  1, 1, 1, 1, 128, 0, 0, None, None, 1e-6, None, None, 0,
                                  None, None, 0, None, 0, None) == _lib.NQ_OK
    assert loaded.nq_last_error() == b""


def test_argument_errors_need_no_gpu():
    """Validation happens before any HIP call, so it is testable on the CPU."""
    lib = _lib.load()
    st = _lib.strides3((0, 0, 0))
    rc = lib.nq_attn_prefill_fwd(None, st, None, st, None, st, None, st, None, None,
                                 1, 8, 2, 4, 4, 96, 0, None, 1e-6, None, None, 0,
                                 None, None, 0, 1, 0.0, None)
    assert rc == _lib.NQ_ERR_UNSUPPORTED and b"head_dim" in lib.nq_last_error()
    rc = lib.nq_attn_prefill_fwd(None, st, None, st, None, st, None, st, None, None,
                                 1, 8, 3, 4, 4, 128, 0, None, 1e-6, None, None, 0,
                                 None, None, 0, 1, 0.0, None)
    assert rc == _lib.NQ_ERR_INVALID and b"divisible" in lib.nq_last_error()
    rc = lib.nq_attn_prefill_fwd(None, st, None, st, None, st, None, st, None, None,
                                 1, 8, 2, 8, 4, 128, 0, None, 1e-6, None, None, 0,
                                 None, None, 0, 1, 0.0, None)
    assert rc == _lib.NQ_ERR_INVALID and b"S <= T" in lib.nq_last_error()
    # table rows are DMA'd to LDS in 16-byte pieces: a misaligned table is refused
    # (never dereferenced: the check precedes every launch)
    a, odd = ctypes.c_void_p(1 << 20), ctypes.c_void_p((1 << 20) + 4)
    rc = lib.nq_attn_prefill_fwd(a, st, a, st, a, st, a, st, None, None,
                                 1, 8, 2, 8, 8, 128, 0, None, 1e-6, odd, a, 16,
                                 None, None, 0, 1, 0.0, None)
    assert rc == _lib.NQ_ERR_INVALID and b"aligned" in lib.nq_last_error()
    # slots = waves + rows; a slot holds 16 heads x (D outputs + max + sum) in
    # fp32, and each row records its first and last covering wave (2 x int32)
    slot = 16 * 130 * 4
    assert lib.nq_attn_decode_workspace_bytes(64, 64, 4, 128, 32768, 0) == (1024 + 256) * slot + 256 * 8
    # chunk 1024 = 32 steps per wave over 64 x 4 rows of 1024 steps
    assert lib.nq_attn_decode_workspace_bytes(64, 64, 4, 128, 32768, 1024) == (8192 + 256) * slot + 256 * 8
    # G = 4 -> one head group per kv head; 4 rows x 32 steps / 32 = 4 waves
    assert lib.nq_attn_decode_workspace_bytes(2, 8, 2, 128, 1000, 1024) == (4 + 4) * slot + 4 * 8
    # G = 32 -> two head groups per kv head
    assert lib.nq_attn_decode_workspace_bytes(1, 32, 1, 128, 64, 32) == (4 + 2) * slot + 2 * 8
    assert lib.nq_attn_decode_workspace_bytes(2, 8, 3, 128, 1000, 0) == 0
    rc = lib.nq_attn_decode_fwd(None, None, None, st, None, st, None, None, None, None, 0,
                                2, 8, 2, 128, 5000, 1024, 0, None, 1e-6, None, None, 0,
                                None, -1, 0.0, None)
    assert rc == _lib.NQ_ERR_INVALID
    # the no-allocation decode reports an unsupported head_dim as the others do
    z = _lib.strides3((0, 0, 0))
    rc = lib.nq_attn_decode_paged_fwd_noalloc(
        None, z, None, None, None, None, None, None, z, None, z, None, 1, 32, None, None, None, z,
        2, 8, 2, 96, 64, 0, _lib.NQ_DTYPE_BF16, None, 1e-6, None, None, 0, None, -1, 0.0, None)
    assert rc == _lib.NQ_ERR_UNSUPPORTED and b"head_dim" in lib.nq_last_error()


def test_fp32_side_inputs_are_realigned():
    """Norm weights and tables handed to the kernels start on 16-byte boundaries:
    a contiguous fp32 view at an odd offset is copied, an aligned one passed as is."""
    from nano_qwen_amd.ops import _f32
    base = torch.arange(40, dtype=torch.float32)
    view = base[1:33]
    assert view.is_contiguous() and view.data_ptr() % 16
    out = _f32(view, base.device)
    assert out.data_ptr() % 16 == 0 and torch.equal(out, view)
    aligned = base[4:36]
    assert _f32(aligned, base.device).data_ptr() == aligned.data_ptr()


def test_cpu_tensors_are_refused():
    q = torch.zeros(1, 2, 4, 64)
    with pytest.raises(RuntimeError, match="HIP device"):
        nq.attention_prefill(q, q[:, :1], q[:, :1])
    cfg = AttentionConfig(hidden_size=128, num_attention_heads=2, num_key_value_heads=1,
                          head_dim=64, max_position_embeddings=64)
    with pytest.raises(RuntimeError, match="HIP devices only"):
        nq.Attention(cfg)(torch.zeros(1, 3, 128))


def test_state_dict_keys_match_reference_layout():
    cfg = AttentionConfig(hidden_size=256, num_attention_heads=8, num_key_value_heads=2,
                          max_position_embeddings=128)
    attn = nq.Attention(cfg)
    assert sorted(attn.state_dict()) == sorted([
        "q_proj.weight", "k_proj.weight", "v_proj.weight", "o_proj.weight",
        "q_norm.weight", "k_norm.weight"])
    assert attn.q_proj.weight.shape == (8 * 32, 256)
    assert attn.k_proj.weight.shape == (2 * 32, 256)
    assert attn.num_kv_groups == 4 and attn.head_dim == 32


def test_config_from_yaml_keeps_attention_fields(tmp_path):
    p = tmp_path / "m.yaml"
    p.write_text("hidden_size: 4096\nnum_hidden_layers: 94\nnum_attention_heads: 64\n"
                 "num_key_value_heads: 4\nhead_dim: 128\nmax_position_embeddings: 131072\n"
                 "rope_theta: 1000000.0\nnum_experts: 128\n")
    cfg = AttentionConfig.from_yaml(p)
    assert (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) == (64, 4, 128)
    assert cfg.num_kv_groups == 16 and cfg.rope_theta == 1e6
    assert AttentionConfig(hidden_size=2048, num_attention_heads=16).head_dim == 128


def test_rope_tables_match_reference_rows():
    import numpy as np
    from tests.conftest import GOLDEN
    fr = np.load(os.path.join(GOLDEN, "rope_tables.npz"), allow_pickle=False)
    rows = torch.from_numpy(fr["rows"])
    rope = nq.RotaryEmbedding(128, 131072, 1e6, {"type": "yarn", "factor": 4.0,
                                                 "original_max_position_embeddings": 32768})
    np.testing.assert_array_equal(rope.cos_cached[rows].numpy(), fr["yarn128_cos"])
    np.testing.assert_array_equal(rope.sin_cached[rows].numpy(), fr["yarn128_sin"])
    cos, sin = nq.build_tables(128, 131072, 1e6)
    np.testing.assert_array_equal(cos[rows].numpy(), fr["plain128_cos"])
    np.testing.assert_array_equal(sin[rows].numpy(), fr["plain128_sin"])


def test_kvcache_host_semantics_match_concatenation():
    """update() on host tensors behaves like the reference's torch.cat cache."""
    g = torch.Generator().manual_seed(0)
    cache = nq.KVCache()
    ks, vs = [], []
    for S in (5, 1, 1, 70, 1):
        k = torch.randn(2, 3, S, 64, generator=g)
        v = torch.randn(2, 3, S, 64, generator=g)
        ks.append(k), vs.append(v)
        K, V = cache.update(k, v)
        torch.testing.assert_close(K, torch.cat(ks, 2), rtol=0, atol=0)
        torch.testing.assert_close(V, torch.cat(vs, 2), rtol=0, atol=0)
    assert cache.seq_len == 78 and cache.capacity >= 78
    cache.reset()
    assert cache.seq_len == 0 and cache.key.shape[2] == 0


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with a message before any GPU work."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""
