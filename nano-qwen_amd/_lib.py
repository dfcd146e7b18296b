"""ctypes binding of libnqattn.so, the C ABI declared in include/nq_attn.h.

The library is loaded lazily and only from this package's directory.  torch is
imported first so that the library's libamdhip64.so.7 dependency resolves to
the HIP runtime torch already loaded (one runtime per process).  There is no
fallback: if the library is missing, every call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnqattn.so")

NQ_OK = 0
NQ_ERR_INVALID = 1
NQ_ERR_UNSUPPORTED = 2
NQ_ERR_WORKSPACE = 3
NQ_DTYPE_BF16 = 0
NQ_DTYPE_F32 = 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/nq_attn.h
SIGNATURES = {
    "nq_version": (_i32, []),
    "nq_last_error": (ctypes.c_char_p, []),
    "nq_qk_norm_rope": (_i32, [
        _p, _i64p, _p, _i64p,          # q, q_strides, q_out, q_out_strides
        _p, _i64p, _p, _i64p,          # k ...
        _p, _i64p, _p, _i64p,          # v ...
        _i32, _i32, _i32, _i32, _i32,  # B, S, Hq, Hkv, D
        _i32, _i32,                    # dtype_in, dtype_out
        _p, _p, _f32,                  # q_weight, k_weight, eps
        _p, _p, _i32,                  # cos, sin, max_pos
        _p, _p, _i32,                  # pos, pos_base, pos0
        _p, _i32,                      # kv_row_base, kv_row0
        _p,                            # stream
    ]),
    "nq_rmsnorm": (_i32, [
        _p, _i64, _p, _p, _i64,                      # x, x_row_stride, weight, y, y_row_stride
        _i64, _i32, _i32, _i32, _i32,                # rows, width, dtype_x, dtype_w, dtype_y
        _f32, _p,                                    # eps, stream
    ]),
    "nq_attn_prefill_fwd": (_i32, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p,  # q, k, v, o (+ strides)
        _p, _p,                                      # lse, key_lens
        _i32, _i32, _i32, _i32, _i32, _i32, _i32,    # B, Hq, Hkv, S, T, D, dtype
        _p, _f32,                                    # q_weight, eps
        _p, _p, _i32,                                # cos, sin, max_pos
        _p, _p, _i32,                                # q_pos, q_pos_base, q_pos0
        _i32, _f32, _p,                              # causal, sm_scale, stream
    ]),
    "nq_attn_prefill_paged_fwd": (_i32, [
        _p, _i64p,                                   # q, q_strides
        _p, _i64p, _p, _i64p,                        # k_pool, v_pool (+ strides)
        _p, _i64, _i32,                              # block_table, bt_stride, page_size
        _p, _i64p, _p,                               # o, o_strides, lse
        _i32, _i32, _i32, _i32, _i32, _i32, _i32,    # B, Hq, Hkv, S, T, D, dtype
        _p, _f32,                                    # q_weight, eps
        _p, _p, _i32,                                # cos, sin, max_pos
        _p, _p, _i32,                                # q_pos, q_pos_base, q_pos0
        _i32, _f32, _p,                              # causal, sm_scale, stream
    ]),
    "nq_attn_prefill_bias_fwd": (_i32, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p,  # q, k, v, o (+ strides)
        _p, _p,                                      # lse, key_lens
        _p, _i64p,                                   # bias, bias_strides
        _i32, _i32, _i32, _i32, _i32, _i32, _i32,    # B, Hq, Hkv, S, T, D, dtype
        _p, _f32,                                    # q_weight, eps
        _p, _p, _i32,                                # cos, sin, max_pos
        _p, _p, _i32,                                # q_pos, q_pos_base, q_pos0
        _i32, _f32, _p,                              # causal, sm_scale, stream
    ]),
    "nq_attn_decode_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "nq_attn_decode_fwd": (_i32, [
        _p, _i64p, _p, _i64p, _p, _i64p,             # q, k_cache, v_cache (+ strides)
        _p, _p, _i64p,                               # lens, o, o_strides
        _p, _i64,                                    # workspace, workspace_bytes
        _i32, _i32, _i32, _i32, _i32, _i32, _i32,    # B, Hq, Hkv, D, max_len, chunk, dtype
        _p, _f32,                                    # q_weight, eps
        _p, _p, _i32,                                # cos, sin, max_pos
        _p, _i32, _f32, _p,                          # q_pos, q_pos0, sm_scale, stream
    ]),
    "nq_attn_decode_paged_fwd": (_i32, [
        _p, _i64p,                                   # q, q_strides
        _p, _i64p, _p, _i64p, _p,                    # k_new, v_new (+ strides), k_weight
        _p, _i64p, _p, _i64p,                        # k_pool, v_pool (+ strides)
        _p, _i64, _i32,                              # block_table, bt_stride, page_size
        _p, _p,                                      # lens, lens_out
        _p, _i64p, _p, _i64,                         # o, o_strides, workspace, workspace_bytes
        _i32, _i32, _i32, _i32, _i32, _i32, _i32,    # B, Hq, Hkv, D, max_len, chunk, dtype
        _p, _f32,                                    # q_weight, eps
        _p, _p, _i32,                                # cos, sin, max_pos
        _p, _i32, _f32, _p,                          # q_pos, q_pos0, sm_scale, stream
    ]),
    "nq_attn_decode_paged_fwd_noalloc": (_i32, [
        _p, _i64p,                                   # q, q_strides
        _p, _i64p, _p, _i64p, _p,                    # k_new, v_new (+ strides), k_weight
        _p, _i64p, _p, _i64p,                        # k_pool, v_pool (+ strides)
        _p, _i64, _i32,                              # block_table, bt_stride, page_size
        _p, _p,                                      # lens, lens_out
        _p, _i64p,                                   # o, o_strides
        _i32, _i32, _i32, _i32, _i32, _i32, _i32,    # B, Hq, Hkv, D, max_len, chunk, dtype
        _p, _f32,                                    # q_weight, eps
        _p, _p, _i32,                                # cos, sin, max_pos
        _p, _i32, _f32, _p,                          # q_pos, q_pos0, sm_scale, stream
    ]),
    "nq_kv_append_paged": (_i32, [
        _p, _i64p, _p, _i64p,                        # k, k_strides, v, v_strides
        _p, _i64p, _p, _i64p,                        # k_pool, v_pool (+ strides)
        _p, _i64, _i32,                              # block_table, bt_stride, page_size
        _i32, _i32, _i32, _i32,                      # B, S, Hkv, D
        _i32, _i32,                                  # dtype_in, dtype_out
        _p, _f32,                                    # k_weight, eps
        _p, _p, _i32,                                # cos, sin, max_pos
        _p, _p, _i32,                                # pos, pos_base, pos0
        _p, _i32,                                    # row_base, row0
        _p,                                          # stream
    ]),
    "nq_attn_merge": (_i32, [
        _p, _i64p, _p,                               # o, o_strides, lse
        _p, _i64p, _p,                               # o_part, part_strides, lse_part
        _i32, _i32, _i32, _i32, _i32,                # B, H, S, D, dtype
        _p,                                          # stream
    ]),
    "nq_attn_bwd_workspace_bytes": (_i64, [_i32, _i32, _i32]),
    "nq_attn_bwd": (_i32, [
        _p, _i64p, _p, _i64p, _p, _i64p,             # q, k, v (+ strides)
        _p, _i64p, _p, _i64p, _p, _p,                # o, dout (+ strides), lse, key_lens
        _p, _i64p, _p, _i64p, _p, _i64p,             # dq, dk, dv (+ strides)
        _p, _i64,                                    # workspace, workspace_bytes
        _i32, _i32, _i32, _i32, _i32, _i32, _i32,    # B, Hq, Hkv, S, T, D, dtype
        _i32, _f32, _p,                              # causal, sm_scale, stream
    ]),
    "nq_attn_bwd_bias": (_i32, [
        _p, _i64p, _p, _i64p, _p, _i64p,             # q, k, v (+ strides)
        _p, _i64p, _p, _i64p, _p, _p,                # o, dout (+ strides), lse, key_lens
        _p, _i64p, _p, _i64p,                        # bias, bias_strides, bias_t, bias_t_strides
        _p, _i64p, _p, _i64p, _p, _i64p,             # dq, dk, dv (+ strides)
        _p, _i64,                                    # workspace, workspace_bytes
        _i32, _i32, _i32, _i32, _i32, _i32, _i32,    # B, Hq, Hkv, S, T, D, dtype
        _i32, _f32, _p,                              # causal, sm_scale, stream
    ]),
    "nq_qk_norm_rope_bwd_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "nq_qk_norm_rope_bwd": (_i32, [
        _p, _i64p, _p, _i64p, _p, _i64p,             # x, dy, dx (+ strides)
        _p, _p, _p, _i64,                            # weight, dweight, workspace, workspace_bytes
        _i32, _i32, _i32, _i32, _i32,                # B, S, H, D, dtype
        _f32, _p, _p, _i32,                          # eps, cos, sin, max_pos
        _p, _p, _i32,                                # pos, pos_base, pos0
        _p,                                          # stream
    ]),
}

_lock = threading.Lock()
_lib = None


class NQError(RuntimeError):
    """A failed call into libnqattn.so (argument error or launch failure)."""


def load():
    """Load libnqattn.so (once) and bind its signatures; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise NQError(
                f"{LIB_PATH} is not built; run `python -m nano_qwen_amd.build` "
                "(the attention kernels have no fallback)")
        import torch  # noqa: F401  -- loads torch's HIP runtime first
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def strides3(vals) -> ctypes.Array:
    arr = (ctypes.c_int64 * 3)()
    for i, v in enumerate(vals):
        arr[i] = int(v)
    return arr


def check(rc: int, what: str) -> None:
    if rc != NQ_OK:
        msg = load().nq_last_error().decode(errors="replace")
        raise NQError(f"{what} failed (code {rc}): {msg}")
