"""RMSNorm module with the reference's parameter layout (model/norm.py:11-22).

Used as QK-Norm by ``Attention``; there the normalisation is fused into the
HIP kernels, which read ``weight`` as fp32.  The module's own ``forward`` on a
device tensor of shape (..., head_dim) runs the gfx950 row kernel.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib, ops


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """RMSNorm over the last dim, fp32 arithmetic, output in x.dtype.

        Rows of 64 or 128 elements run on the row kernel; other widths are not
        part of the attention path and raise.
        """
        D = x.shape[-1]
        if D not in (64, 128):
            raise ValueError(f"RMSNorm kernel supports head_dim 64 or 128, got {D}")
        ops._require_device(x)
        rows = ops._rows_in(x.reshape(1, 1, -1, D))
        out = torch.empty(rows.shape, dtype=x.dtype, device=x.device)
        lib = _lib.load()
        st = _lib.strides3
        rc = lib.nq_qk_norm_rope(
            ops._ptr(rows), st(rows.stride()[:3]), ops._ptr(out),
            st(out.stride()[:3]), None, None, None, None, None, None, None, None,
            1, rows.shape[2], 1, 1, D, ops._code(x), ops._code(out),
            ops._ptr(ops._f32(self.weight, x.device)), None, float(self.eps),
            None, None, 0, None, None, 0, None, 0, ops._stream(x))
        _lib.check(rc, "RMSNorm")
        return out.view(x.shape)
