"""RMSNorm module with the reference's parameter layout (model/norm.py:11-22).

``Attention`` fuses QK-Norm into its HIP kernels, which read ``weight`` as
fp32.  The module's own ``forward`` runs ``nq_rmsnorm``: rows of any width (a
multiple of 8), the reference's cast order (the normalised value is cast back
to ``x.dtype`` before the weight multiply) and its dtype promotion (a bf16
input with an fp32 weight gives fp32, as ``output.type_as(x) * weight`` does).
Under autograd dx comes from ``nq_qk_norm_rope_bwd`` at widths 32, 64 and 128
(QK-Norm's head dims) and from a torch composition of the same formula at other
widths (the model's hidden-size norms); the weight gradient is reduced from the
incoming gradient in fp32, as the reference's autograd does.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib, ops


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """model/norm.py:20-22 on the device: (x, weight) -> y in their promoted dtype."""
    ops._require_device(x, weight)
    W = x.shape[-1]
    if W % 8:
        raise ValueError(f"nq_rmsnorm takes widths that are multiples of 8, got {W}")
    out_dtype = torch.promote_types(x.dtype, weight.dtype)
    rows = x.reshape(-1, W)
    if rows.stride(-1) != 1 or not ops._aligned(rows):
        rows = rows.contiguous()
    w = weight if weight.is_contiguous() else weight.contiguous()
    y = torch.empty(rows.shape, dtype=out_dtype, device=x.device)
    rc = _lib.load().nq_rmsnorm(ops._ptr(rows), rows.stride(0), ops._ptr(w), ops._ptr(y), y.stride(0),
                                rows.shape[0], W, ops._code(rows), ops._code(w), ops._code(y), float(eps),
                                ops._stream(x))
    _lib.check(rc, "nq_rmsnorm")
    return y.view(x.shape)


class _RMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps: float):
        ctx.save_for_backward(x, weight)
        ctx.eps = eps
        return rms_norm(x, weight, eps)

    @staticmethod
    def backward(ctx, dy):
        # y = n.to(x.dtype) * w with n = x * rsqrt(mean(x^2) + eps) in fp32
        # (model/norm.py:17-22).  dw = sum over rows of dy * n.to(x.dtype), in
        # fp32 from dy as it arrives; dx = r * (g - n * mean(g * n)) with g the
        # gradient of the cast value, (dy * w) in x's dtype.
        x, weight = ctx.saved_tensors
        W = x.shape[-1]
        ones = torch.ones(W, dtype=torch.float32, device=x.device)
        ncast = rms_norm(x, ones, ctx.eps)  # n.to(x.dtype), held in fp32 exactly
        dw = (dy.float() * ncast).reshape(-1, W).sum(0).to(weight.dtype)
        if W in (32, 64, 128):
            x4 = x.reshape(1, 1, -1, W)
            dy4 = dy.to(x.dtype).reshape(1, 1, -1, W)
            dx, _ = ops.qk_norm_rope_backward(x4, dy4, weight=weight, eps=ctx.eps)
            return dx.reshape(x.shape), dw, None
        xf = x.float()
        r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + ctx.eps)
        n = xf * r
        g = (dy * weight).to(x.dtype).float()
        dx = r * (g - n * (g * n).mean(-1, keepdim=True))
        return dx.to(x.dtype), dw, None


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad):
            return _RMSNormFn.apply(x, self.weight, self.eps)
        return rms_norm(x, self.weight, self.eps)
