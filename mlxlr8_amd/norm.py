"""Residual add + RMSNorm of decode rows (mirrors ``exlr8/fast_norm.py:20-28``).

``residual_rms_pair(x, residual, weight)`` returns ``(h, out)`` with ``h = T(x + residual)`` and
``out = T(weight * T(h * rsqrt(mean(h^2) + eps)))`` (T = bf16, fp32 mean), as the reference's
fused Metal kernel does for ``DecoderLayer.__call__`` (``exlr8/model.py:376-384``).
"""
import torch

from ._lib import check, lib, ptr, require_cuda, stream
from .trellis import BF16

EPS = 1e-5


def _rows(x):
    n = x.shape[-1]
    if n % 2048 or n > 8192:
        raise ValueError("the normalised width must be a multiple of 2048 up to 8192")
    if x.dtype != BF16:
        raise ValueError("this build normalises bf16 rows")
    return x.numel() // n, n


def residual_rms_pair(x, residual, weight, eps=EPS):
    """(h, out) = (T(x + residual), rms_norm(h, weight)); residual may be None."""
    rows, n = _rows(x)
    tensors = [x, weight] + ([residual] if residual is not None else [])
    require_cuda(*tensors)
    xr = x.reshape(rows, n).contiguous()
    rr = residual.reshape(rows, n).to(BF16).contiguous() if residual is not None else None
    w = weight.to(BF16).contiguous()
    if w.numel() != n:
        raise ValueError("the norm weight must have one entry per feature")
    h = torch.empty_like(xr)
    out = torch.empty_like(xr)
    check(lib().moe_residual_rmsnorm(ptr(xr), ptr(rr) if rr is not None else None, ptr(w), rows, n, float(eps),
                                     ptr(h), ptr(out), stream(x.device)))
    return h.reshape(x.shape), out.reshape(x.shape)


def rms_norm(x, weight, eps=EPS):
    """``mx.fast.rms_norm`` for bf16 rows (the ``out`` half of ``residual_rms_pair``)."""
    return residual_rms_pair(x, None, weight, eps)[1]
