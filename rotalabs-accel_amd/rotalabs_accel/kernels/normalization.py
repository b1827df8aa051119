"""RMSNorm (the prologue of the decoder MLP path).

Same names and semantics as src/rotalabs_accel/kernels/normalization.py:
``rmsnorm_torch`` (:32-45), ``rmsnorm_residual_torch`` (:48-64), ``rmsnorm``
(:186-216), ``rmsnorm_residual_fused`` (:219-255) and the ``TritonRMSNorm``
module (:258-285). The GPU branches run ``ra_rmsnorm`` /
``ra_rmsnorm_residual`` (librotaccel.so), which follow the fallbacks'
arithmetic: x + residual rounded to the promoted dtype, fp32 statistics, the
normalised value rounded to x's dtype, then multiplied by the weight in the
promoted dtype.
"""
from __future__ import annotations

import torch

from rotalabs_accel import _backend


def rmsnorm_torch(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``(x.float() * rsqrt(mean(x.float()**2, -1) + eps)).to(x.dtype) * weight``."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)).to(x.dtype) * weight


def rmsnorm_residual_torch(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                           eps: float = 1e-6) -> torch.Tensor:
    """``rmsnorm_torch`` of ``x + residual`` (the sum in the promoted dtype);
    the normalised value is rounded to x's dtype."""
    x_plus_r = (x + residual).float()
    rms = torch.rsqrt(x_plus_r.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (x_plus_r * rms).to(x.dtype) * weight


def _row_view(t: torch.Tensor, hidden: int) -> tuple[torch.Tensor, int]:
    """(rows, hidden) view with unit column stride, and its row stride."""
    t2 = t.reshape(-1, hidden)
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < hidden):
        t2 = t2.contiguous()
    return t2, (t2.stride(0) if t2.shape[0] > 1 else hidden)


def _rmsnorm_hip(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    lib = _backend.load()
    if weight.device != x.device:
        raise RuntimeError(f"rmsnorm: weight must be on {x.device}")
    hidden = x.shape[-1]
    out_dtype = torch.promote_types(x.dtype, weight.dtype)
    x2 = x.reshape(-1, hidden)
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < hidden):
        x2 = x2.contiguous()
    rows = x2.shape[0]
    ldx = x2.stride(0) if rows > 1 else hidden
    w = weight.contiguous()
    y = torch.empty((rows, hidden), dtype=out_dtype, device=x.device)
    with _backend.on_device(x.device):
        _backend.check(lib.ra_rmsnorm(
            x2.data_ptr(), ldx, _backend.dtype_code(x.dtype), w.data_ptr(), _backend.dtype_code(w.dtype),
            y.data_ptr(), hidden, _backend.dtype_code(out_dtype), rows, hidden, float(eps),
            _backend.stream_handle(x.device)))
    return y.view(x.shape)


def _rmsnorm_residual_hip(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                          eps: float) -> torch.Tensor:
    lib = _backend.load()
    if weight.device != x.device or residual.device != x.device:
        raise RuntimeError(f"rmsnorm_residual_fused: all tensors must be on {x.device}")
    hidden = x.shape[-1]
    out_dtype = torch.promote_types(x.dtype, weight.dtype)
    x2, ldx = _row_view(x, hidden)
    r2, ldr = _row_view(residual, hidden)
    rows = x2.shape[0]
    w = weight.contiguous()
    y = torch.empty((rows, hidden), dtype=out_dtype, device=x.device)
    with _backend.on_device(x.device):
        _backend.check(lib.ra_rmsnorm_residual(
            x2.data_ptr(), ldx, _backend.dtype_code(x.dtype), r2.data_ptr(), ldr,
            _backend.dtype_code(residual.dtype), w.data_ptr(), _backend.dtype_code(w.dtype),
            y.data_ptr(), hidden, _backend.dtype_code(out_dtype), rows, hidden, float(eps),
            _backend.stream_handle(x.device)))
    return y.view(x.shape)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMS normalisation over the last dimension, times ``weight``."""
    assert x.shape[-1] == weight.shape[0], f"Hidden dim mismatch: {x.shape[-1]} vs {weight.shape[0]}"
    if x.is_cuda and weight.is_cuda:
        return _rmsnorm_hip(x, weight, eps)
    return rmsnorm_torch(x, weight, eps)


def rmsnorm_residual_fused(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                           eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm of ``x + residual`` times ``weight`` (one pass on the GPU)."""
    assert x.shape == residual.shape, f"Shape mismatch: x={x.shape}, residual={residual.shape}"
    assert x.shape[-1] == weight.shape[0], f"Hidden dim mismatch: {x.shape[-1]} vs {weight.shape[0]}"
    if x.is_cuda and residual.is_cuda and weight.is_cuda:
        return _rmsnorm_residual_hip(x, residual, weight, eps)
    return rmsnorm_residual_torch(x, residual, weight, eps)


class TritonRMSNorm(torch.nn.Module):
    """RMSNorm module (reference name kept for drop-in use; runs the HIP kernel
    on GPU tensors)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.hidden_size = hidden_size
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rmsnorm(x, self.weight, self.eps)

    def extra_repr(self) -> str:
        return f"{self.hidden_size}, eps={self.eps}"
