"""RMSNorm (the prologue of the decoder MLP path).

Same names and semantics as src/rotalabs_accel/kernels/normalization.py:
``rmsnorm_torch`` (:32-45), ``rmsnorm`` (:186-216) and the ``TritonRMSNorm``
module (:258-285). The GPU branch runs ``ra_rmsnorm`` (librotaccel.so), which
follows the fallback's arithmetic: fp32 statistics, the normalised value
rounded to x's dtype, then multiplied by the weight in the promoted dtype.
"""
from __future__ import annotations

import torch

from rotalabs_accel import _backend


def rmsnorm_torch(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``(x.float() * rsqrt(mean(x.float()**2, -1) + eps)).to(x.dtype) * weight``."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)).to(x.dtype) * weight


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


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMS normalisation over the last dimension, times ``weight``."""
    assert x.shape[-1] == weight.shape[0], f"Hidden dim mismatch: {x.shape[-1]} vs {weight.shape[0]}"
    if x.is_cuda and weight.is_cuda:
        return _rmsnorm_hip(x, weight, eps)
    return rmsnorm_torch(x, weight, eps)


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
