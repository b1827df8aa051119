"""SwiGLU activation module and the biased variant.

Same names and semantics as src/rotalabs_accel/kernels/swiglu.py (a module
the reference package does not import from its ``__init__``):

* ``swiglu_fused`` / ``swiglu_torch`` (:79-146): the same functions as
  ``rotalabs_accel.kernels.activations`` (re-exported).
* ``SwiGLU`` (:149-177): the activation-only module, ``forward(gate, up)``.
  (``rotalabs_accel.SwiGLU`` is the other reference class of that name, the
  FFN module of activations.py:141-181.)
* ``swiglu_with_bias`` (:221-260): ``silu(gate + bias_gate) * (up + bias_up)``
  with the biases broadcast over the last dimension. GPU tensors run
  ``ra_swiglu_bias`` (fp32 math, one rounding, like the reference's Triton
  kernel :180-218); CPU tensors run the same arithmetic with torch ops in
  fp32.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from rotalabs_accel import _backend
from rotalabs_accel.kernels.activations import swiglu_fused, swiglu_torch

__all__ = ["swiglu_fused", "swiglu_torch", "SwiGLU", "swiglu_with_bias"]


class SwiGLU(torch.nn.Module):
    """Activation-only SwiGLU: ``forward(gate, up) = silu(gate) * up``."""

    def forward(self, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
        return swiglu_fused(gate, up)


def _swiglu_with_bias_torch(gate, up, bias_gate, bias_up):
    g = gate.float() + bias_gate.float()
    u = up.float() + bias_up.float()
    return (F.silu(g) * u).to(gate.dtype)


def swiglu_with_bias(
    gate: torch.Tensor,
    up: torch.Tensor,
    bias_gate: torch.Tensor,
    bias_up: torch.Tensor,
) -> torch.Tensor:
    """``silu(gate + bias_gate) * (up + bias_up)``; biases of shape (hidden,)
    broadcast over the last dimension of gate / up. Output dtype = gate's."""
    assert gate.shape == up.shape
    assert gate.shape[-1] == bias_gate.shape[0] == bias_up.shape[0]
    if not gate.is_cuda:
        return _swiglu_with_bias_torch(gate, up, bias_gate, bias_up)
    lib = _backend.load()
    dev = gate.device
    if up.device != dev or bias_gate.device != dev or bias_up.device != dev:
        raise RuntimeError(f"swiglu_with_bias: all tensors must be on {dev}")
    if up.dtype != gate.dtype:
        raise RuntimeError("swiglu_with_bias: gate and up must share a dtype")
    bdt = torch.promote_types(bias_gate.dtype, bias_up.dtype)
    g = gate.contiguous()
    u = up.contiguous()
    bg = bias_gate.to(bdt).contiguous()
    bu = bias_up.to(bdt).contiguous()
    out = torch.empty_like(g)
    if g.numel() == 0:
        return out
    with _backend.on_device(dev):
        _backend.check(lib.ra_swiglu_bias(g.data_ptr(), u.data_ptr(), bg.data_ptr(), bu.data_ptr(),
                                          _backend.dtype_code(bdt), out.data_ptr(), g.numel(), g.shape[-1],
                                          _backend.dtype_code(g.dtype), _backend.stream_handle(dev)))
    return out
