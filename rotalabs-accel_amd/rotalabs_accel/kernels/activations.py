"""SwiGLU activation ``silu(gate) * up``.

Same names and semantics as src/rotalabs_accel/kernels/activations.py:
``swiglu_torch`` (:36-45) and ``swiglu_fused`` (:108-138). The GPU branch runs
``ra_swiglu`` (fp32 math, one rounding, like the reference's Triton kernel
:51-80). On the MLP path the activation is fused into the gate/up GEMM
epilogue instead (see ``rotalabs_accel.kernels.mlp``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from rotalabs_accel import _backend


def swiglu_torch(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    return F.silu(gate) * up


def swiglu_fused(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` elementwise."""
    assert gate.shape == up.shape, f"Shape mismatch: gate={gate.shape}, up={up.shape}"
    if gate.is_cuda and up.is_cuda:
        lib = _backend.load()
        if gate.dtype != up.dtype or gate.device != up.device:
            raise RuntimeError("swiglu_fused: gate and up must share dtype and device")
        g = gate.contiguous()
        u = up.contiguous()
        out = torch.empty_like(g)
        with _backend.on_device(g.device):
            _backend.check(lib.ra_swiglu(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(),
                                         _backend.dtype_code(g.dtype), _backend.stream_handle(g.device)))
        return out
    return swiglu_torch(gate, up)


class SwiGLU(torch.nn.Module):
    """SwiGLU FFN ``w_down(silu(w_gate(x)) * w_up(x))`` with nn.Linear
    projections -- the reference's module (activations.py:141-181), same
    constructor, parameters and forward; the activation runs ``swiglu_fused``
    (the HIP kernel on GPU tensors). ``Int8SwiGLU.from_swiglu`` turns it into
    the int8 FFN."""

    def __init__(self, hidden_size: int, intermediate_size: int, bias: bool = False):
        super().__init__()
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.w_gate = torch.nn.Linear(hidden_size, intermediate_size, bias=bias)
        self.w_up = torch.nn.Linear(hidden_size, intermediate_size, bias=bias)
        self.w_down = torch.nn.Linear(intermediate_size, hidden_size, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate = self.w_gate(x)
        up = self.w_up(x)
        return self.w_down(swiglu_fused(gate, up))

    def extra_repr(self) -> str:
        return f"hidden_size={self.hidden_size}, intermediate_size={self.intermediate_size}"
