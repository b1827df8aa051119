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
