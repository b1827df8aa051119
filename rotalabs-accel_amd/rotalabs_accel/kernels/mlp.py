"""Decoder MLP with int8 projections: RMSNorm -> gate/up -> SwiGLU -> down.

The reference composes this dataflow in its SwiGLU module
(src/rotalabs_accel/kernels/activations.py:141-178) with fp16/fp32
nn.Linear projections, after an RMSNorm (kernels/normalization.py:186-216).
Here the projections are W8A16 int8 GEMMs and the gate and up projections
run as ONE GEMM over the row-concatenated weight [Wg; Wu] ([2I, H], per-row
scales -- identical to quantizing Wg and Wu separately) with SwiGLU applied
to the fp32 accumulators in the epilogue, so gate and up are never written
to memory:

    h = rmsnorm(x, norm_weight, eps)                       ra_rmsnorm
        (or rmsnorm_residual_fused(x, residual, ...)      ra_rmsnorm_residual)
    a = silu(h @ Wg^T * sg) * (h @ Wu^T * su)              ra_w8a16_gateup_swiglu
    y = a @ Wd^T * sd                                      ra_w8a16_gemm

On CPU tensors the same composition runs with the PyTorch ops
(rmsnorm_torch / rmsnorm_residual_torch, int8_gemm_torch, swiglu_torch).
"""
from __future__ import annotations

from typing import Optional

import torch

from rotalabs_accel import _backend
from rotalabs_accel.kernels.activations import SwiGLU, swiglu_fused, swiglu_torch
from rotalabs_accel.kernels.gemm import _rows, _workspace_size, int8_gemm, int8_gemm_torch
from rotalabs_accel.kernels.normalization import rmsnorm, rmsnorm_residual_fused
from rotalabs_accel.quantization.symmetric import quantize_weight_per_channel


def int8_gateup_swiglu(x: torch.Tensor, weight_gate_up: torch.Tensor, scale_gate_up: torch.Tensor) -> torch.Tensor:
    """``silu(x @ Wg^T * sg) * (x @ Wu^T * su)`` with ``weight_gate_up = [Wg; Wu]``.

    x: (..., K); weight_gate_up: int8 (2I, K); scale_gate_up: fp32 (2I,).
    Returns (..., I) in x's dtype.
    """
    assert weight_gate_up.dtype == torch.int8, "Weight must be INT8"
    K = x.shape[-1]
    n2 = weight_gate_up.shape[0]
    assert n2 % 2 == 0 and weight_gate_up.shape == (n2, K), \
        f"gate/up weight must be (2I, {K}), got {tuple(weight_gate_up.shape)}"
    assert scale_gate_up.shape == (n2,), f"Scale shape mismatch: {scale_gate_up.shape} vs ({n2},)"
    inter = n2 // 2
    if not (x.is_cuda and weight_gate_up.is_cuda and scale_gate_up.is_cuda):
        gu = int8_gemm_torch(x, weight_gate_up, scale_gate_up)
        return swiglu_torch(gu[..., :inter], gu[..., inter:])
    lib = _backend.load()
    dev = x.device
    if weight_gate_up.device != dev or scale_gate_up.device != dev:
        raise RuntimeError(f"int8_gateup_swiglu: all tensors must be on {dev}")
    x2, ldx = _rows(x.reshape(-1, K), align=16)
    w, ldw = _rows(weight_gate_up, align=16)
    s = scale_gate_up.float().contiguous()
    M = x2.shape[0]
    h = torch.empty((M, inter), dtype=x.dtype, device=dev)
    xdt = _backend.dtype_code(x.dtype)
    with _backend.on_device(dev):
        ws, ws_bytes = _backend.workspace(dev, _workspace_size(lib, M, inter, K, xdt, gateup=True))
        _backend.check(lib.ra_w8a16_gateup_swiglu_ws(
            x2.data_ptr(), ldx, xdt, w.data_ptr(), ldw, s.data_ptr(),
            h.data_ptr(), inter, M, inter, K, ws, ws_bytes, _backend.stream_handle(dev)))
    return h.view(*x.shape[:-1], inter)


def int8_mlp(x: torch.Tensor, norm_weight: torch.Tensor, weight_gate_up: torch.Tensor,
             scale_gate_up: torch.Tensor, weight_down: torch.Tensor, scale_down: torch.Tensor,
             eps: float = 1e-6, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm (of ``x + residual`` when given) -> fused gate/up + SwiGLU ->
    down projection."""
    if residual is not None:
        h = rmsnorm_residual_fused(x, residual, norm_weight, eps)
    else:
        h = rmsnorm(x, norm_weight, eps)
    a = int8_gateup_swiglu(h, weight_gate_up, scale_gate_up)
    return int8_gemm(a, weight_down, scale_down)


class Int8SwiGLUMLP(torch.nn.Module):
    """Pre-norm SwiGLU MLP block with int8 weights.

    Buffers: ``weight_gate_up`` int8 [2I, H] (= [Wg; Wu]), ``scale_gate_up``
    fp32 [2I], ``weight_down`` int8 [H, I], ``scale_down`` fp32 [H]; parameter
    ``norm_weight`` [H] of ``norm_dtype`` (keep it equal to the activation
    dtype so the normalised activations stay 16-bit, as torch promotes
    x.dtype with the weight dtype).
    """

    def __init__(self, hidden_size: int, intermediate_size: int, eps: float = 1e-6,
                 norm_dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.eps = eps
        self.norm_weight = torch.nn.Parameter(torch.ones(hidden_size, dtype=norm_dtype))
        self.register_buffer("weight_gate_up",
                             torch.zeros(2 * intermediate_size, hidden_size, dtype=torch.int8))
        self.register_buffer("scale_gate_up", torch.ones(2 * intermediate_size, dtype=torch.float32))
        self.register_buffer("weight_down", torch.zeros(hidden_size, intermediate_size, dtype=torch.int8))
        self.register_buffer("scale_down", torch.ones(hidden_size, dtype=torch.float32))
        self._quantized = False

    def quantize_weights(self, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor) -> None:
        """Per-output-channel quantization of the three projection weights
        ([I, H], [I, H], [H, I])."""
        H, inter = self.hidden_size, self.intermediate_size
        assert w_gate.shape == (inter, H) and w_up.shape == (inter, H) and w_down.shape == (H, inter)
        dev = self.weight_gate_up.device
        qg, sg = quantize_weight_per_channel(w_gate)
        qu, su = quantize_weight_per_channel(w_up)
        qd, sd = quantize_weight_per_channel(w_down)
        self.weight_gate_up[:inter].copy_(qg.to(dev))
        self.weight_gate_up[inter:].copy_(qu.to(dev))
        self.scale_gate_up[:inter].copy_(sg.to(dev))
        self.scale_gate_up[inter:].copy_(su.to(dev))
        self.weight_down.copy_(qd.to(dev))
        self.scale_down.copy_(sd.to(dev))
        self._quantized = True

    @classmethod
    def from_linears(cls, w_gate: torch.nn.Linear, w_up: torch.nn.Linear, w_down: torch.nn.Linear,
                     norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6) -> "Int8SwiGLUMLP":
        """Build from the three bias-free projections of a SwiGLU FFN (the
        reference SwiGLU module's w_gate / w_up / w_down) and an RMSNorm weight."""
        for lin in (w_gate, w_up, w_down):
            if lin.bias is not None:
                raise ValueError("Int8SwiGLUMLP supports bias-free projections only")
        H, inter = w_gate.in_features, w_gate.out_features
        dtype = norm_weight.dtype if norm_weight is not None else torch.bfloat16
        module = cls(H, inter, eps=eps, norm_dtype=dtype).to(w_gate.weight.device)
        module.quantize_weights(w_gate.weight.data, w_up.weight.data, w_down.weight.data)
        if norm_weight is not None:
            module.norm_weight.data.copy_(norm_weight)
        return module

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """MLP of ``rmsnorm(x)``, or of ``rmsnorm(x + residual)`` (one fused
        pass) when the residual stream is given."""
        if not self._quantized:
            raise RuntimeError("Weights not quantized. Call quantize_weights() first.")
        return int8_mlp(x, self.norm_weight, self.weight_gate_up, self.scale_gate_up,
                        self.weight_down, self.scale_down, self.eps, residual)

    def extra_repr(self) -> str:
        return (f"hidden_size={self.hidden_size}, intermediate_size={self.intermediate_size}, "
                f"eps={self.eps}, quantized={self._quantized}")


class Int8SwiGLU(torch.nn.Module):
    """The reference's SwiGLU FFN (activations.py:141-181:
    ``w_down(silu(w_gate(x)) * w_up(x))``) with W8A16 int8 projections.

    Same constructor as the reference module. Buffers: ``weight_gate_up``
    int8 [2I, H] (= [Wg; Wu], per-row scales, so identical to quantizing the
    two projections separately), ``scale_gate_up`` fp32 [2I], ``weight_down``
    int8 [H, I], ``scale_down`` fp32 [H]; with ``bias=True`` fp16 parameters
    ``bias_gate_up`` [2I] and ``bias_down`` [H] (fp16 like ``Int8Linear``'s).
    Without biases the gate and up projections run as one GEMM with SwiGLU in
    its epilogue (``int8_gateup_swiglu``); with biases they run as one biased
    GEMM, then ``swiglu_fused``. CPU tensors run the same composition with the
    PyTorch ops.
    """

    def __init__(self, hidden_size: int, intermediate_size: int, bias: bool = False):
        super().__init__()
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.register_buffer("weight_gate_up",
                             torch.zeros(2 * intermediate_size, hidden_size, dtype=torch.int8))
        self.register_buffer("scale_gate_up", torch.ones(2 * intermediate_size, dtype=torch.float32))
        self.register_buffer("weight_down", torch.zeros(hidden_size, intermediate_size, dtype=torch.int8))
        self.register_buffer("scale_down", torch.ones(hidden_size, dtype=torch.float32))
        if bias:
            self.bias_gate_up = torch.nn.Parameter(torch.zeros(2 * intermediate_size, dtype=torch.float16))
            self.bias_down = torch.nn.Parameter(torch.zeros(hidden_size, dtype=torch.float16))
        else:
            self.register_parameter("bias_gate_up", None)
            self.register_parameter("bias_down", None)
        self._quantized = False

    def quantize_weights(self, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor) -> None:
        """Per-output-channel quantization of the projection weights
        ([I, H], [I, H], [H, I]), on the CPU like ``Int8Linear.quantize_weights``."""
        H, inter = self.hidden_size, self.intermediate_size
        assert w_gate.shape == (inter, H) and w_up.shape == (inter, H) and w_down.shape == (H, inter)
        dev = self.weight_gate_up.device
        qg, sg = quantize_weight_per_channel(w_gate.detach().cpu())
        qu, su = quantize_weight_per_channel(w_up.detach().cpu())
        qd, sd = quantize_weight_per_channel(w_down.detach().cpu())
        self.weight_gate_up[:inter].copy_(qg.to(dev))
        self.weight_gate_up[inter:].copy_(qu.to(dev))
        self.scale_gate_up[:inter].copy_(sg.to(dev))
        self.scale_gate_up[inter:].copy_(su.to(dev))
        self.weight_down.copy_(qd.to(dev))
        self.scale_down.copy_(sd.to(dev))
        self._quantized = True

    @classmethod
    def from_swiglu(cls, module: SwiGLU) -> "Int8SwiGLU":
        """Quantize a ``SwiGLU`` FFN (on the device of its weights)."""
        has_bias = module.w_gate.bias is not None
        out = cls(module.hidden_size, module.intermediate_size, bias=has_bias).to(module.w_gate.weight.device)
        out.quantize_weights(module.w_gate.weight.data, module.w_up.weight.data, module.w_down.weight.data)
        if has_bias:
            inter = module.intermediate_size
            out.bias_gate_up.data[:inter].copy_(module.w_gate.bias.data.half())
            out.bias_gate_up.data[inter:].copy_(module.w_up.bias.data.half())
            out.bias_down.data.copy_(module.w_down.bias.data.half())
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self._quantized:
            raise RuntimeError("Weights not quantized. Call quantize_weights() first.")
        inter = self.intermediate_size
        if self.bias_gate_up is None:
            a = int8_gateup_swiglu(x, self.weight_gate_up, self.scale_gate_up)
        else:
            gu = int8_gemm(x, self.weight_gate_up, self.scale_gate_up, self.bias_gate_up)
            a = swiglu_fused(gu[..., :inter].contiguous(), gu[..., inter:].contiguous())
        return int8_gemm(a, self.weight_down, self.scale_down, self.bias_down)

    def extra_repr(self) -> str:
        return (f"hidden_size={self.hidden_size}, intermediate_size={self.intermediate_size}, "
                f"bias={self.bias_down is not None}, quantized={self._quantized}")
