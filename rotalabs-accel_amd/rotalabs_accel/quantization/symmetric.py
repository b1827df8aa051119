"""Symmetric int8 quantization (W8A16 weights) and the QuantizedLinear module.

Same names, signatures, semantics and error behaviour as
src/rotalabs_accel/quantization/symmetric.py:

* scale = max|t| / 127 (per tensor, or per slice when ``dim`` names the
  reduced axis), 1 where that is 0;
* q = round_half_even(t / scale).clamp(-128, 127) as int8, scale as fp32.

For a 2-D weight on the GPU, per-output-channel quantization runs the HIP
kernel ``ra_quantize_per_channel``, which is bit-exact with the CPU op
sequence (IEEE division, round-half-even). ``QuantizedLinear.forward`` runs
the W8A16 GEMM (``int8_gemm``) instead of dequantize + F.linear; on CPU
tensors that is the same dequantize + F.linear computation.
"""
from __future__ import annotations

from typing import Optional

import torch

from rotalabs_accel import _backend

_QMAX = 127


def quantize_symmetric(
    tensor: torch.Tensor,
    bits: int = 8,
    dim: Optional[int] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric int8 quantization (reference: symmetric.py:24-82).

    ``dim`` is the axis reduced for the scale (``dim=1`` on an [N, K] weight
    gives one scale per output row). Returns (int8 tensor, fp32 scale).
    """
    assert bits == 8, f"Only 8-bit quantization supported, got {bits}"
    if dim is not None and tensor.is_cuda and tensor.dim() == 2 and dim in (1, -1) \
            and tensor.dtype in (torch.float32, torch.float16, torch.bfloat16):
        return _quantize_rows_hip(tensor)
    if dim is None:
        amax = tensor.abs().max()
    else:
        amax = tensor.abs().amax(dim=dim, keepdim=True)
    scale = amax / _QMAX
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    q = torch.round(tensor / scale).clamp(-128, 127).to(torch.int8)
    scale = scale.float()
    if dim is not None:
        scale = scale.squeeze(dim)
    return q, scale


def _quantize_rows_hip(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _backend.load()
    if w.stride(-1) != 1:
        w = w.contiguous()
    n, k = w.shape
    q = torch.empty((n, k), dtype=torch.int8, device=w.device)
    s = torch.empty((n,), dtype=torch.float32, device=w.device)
    with _backend.on_device(w.device):
        _backend.check(lib.ra_quantize_per_channel(
            w.data_ptr(), w.stride(0), _backend.dtype_code(w.dtype), n, k,
            q.data_ptr(), q.stride(0), s.data_ptr(), _backend.stream_handle(w.device)))
    return q, s


def dequantize(
    quantized: torch.Tensor,
    scale: torch.Tensor,
    dtype: torch.dtype = torch.float16,
    dim: Optional[int] = None,
) -> torch.Tensor:
    """q.float() * scale (broadcast per row for dim in (None, 0), per column
    for dim=1 when q is 2-D and scale 1-D), cast to ``dtype``
    (reference: symmetric.py:85-123)."""
    qf = quantized.float()
    if scale.dim() == 1 and quantized.dim() == 2:
        scale = scale.unsqueeze(1) if dim in (None, 0) else scale.unsqueeze(0)
    return (qf * scale).to(dtype)


def quantize_weight_per_channel(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel quantization of an [out, in] weight
    (reference: symmetric.py:126-151)."""
    assert weight.dim() == 2, f"Expected 2D weight matrix, got {weight.dim()}D"
    return quantize_symmetric(weight, bits=8, dim=1)


def calculate_quantization_error(
    original: torch.Tensor,
    quantized: torch.Tensor,
    scale: torch.Tensor,
    dim: Optional[int] = None,
) -> dict[str, float]:
    """Max / mean absolute error, max relative error (%) over values above 10%
    of the max magnitude, and SNR in dB (reference: symmetric.py:154-207)."""
    restored = dequantize(quantized, scale, dtype=original.dtype, dim=dim)
    diff = (original - restored).float()
    orig = original.float()
    max_abs = diff.abs().max().item()
    mean_abs = diff.abs().mean().item()
    significant = orig.abs() > orig.abs().max() * 0.1
    if significant.any():
        rel = (diff[significant].abs() / orig[significant].abs()).max().item() * 100
    else:
        rel = 0.0
    snr = 10 * torch.log10((orig ** 2).mean() / ((diff ** 2).mean() + 1e-10)).item()
    return {
        "max_abs_error": max_abs,
        "mean_abs_error": mean_abs,
        "relative_error_pct": rel,
        "snr_db": snr,
    }


_TORCH_DTYPE_NAMES = {torch.float32: "Float", torch.float16: "Half", torch.bfloat16: "BFloat16",
                      torch.float64: "Double"}


class QuantizedLinear(torch.nn.Module):
    """Linear layer with int8 per-channel weights (reference: symmetric.py:210-317).

    Buffers ``weight_int8`` [out, in] int8 and ``weight_scale`` [out] fp32 and
    an optional fp32 ``bias`` parameter, as in the reference, so its state
    dicts load unchanged. ``forward`` runs the W8A16 GEMM.
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("weight_int8", torch.zeros(out_features, in_features, dtype=torch.int8))
        self.register_buffer("weight_scale", torch.ones(out_features, dtype=torch.float32))
        if bias:
            self.bias = torch.nn.Parameter(torch.zeros(out_features))
        else:
            self.register_parameter("bias", None)
        self._quantized = False

    def quantize_weights(self, weight: torch.Tensor) -> None:
        """Quantize ``weight`` [out, in] on its own device and store it."""
        assert weight.shape == (self.out_features, self.in_features)
        q, s = quantize_weight_per_channel(weight)
        self.weight_int8.copy_(q)
        self.weight_scale.copy_(s)
        self._quantized = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self._quantized:
            raise RuntimeError("Weights not quantized. Call quantize_weights() first.")
        # The reference runs F.linear(x, dequantize(..., dtype=x.dtype), bias)
        # (symmetric.py:288-291), which rejects a bias whose dtype differs
        # from x's -- e.g. this module's fp32 bias with fp16/bf16 activations
        # -- on every device; the same error is raised here before the GEMM.
        if self.bias is not None and self.bias.dtype != x.dtype:
            raise RuntimeError(f"self and mat2 must have the same dtype, but got "
                               f"{_TORCH_DTYPE_NAMES.get(self.bias.dtype, self.bias.dtype)} and "
                               f"{_TORCH_DTYPE_NAMES.get(x.dtype, x.dtype)}")
        from rotalabs_accel.kernels.gemm import int8_gemm
        return int8_gemm(x, self.weight_int8, self.weight_scale, self.bias)

    @classmethod
    def from_linear(cls, linear: torch.nn.Linear) -> "QuantizedLinear":
        has_bias = linear.bias is not None
        module = cls(linear.in_features, linear.out_features, bias=has_bias)
        module.quantize_weights(linear.weight.data)
        if has_bias:
            module.bias.data.copy_(linear.bias.data)
        return module

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, quantized={self._quantized}")
