"""W8A16 GEMM: int8 per-output-channel weights, fp16/bf16 activations.

Same names, signatures and error behaviour as
src/rotalabs_accel/kernels/gemm.py:

* ``int8_gemm_torch`` (gemm.py:31-48): dequantize to x.dtype, then F.linear.
* ``int8_gemm`` (gemm.py:189-238): the same asserts, then the GPU kernels when
  x, weight and scale are GPU tensors, else ``int8_gemm_torch``.
* ``Int8Linear`` (gemm.py:241-336): same buffers (``weight_int8``, ``scale``,
  ``weight_transposed``, fp16 ``bias``), ``quantize_weights``, ``forward``,
  ``from_linear``.

The GPU branch calls ``ra_w8a16_gemm`` (librotaccel.so), which picks a
split-K MFMA kernel for small M (decode) or an LDS-staged MFMA GEMM for large
M (prefill). It reads ``weight_int8`` in its [N, K] layout, so
``weight_transposed`` is accepted and ignored (as are ``scale_fp16`` and
``use_cublas``, which the reference also ignores). The output has x's dtype
(the fallback's output dtype) and a bias of any float dtype is added to the
fp32 accumulator before the single rounding.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from rotalabs_accel import _backend
from rotalabs_accel.quantization.symmetric import dequantize, quantize_weight_per_channel


def int8_gemm_torch(
    x: torch.Tensor,
    weight_int8: torch.Tensor,
    scale: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """PyTorch W8A16 GEMM: ``F.linear(x, dequantize(W, s, x.dtype), bias)``."""
    return F.linear(x, dequantize(weight_int8, scale, dtype=x.dtype, dim=0), bias)


def _rows(t: torch.Tensor, align: int) -> tuple[torch.Tensor, int]:
    """Return (t2, ld): a 2-D view with unit column stride and row stride ld
    (in elements) whose rows start on ``align``-byte boundaries when the row
    length allows it; copies only when ``t`` is not already laid out so."""
    if t.is_contiguous() and t.data_ptr() % align == 0:  # the common case, checked cheaply
        cols = t.shape[1]
        if (cols * t.element_size()) % align == 0 or t.shape[0] <= 1:
            return t, cols
    rows, cols = t.shape
    ld = t.stride(0) if rows > 1 else cols
    esz = t.element_size()
    ok = (cols <= 1 or t.stride(1) == 1) and ld >= cols
    if ok and (cols * esz) % align == 0:
        ok = t.data_ptr() % align == 0 and (ld * esz) % align == 0
    if not ok:
        t = torch.empty((rows, cols), dtype=t.dtype, device=t.device).copy_(t)
        ld = cols
    return t, ld


_KERNEL_BIAS_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _split_bias(bias: Optional[torch.Tensor], N: int):
    """Split ``bias`` into (kernel_bias, post_bias).

    The kernels read a contiguous [N] bias at every output column n < N and
    add it to the fp32 accumulator. The reference adds the bias by
    broadcasting (``y = y + bias`` on the 2-D output, gemm.py:181-182), so
    any shape that broadcasts to [M, N] is legal there:

    * a bias holding exactly N values along its last dimension (shape (N,),
      (1, N), ...) of a kernel dtype goes to the kernel;
    * a one-element bias is expanded to [N] for the kernel;
    * anything else is returned as ``post_bias``, to be added to the GEMM
      output by broadcasting (torch raises for shapes that do not
      broadcast, as ``y + bias`` does in the reference).
    """
    if bias is None:
        return None, None
    if bias.dtype in _KERNEL_BIAS_DTYPES:
        if bias.dim() >= 1 and bias.shape[-1] == N and bias.numel() == N:
            return bias.reshape(N).contiguous(), None
        if bias.numel() == 1:
            return bias.reshape(1).expand(N).contiguous(), None
    return None, bias


_WS_SIZES: dict = {}


def _workspace_size(lib, M: int, N: int, K: int, xdt: int, gateup: bool = False) -> int:
    """Workspace bytes of ra_w8a16_gemm_ws / ra_w8a16_gateup_swiglu_ws for
    this problem (cached per shape)."""
    key = (M, N, K, xdt, gateup)
    n = _WS_SIZES.get(key)
    if n is None:
        fn = lib.ra_w8a16_gateup_workspace_size if gateup else lib.ra_w8a16_gemm_workspace_size
        n = _WS_SIZES[key] = int(fn(M, N, K, xdt))
    return n


def _int8_gemm_hip(x: torch.Tensor, weight_int8: torch.Tensor, scale: torch.Tensor,
                   bias: Optional[torch.Tensor], variant: int = _backend.VARIANT_AUTO) -> torch.Tensor:
    lib = _backend.load()
    dev = x.device
    if weight_int8.device != dev or scale.device != dev or (bias is not None and bias.device != dev):
        raise RuntimeError(f"int8_gemm: all tensors must be on {dev}")
    K = x.shape[-1]
    N = weight_int8.shape[0]
    xdt = _backend.dtype_code(x.dtype)
    x2, ldx = _rows(x if x.dim() == 2 else x.reshape(-1, K), align=16)
    M = x2.shape[0]
    w, ldw = _rows(weight_int8, align=16)
    s = scale if (scale.dtype == torch.float32 and scale.is_contiguous()) else scale.float().contiguous()
    b, post_bias = _split_bias(bias, N)
    b_ptr, b_dt = (None, _backend.F32) if b is None else (b.data_ptr(), _backend.dtype_code(b.dtype))
    y = torch.empty((M, N), dtype=x.dtype, device=dev)
    with _backend.on_device(dev):
        ws, ws_bytes = _backend.workspace(dev, _workspace_size(lib, M, N, K, xdt))
        code = lib.ra_w8a16_gemm_ex(
            x2.data_ptr(), ldx, xdt, w.data_ptr(), ldw, s.data_ptr(), b_ptr, b_dt,
            y.data_ptr(), N, M, N, K, variant, ws, ws_bytes, _backend.stream_handle(dev))
    _backend.check(code)
    if post_bias is not None:
        y.add_(post_bias)
    return y if x.dim() == 2 else y.view(*x.shape[:-1], N)


def int8_gemm(
    x: torch.Tensor,
    weight_int8: torch.Tensor,
    scale: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    weight_transposed: Optional[torch.Tensor] = None,
    scale_fp16: Optional[torch.Tensor] = None,
    use_cublas: Optional[bool] = None,
) -> torch.Tensor:
    """W8A16 GEMM: ``y = x @ (weight_int8 * scale[:, None]).T + bias``.

    Args:
        x: activations (..., K), fp16 / bf16 (fp32 also accepted).
        weight_int8: int8 weight (N, K).
        scale: fp32 per-output-channel scale (N,).
        bias: optional bias (N,).
        weight_transposed, scale_fp16, use_cublas: accepted for API
            compatibility and ignored.

    Returns:
        (..., N) tensor of x's dtype.
    """
    assert weight_int8.dtype == torch.int8, "Weight must be INT8"
    K = x.shape[-1]
    N = weight_int8.shape[0]
    assert weight_int8.shape == (N, K), f"Weight shape mismatch: {weight_int8.shape} vs ({N}, {K})"
    assert scale.shape == (N,), f"Scale shape mismatch: {scale.shape} vs ({N},)"
    if x.is_cuda and weight_int8.is_cuda and scale.is_cuda:
        return _int8_gemm_hip(x, weight_int8, scale, bias)
    return int8_gemm_torch(x, weight_int8, scale, bias)


class Int8Linear(torch.nn.Module):
    """Linear layer with int8 weights running the W8A16 GEMM
    (reference: gemm.py:241-336).

    Buffers as in the reference -- ``weight_int8`` [out, in] int8, ``scale``
    [out] fp32, ``weight_transposed`` [in, out] int8 -- and an optional fp16
    ``bias`` parameter, so reference checkpoints load unchanged. The kernels
    read ``weight_int8``; ``weight_transposed`` is kept only for checkpoint
    compatibility.
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("weight_int8", torch.zeros(out_features, in_features, dtype=torch.int8))
        self.register_buffer("scale", torch.ones(out_features, dtype=torch.float32))
        self.register_buffer("weight_transposed", torch.zeros(in_features, out_features, dtype=torch.int8))
        if bias:
            self.bias = torch.nn.Parameter(torch.zeros(out_features, dtype=torch.float16))
        else:
            self.register_parameter("bias", None)
        self._quantized = False

    def quantize_weights(self, weight: torch.Tensor) -> None:
        """Quantize an fp16/fp32 [out, in] weight per output channel and store it.

        The reference always quantizes on the CPU; a GPU weight is quantized on
        the GPU here by a kernel that produces the same bits.
        """
        assert weight.shape == (self.out_features, self.in_features)
        q, s = quantize_weight_per_channel(weight)
        dev = self.weight_int8.device
        self.weight_int8.copy_(q.to(dev))
        self.scale.copy_(s.to(dev))
        self.weight_transposed.copy_(q.t().contiguous().to(dev))
        self._quantized = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self._quantized:
            raise RuntimeError("Weights not quantized. Call quantize_weights() first.")
        return int8_gemm(x, self.weight_int8, self.scale, self.bias,
                         weight_transposed=self.weight_transposed)

    @classmethod
    def from_linear(cls, linear: torch.nn.Linear) -> "Int8Linear":
        has_bias = linear.bias is not None
        module = cls(linear.in_features, linear.out_features, bias=has_bias)
        module = module.to(linear.weight.device)
        module.quantize_weights(linear.weight.data)
        if has_bias:
            module.bias.data.copy_(linear.bias.data.half())
        return module

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, quantized={self._quantized}")
