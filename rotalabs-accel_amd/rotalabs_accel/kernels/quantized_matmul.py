"""Opt-in W8A8 route: int8 activations x int8 weights on the int8 matrix cores.

Same names and dispatch as src/rotalabs_accel/kernels/quantized_matmul.py
(a module the reference package itself does not import):

* ``_int8_gemm_cublas`` (:43-102): per-row absmax quantisation of the
  activations (:85-87), an int8 x int8 -> int32 GEMM (``torch._int_mm`` at
  :93) and the dequantisation ``sum * x_scale * w_scale`` (:99-100). Here the
  two GPU steps are ``ra_quantize_act_rows`` and ``ra_w8a8_gemm``
  (v_mfma_i32_32x32x32_i8, twice the fp16 MFMA rate).
* ``int8_gemm`` (:369-480): ``use_cublas=True`` with more than 16 rows takes
  the W8A8 route (:441-447); everything else is the W8A16 GEMM of
  ``rotalabs_accel.kernels.gemm``. ``use_cublas=None`` means False, as there.

The route is opt-in because quantising the activations adds error (the
reference quotes ~3-8% extra, :438-440); the package-level ``int8_gemm``
ignores ``use_cublas`` exactly as the reference's gemm.py does.

Two deliberate differences from the reference's cuBLAS route, both shared
with its fused int8 kernel (:162-264):

* the int32 sums are scaled in fp32 and rounded once to the output dtype
  (:259). ``_dequantize_output`` (:38-40) converts them to fp16 first, which
  turns every |sum| > 65504 into inf -- a common case at K = 4096;
* ``x_scale`` keeps the activation dtype (fp16 or bf16); the reference only
  accepts fp16 (:421).

CPU tensors run the same arithmetic with torch ops (an exact float64 matmul
stands in for the int32 GEMM), so both devices give the same bits.
"""
from __future__ import annotations

from typing import Optional

import torch

from rotalabs_accel import _backend
from rotalabs_accel.kernels import gemm as _gemm
from rotalabs_accel.kernels.gemm import Int8Linear, int8_gemm_torch  # noqa: F401  (re-exported as there)

# Rows above which use_cublas=True takes the W8A8 route (quantized_matmul.py:441).
W8A8_MIN_M = 17
ACT_SCALE = 127.0


def _quantize_activations_torch(x2: torch.Tensor, act_scale: float):
    """The reference's ops (quantized_matmul.py:85-87), x_scale in x's dtype."""
    absmax = x2.abs().amax(dim=1, keepdim=True).clamp(min=1e-5)
    x_scale = (absmax / act_scale).to(x2.dtype)
    q = (x2 * (act_scale / absmax)).round().clamp(-128, 127).to(torch.int8)
    return q, x_scale.reshape(-1)


def quantize_activations(x: torch.Tensor, act_scale: float = ACT_SCALE):
    """Per-row symmetric int8 quantisation of activations ``x`` (..., K).

    Returns ``(x_int8, x_scale)``: int8 (M, K) and the per-row scale (M,) in
    x's dtype, M = x.numel() // K, with ``x ~= x_int8 * x_scale[:, None]``:
    ``x_scale = absmax / act_scale`` and ``x_int8 = round(x * (act_scale /
    absmax))`` clamped to [-128, 127], as quantized_matmul.py:85-87. GPU
    tensors (fp16 / bf16) run ``ra_quantize_act_rows``, which rounds every
    step as torch does on the CPU (``act_scale`` taken as an fp32 value; for
    127, the default, CPU and GPU torch agree).
    """
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if not x.is_cuda:
        return _quantize_activations_torch(x2, act_scale)
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"W8A8 route: activations must be float16 or bfloat16 on the GPU, got {x.dtype}")
    lib = _backend.load()
    xr, ldx = _gemm._rows(x2, align=16)
    M = xr.shape[0]
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    xs = torch.empty((M,), dtype=x.dtype, device=x.device)
    with _backend.on_device(x.device):
        _backend.check(lib.ra_quantize_act_rows(xr.data_ptr(), ldx, _backend.dtype_code(x.dtype), M, K,
                                                q.data_ptr(), K, xs.data_ptr(), float(act_scale),
                                                _backend.stream_handle(x.device)))
    return q, xs


def _w8a8_gemm_torch(x_int8, x_scale, weight_int8, scale, bias, out_dtype):
    acc = x_int8.double() @ weight_int8.double().t()  # exact: |sum| < 2^53
    y = (acc.float() * x_scale.float()[:, None]) * scale.float()[None, :]
    if bias is not None:
        y = y + bias.float()
    return y.to(out_dtype)


def w8a8_gemm(
    x_int8: torch.Tensor,
    x_scale: torch.Tensor,
    weight_int8: torch.Tensor,
    scale: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """``y = (float(x_int8 @ weight_int8.T) * x_scale[:, None]) * scale + bias``.

    x_int8: int8 (M, K); x_scale: (M,) fp16 / bf16 (the output dtype);
    weight_int8: int8 (N, K); scale: fp32 (N,); bias: optional (N,).
    Exact int32 sums, fp32 scaling, one rounding. GPU tensors run
    ``ra_w8a8_gemm``.
    """
    assert x_int8.dtype == torch.int8 and weight_int8.dtype == torch.int8, "Operands must be INT8"
    M, K = x_int8.shape
    N = weight_int8.shape[0]
    assert weight_int8.shape == (N, K), f"Weight shape mismatch: {weight_int8.shape} vs ({N}, {K})"
    assert scale.shape == (N,), f"Scale shape mismatch: {scale.shape} vs ({N},)"
    assert x_scale.shape == (M,), f"Activation scale shape mismatch: {x_scale.shape} vs ({M},)"
    out_dtype = x_scale.dtype
    if not x_int8.is_cuda:
        return _w8a8_gemm_torch(x_int8, x_scale, weight_int8, scale, bias, out_dtype)
    if out_dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"W8A8 route: x_scale must be float16 or bfloat16 on the GPU, got {out_dtype}")
    dev = x_int8.device
    for t in (x_scale, weight_int8, scale) + ((bias,) if bias is not None else ()):
        if t.device != dev:
            raise RuntimeError(f"w8a8_gemm: all tensors must be on {dev}")
    lib = _backend.load()
    xq, ldxq = _gemm._rows(x_int8, align=16)
    w, ldw = _gemm._rows(weight_int8, align=16)
    xs = x_scale.contiguous()
    s = scale if (scale.dtype == torch.float32 and scale.is_contiguous()) else scale.float().contiguous()
    b, post_bias = _gemm._split_bias(bias, N)
    b_ptr, b_dt = (None, _backend.F32) if b is None else (b.data_ptr(), _backend.dtype_code(b.dtype))
    y = torch.empty((M, N), dtype=out_dtype, device=dev)
    with _backend.on_device(dev):
        _backend.check(lib.ra_w8a8_gemm(xq.data_ptr(), ldxq, xs.data_ptr(), w.data_ptr(), ldw, s.data_ptr(),
                                        b_ptr, b_dt, y.data_ptr(), N, _backend.dtype_code(out_dtype), M, N, K,
                                        _backend.stream_handle(dev)))
    if post_bias is not None:
        y.add_(post_bias)
    return y


def _int8_gemm_cublas(
    x: torch.Tensor,
    weight_int8: torch.Tensor,
    scale: torch.Tensor,
    scale_fp16: Optional[torch.Tensor] = None,
    act_scale: float = ACT_SCALE,
) -> torch.Tensor:
    """W8A8 GEMM of 2-D activations x (M, K) with int8 weights (N, K): the
    reference's function (quantized_matmul.py:43-102) on the int8 MFMA
    kernels. ``scale_fp16`` is accepted and ignored (the scaling is fp32)."""
    M, K = x.shape
    N, K2 = weight_int8.shape
    assert K == K2, f"Dimension mismatch: x has K={K}, weight has K={K2}"
    x_int8, x_scale = quantize_activations(x, act_scale)
    return w8a8_gemm(x_int8, x_scale, weight_int8, scale)


def int8_gemm(
    x: torch.Tensor,
    weight_int8: torch.Tensor,
    scale: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    weight_transposed: Optional[torch.Tensor] = None,
    scale_fp16: Optional[torch.Tensor] = None,
    use_cublas: Optional[bool] = None,
) -> torch.Tensor:
    """INT8-weight GEMM ``y = x @ (weight_int8 * scale[:, None]).T + bias``.

    ``use_cublas=True`` with more than 16 rows quantises the activations per
    row and runs the int8 x int8 GEMM (W8A8, faster for prefill, less
    accurate); otherwise the W8A16 GEMM. ``weight_transposed`` and
    ``scale_fp16`` are accepted and ignored.
    """
    assert weight_int8.dtype == torch.int8, "Weight must be INT8"
    K = x.shape[-1]
    N = weight_int8.shape[0]
    assert weight_int8.shape == (N, K), f"Weight shape mismatch: {weight_int8.shape} vs ({N}, {K})"
    assert scale.shape == (N,), f"Scale shape mismatch: {scale.shape} vs ({N},)"
    x2 = x.reshape(-1, K)
    if use_cublas and x2.shape[0] >= W8A8_MIN_M:
        x_int8, x_scale = quantize_activations(x2)
        y = w8a8_gemm(x_int8, x_scale, weight_int8, scale, bias)
        return y.view(*x.shape[:-1], N)
    return _gemm.int8_gemm(x, weight_int8, scale, bias)
