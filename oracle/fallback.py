"""torch-CPU restatement of the reference's PyTorch fallback for the W8A16 path.

The reference's own fallback *is* a sequence of torch ops, so the restatement
uses the same ops, on CPU tensors only:

  int8_gemm_torch  src/rotalabs_accel/kernels/gemm.py:31-48
                   = F.linear(x, dequantize(W, s, dtype=x.dtype, dim=0), bias)
  dequantize       src/rotalabs_accel/quantization/symmetric.py:85-123
                   = (q.float() * s[:, None]).to(dtype)
  rmsnorm_torch    src/rotalabs_accel/kernels/normalization.py:32-45
                   = (x.float() * rsqrt(mean(x.float()^2, -1) + eps)).to(x.dtype) * w
  rmsnorm_residual_torch  normalization.py:48-64
                   = the same on v = (x + residual).float(), rounded to x.dtype
  swiglu_torch     src/rotalabs_accel/kernels/activations.py:36-45
                   = silu(gate) * up
  swiglu_with_bias src/rotalabs_accel/kernels/swiglu.py:221-260
                   = (silu(gate.f32 + bg.f32) * (up.f32 + bu.f32)).to(gate.dtype)

plus ``mlp_ref`` (RMSNorm -> gate/up -> SwiGLU -> down, the decoder-MLP
composition of the reference's SwiGLU module, activations.py:141-178, with
int8 projections) and float64 numpy references used for tolerance budgets.

This is also the CPU baseline that ``bench.py`` times ("port" kind).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def dequantize_ref(q: torch.Tensor, s: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return (q.float() * s.unsqueeze(1)).to(dtype)


def int8_gemm_ref(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor, bias=None) -> torch.Tensor:
    """gemm.py:31-48 on CPU tensors."""
    assert not x.is_cuda and not q.is_cuda and not s.is_cuda
    return F.linear(x, dequantize_ref(q, s, x.dtype), bias)


def rmsnorm_ref(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """normalization.py:32-45 on CPU tensors."""
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * r).to(x.dtype) * w


def rmsnorm_exact_ref(x32: np.ndarray, w32: np.ndarray, eps: float = 1e-6, dtype: str = "bf16",
                      out_dtype: str | None = None) -> np.ndarray:
    """normalization.py:43-45 with its fp32 ops exactly rounded.

    The fallback computes ``mean(x.float()**2)`` as an fp32 reduction whose
    last bit depends on the summation order (torch's CPU and GPU orders
    differ). Here the fp32 squares (exact for 16-bit x) are summed in float64
    and rounded once to fp32 -- the exactly rounded fp32 sum -- and the rest
    are single IEEE fp32 ops as in the fallback:
      s = fl32(sum_k fl32(x_k^2)); m = fl32(s / H); v = fl32(m + fl32(eps));
      r = fl32(1 / fl32(sqrt(v))); h = round_x(fl32(x * r)); y = round_y(h * w)
    x32, w32: values (as fp32) of 16-bit tensors of ``dtype`` (x) and
    ``out_dtype`` (w, default the same); returns y's values as fp32.
    """
    from oracle.quant import round_to
    out_dtype = out_dtype or dtype
    x32 = np.asarray(x32, np.float32)
    sq = (x32 * x32).astype(np.float32)
    s = sq.astype(np.float64).sum(axis=-1, keepdims=True).astype(np.float32)
    m = (s / np.float32(x32.shape[-1])).astype(np.float32)
    v = (m + np.float32(eps)).astype(np.float32)
    r = (np.float32(1) / np.sqrt(v)).astype(np.float32)
    h = round_to((x32 * r).astype(np.float32), dtype)
    return round_to((h * np.asarray(w32, np.float32)).astype(np.float32), out_dtype)


def rmsnorm_residual_ref(x: torch.Tensor, r: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """normalization.py:48-64 on CPU tensors."""
    v = (x + r).float()
    rr = torch.rsqrt(v.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (v * rr).to(x.dtype) * w


def quantized_tensor_ref(t: torch.Tensor, bits: int = 8, per_channel: bool = True):
    """kv_compression.py:51-78 (QuantizedTensor.__init__) on a CPU tensor:
    returns (data int8, scale)."""
    qmax = 2 ** (bits - 1) - 1
    if per_channel:
        scale = (t.abs().amax(dim=-1, keepdim=True) / qmax).clamp(min=1e-8)
    else:
        scale = max((t.abs().max() / qmax).item(), 1e-8)
    lo = -128 if bits == 8 else -8
    return (t / scale).round().clamp(lo, qmax).to(torch.int8), scale


def swiglu_ref(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """activations.py:36-45 on CPU tensors."""
    return F.silu(gate) * up


def swiglu_with_bias_ref(gate: torch.Tensor, up: torch.Tensor, bias_gate: torch.Tensor,
                         bias_up: torch.Tensor) -> torch.Tensor:
    """swiglu_with_bias (src/rotalabs_accel/kernels/swiglu.py:221-260): its
    Triton kernel (:201-218) loads gate, up and both biases as fp32, adds,
    computes silu(g) * u in fp32 and rounds once to gate's dtype."""
    g = gate.float() + bias_gate.float()
    u = up.float() + bias_up.float()
    return (F.silu(g) * u).to(gate.dtype)


def swiglu_with_bias_f64(gate: np.ndarray, up: np.ndarray, bias_gate: np.ndarray, bias_up: np.ndarray):
    """float64 closed form of the same, for pinning the restatement."""
    g = gate.astype(np.float64) + bias_gate.astype(np.float64)[None, :]
    u = up.astype(np.float64) + bias_up.astype(np.float64)[None, :]
    return g / (1.0 + np.exp(-g)) * u


def swiglu_ffn_ref(x, q_gu, s_gu, q_down, s_down, b_gu=None, b_down=None):
    """The reference SwiGLU module's forward (activations.py:175-178) with
    int8 projections: down(silu(gate(x)) * up(x)), gate/up as one [2I,H]
    weight."""
    inter = q_gu.shape[0] // 2
    gu = int8_gemm_ref(x, q_gu, s_gu, b_gu)
    a = swiglu_ref(gu[..., :inter], gu[..., inter:])
    return int8_gemm_ref(a, q_down, s_down, b_down)


def mlp_ref(x, norm_w, q_gu, s_gu, q_down, s_down, eps: float = 1e-6):
    """RMSNorm -> Int8 gate+up (one [2I,H] weight) -> SwiGLU -> Int8 down."""
    inter = q_gu.shape[0] // 2
    h = rmsnorm_ref(x, norm_w, eps)
    gu = int8_gemm_ref(h, q_gu, s_gu)
    a = swiglu_ref(gu[..., :inter], gu[..., inter:])
    return int8_gemm_ref(a, q_down, s_down)


# ---------------------------------------------------------- float64 references
def gemm_f64(x: np.ndarray, q: np.ndarray, s: np.ndarray, bias=None) -> np.ndarray:
    """y = x @ (fp32(q*s)).T (+ bias), accumulated in float64.

    The dequantized weight is the single fp32 product ``q*s`` (no rounding to
    the activation dtype); this is the 'fp32-accumulated reference' against
    which both the fallback and the kernels are within tolerance.
    """
    w = (q.astype(np.float32) * s.astype(np.float32)[:, None]).astype(np.float64)
    y = x.astype(np.float64) @ w.T
    if bias is not None:
        y = y + bias.astype(np.float64)
    return y


def swiglu_f64(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = g.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u.astype(np.float64)
