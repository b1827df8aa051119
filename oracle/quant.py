"""numpy restatement of the reference's symmetric int8 quantization.

Follows src/rotalabs_accel/quantization/symmetric.py:
  quantize_symmetric           :24-82
  dequantize                   :85-123
  quantize_weight_per_channel  :126-151
  calculate_quantization_error :154-207

Reduced-precision inputs (fp16, bf16) follow PyTorch's CPU semantics for the
same op sequence: every elementwise op is computed in fp32 and rounded once to
the tensor dtype (round-to-nearest-even). bf16 is carried as uint16 bit
patterns because numpy has no bf16 type.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import numpy as np

QMAX = 127  # symmetric.py:57


# ---------------------------------------------------------------- bf16 helpers
def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (round-to-nearest-even), return uint16 bit patterns."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(a)
    out = rounded.astype(np.uint16)
    out[nan] = 0x7FC0
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_to(a32: np.ndarray, dtype: str) -> np.ndarray:
    """Round an fp32 array to ``dtype`` and return the rounded values as fp32."""
    if dtype == "f32":
        return a32.astype(np.float32)
    if dtype == "f16":
        return a32.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(a32))
    raise ValueError(dtype)


# ------------------------------------------------------------- quantization
def quantize_symmetric(t32: np.ndarray, dtype: str = "f32", dim: int | None = None):
    """Closed form of quantize_symmetric (symmetric.py:24-82).

    ``t32`` holds the tensor's values as fp32 (they must already be
    representable in ``dtype``). Returns (q int8, scale fp32).

    Steps, each rounded to ``dtype`` as the CPU tensor ops do:
      max_val = |t|.amax(dim, keepdim)           (:62 / :66, exact)
      scale   = round(max_val / 127)            (:63 / :67, true division)
      scale   = 1 where scale == 0              (:70)
      q       = int8(clamp(rne(round(t / scale)), -128, 127))   (:73)
      scale   = scale.float(); squeeze(dim)     (:76-80)
    NaN propagates through the amax (a row holding NaN gets a NaN scale) and a
    NaN quotient converts to 0, as torch's CPU conversion does.
    """
    t32 = np.asarray(t32, dtype=np.float32)
    a = np.abs(t32)
    if dim is None:
        max_val = a.max() if a.size else np.float32(0)
        max_val = np.asarray(max_val, dtype=np.float32)
    else:
        max_val = a.max(axis=dim, keepdims=True)
    scale = round_to(np.asarray(max_val / np.float32(QMAX), dtype=np.float32), dtype)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    with np.errstate(invalid="ignore"):
        ratio = round_to((t32 / scale).astype(np.float32), dtype)
    r = np.rint(ratio)
    q = np.where(np.isnan(r), 0, np.clip(r, -128, 127)).astype(np.int8)
    scale = scale.astype(np.float32)
    if dim is not None:
        scale = np.squeeze(scale, axis=dim)
    return q, scale


def quantize_weight_per_channel(w32: np.ndarray, dtype: str = "f32"):
    """symmetric.py:126-151: 2-D only, one scale per output row (reduce dim=1)."""
    w32 = np.asarray(w32, dtype=np.float32)
    assert w32.ndim == 2, f"Expected 2D weight matrix, got {w32.ndim}D"
    return quantize_symmetric(w32, dtype, dim=1)


def dequantize(q: np.ndarray, scale: np.ndarray, dtype: str = "f16", dim: int | None = None):
    """symmetric.py:85-123: fp32(q) * scale (one fp32 product), rounded to dtype.

    Returns fp32 values that are exactly representable in ``dtype``.
    """
    qf = q.astype(np.float32)
    s = np.asarray(scale, dtype=np.float32)
    if s.ndim == 1 and q.ndim == 2:
        s = s[:, None] if dim in (None, 0) else s[None, :]
    return round_to((qf * s).astype(np.float32), dtype)


def calculate_quantization_error(orig32: np.ndarray, q: np.ndarray, scale: np.ndarray,
                                 dtype: str = "f32", dim: int | None = None) -> dict:
    """symmetric.py:154-207, with sums done in float64 (so values agree with the
    reference to float32 reduction-order noise, not bit-for-bit)."""
    restored = dequantize(q, scale, dtype, dim)
    diff = round_to((orig32 - restored).astype(np.float32), dtype).astype(np.float64)
    o = orig32.astype(np.float64)
    thr = np.abs(o).max() * 0.1
    mask = np.abs(o) > thr
    rel = float((np.abs(diff[mask]) / np.abs(o[mask])).max() * 100) if mask.any() else 0.0
    signal = (o ** 2).mean()
    noise = (diff ** 2).mean()
    return {
        "max_abs_error": float(np.abs(diff).max()),
        "mean_abs_error": float(np.abs(diff).mean()),
        "relative_error_pct": rel,
        "snr_db": float(10 * np.log10(signal / (noise + 1e-10))),
    }


# ------------------------------------------------------------ KV-cache codec
def quantized_tensor_rows(t32: np.ndarray, dtype: str = "f32", bits: int = 8):
    """Closed form of QuantizedTensor(t, bits, per_channel=True)
    (src/rotalabs_accel/speculative/kv_compression.py:51-78) over the last
    dimension, every step rounded to ``dtype`` as the CPU tensor ops do:
      scale = round(|t|.amax(-1) / qmax), qmax = 2^(bits-1) - 1      (:64)
      scale = round(max(scale, 1e-8))                               (:65)
      q     = int8(clamp(rne(round(t / scale)), -qmax-1, qmax))     (:70-75)
    NaN ratios (0/0 of an all-zero row whose floor underflows in fp16)
    convert to 0. Returns (q int8, scale fp32 values of ``dtype``)."""
    t32 = np.asarray(t32, dtype=np.float32)
    qmax = (1 << (bits - 1)) - 1
    a = np.abs(t32).max(axis=-1, keepdims=True) if t32.shape[-1] else np.zeros(t32.shape[:-1] + (1,), np.float32)
    scale = round_to((a / np.float32(qmax)).astype(np.float32), dtype)
    scale = round_to(np.maximum(scale, np.float32(1e-8)).astype(np.float32), dtype)
    with np.errstate(invalid="ignore", divide="ignore"):
        ratio = round_to((t32 / scale).astype(np.float32), dtype)
    r = np.rint(ratio)
    q = np.where(np.isnan(r), 0, np.clip(r, -qmax - 1, qmax)).astype(np.int8)
    return q, scale


# ------------------------------------------------------------- W8A8 route
def quantize_activations_rows(x32: np.ndarray, dtype: str = "f16", act_scale: float = 127.0):
    """Closed form of the activation quantisation of _int8_gemm_cublas
    (src/rotalabs_accel/kernels/quantized_matmul.py:85-87) over rows of
    x (M, K), every op rounded to ``dtype`` as torch's CPU tensor ops do,
    with c = fp32(act_scale) (127 in the reference's default):
      a    = max(|x|.amax(1), round(1e-5))          (:85; NaN propagates)
      xs   = round(a / c)                           (:86; true division)
      mult = round(round(1 / a) * c)                (:87; torch evaluates
                                                     c / a as reciprocal * c)
      q    = int8(clamp(rne(round(x * mult)), -128, 127)), NaN -> 0
    Returns (q int8 (M, K), xs fp32 values of ``dtype`` (M,))."""
    x32 = np.asarray(x32, dtype=np.float32)
    c = np.float32(act_scale)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        a = np.abs(x32).max(axis=1)
        a = np.maximum(a, round_to(np.float32(1e-5).reshape(1), dtype)[0]).astype(np.float32)
        xs = round_to((a / c).astype(np.float32), dtype)
        recip = round_to((np.float32(1) / a).astype(np.float32), dtype)
        mult = round_to((recip * c).astype(np.float32), dtype)
        r = np.rint(round_to((x32 * mult[:, None]).astype(np.float32), dtype))
    q = np.where(np.isnan(r), 0, np.clip(r, -128, 127)).astype(np.int8)
    return q, xs


def w8a8_gemm_rows(xq: np.ndarray, xs32: np.ndarray, q: np.ndarray, s32: np.ndarray,
                   dtype: str = "f16", bias32: np.ndarray | None = None) -> np.ndarray:
    """The W8A8 GEMM as the reference's fused int8 kernel scales it
    (quantized_matmul.py:259): exact integer sums, then in fp32 with each op
    rounded, (float(sum) * xs[m]) * s[n] (+ bias[n]), rounded once to
    ``dtype``. Returns fp32 values of ``dtype`` (M, N)."""
    acc = xq.astype(np.int64) @ q.astype(np.int64).T
    y = (acc.astype(np.float32) * np.asarray(xs32, np.float32)[:, None]).astype(np.float32)
    y = (y * np.asarray(s32, np.float32)[None, :]).astype(np.float32)
    if bias32 is not None:
        y = (y + np.asarray(bias32, np.float32)[None, :]).astype(np.float32)
    return round_to(y, dtype)
