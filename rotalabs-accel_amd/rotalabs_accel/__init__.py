"""rotalabs_accel for AMD Instinct MI355X (gfx950): the W8A16 INT8 GEMM path.

Drop-in for the W8A16 path of rotalabs-accel (src/rotalabs_accel/__init__.py:
34-70 re-exports): ``int8_gemm`` / ``int8_gemm_torch`` / ``Int8Linear``,
the symmetric quantization utilities and ``QuantizedLinear``, and the
RMSNorm / SwiGLU ops of the decoder MLP, plus the fused int8 MLP block.
GPU tensors run hand-written HIP kernels (librotaccel.so); CPU tensors run
the PyTorch implementation, as in the reference.
"""
from rotalabs_accel._version import __version__
from rotalabs_accel.kernels import (
    HAS_HIP,
    Int8Linear,
    Int8SwiGLU,
    Int8SwiGLUMLP,
    SwiGLU,
    TritonRMSNorm,
    int8_gateup_swiglu,
    int8_gemm,
    int8_gemm_torch,
    int8_mlp,
    rmsnorm,
    rmsnorm_residual_fused,
    rmsnorm_residual_torch,
    rmsnorm_torch,
    swiglu_fused,
    swiglu_torch,
)
from rotalabs_accel.quantization import (
    QuantizedLinear,
    calculate_quantization_error,
    dequantize,
    quantize_symmetric,
    quantize_weight_per_channel,
)

__all__ = [
    "__version__",
    "HAS_HIP",
    "rmsnorm",
    "rmsnorm_torch",
    "rmsnorm_residual_fused",
    "rmsnorm_residual_torch",
    "TritonRMSNorm",
    "swiglu_fused",
    "swiglu_torch",
    "SwiGLU",
    "Int8SwiGLU",
    "int8_gemm",
    "int8_gemm_torch",
    "Int8Linear",
    "int8_gateup_swiglu",
    "int8_mlp",
    "Int8SwiGLUMLP",
    "quantize_symmetric",
    "dequantize",
    "quantize_weight_per_channel",
    "calculate_quantization_error",
    "QuantizedLinear",
]
