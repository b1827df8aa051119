"""W8A16 path kernels (re-export names as src/rotalabs_accel/kernels/__init__.py:38-42).

HAS_TRITON is kept for import compatibility and is always False: the GPU
kernels here are hand-written HIP for gfx950 (see HAS_HIP).
"""
from rotalabs_accel._backend import available as _hip_available
from rotalabs_accel.kernels.activations import SwiGLU, swiglu_fused, swiglu_torch
from rotalabs_accel.kernels.gemm import Int8Linear, int8_gemm, int8_gemm_torch
from rotalabs_accel.kernels.mlp import Int8SwiGLU, Int8SwiGLUMLP, int8_gateup_swiglu, int8_mlp
from rotalabs_accel.kernels.normalization import (
    TritonRMSNorm,
    rmsnorm,
    rmsnorm_residual_fused,
    rmsnorm_residual_torch,
    rmsnorm_torch,
)

HAS_TRITON = False
HAS_HIP = _hip_available()

__all__ = [
    "HAS_TRITON",
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
]
