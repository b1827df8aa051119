"""nn.Module layers of the W8A16 path (names as src/rotalabs_accel/modules/__init__.py:7-11)."""
from rotalabs_accel.kernels.activations import SwiGLU
from rotalabs_accel.kernels.gemm import Int8Linear
from rotalabs_accel.kernels.mlp import Int8SwiGLUMLP
from rotalabs_accel.kernels.normalization import TritonRMSNorm
from rotalabs_accel.quantization.symmetric import QuantizedLinear

__all__ = ["TritonRMSNorm", "SwiGLU", "Int8Linear", "QuantizedLinear", "Int8SwiGLUMLP"]
