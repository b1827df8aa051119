"""nn.Module layer of the W8A16 path (names as src/rotalabs_accel/modules/__init__.py:8-12)."""
from rotalabs_accel.kernels.gemm import Int8Linear
from rotalabs_accel.kernels.mlp import Int8SwiGLUMLP
from rotalabs_accel.kernels.normalization import TritonRMSNorm
from rotalabs_accel.quantization.symmetric import QuantizedLinear

__all__ = ["TritonRMSNorm", "Int8Linear", "QuantizedLinear", "Int8SwiGLUMLP"]
