"""Speculative-decoding support of rotalabs-accel: only the int8 KV-cache
codec ``QuantizedTensor`` is provided here (src/rotalabs_accel/speculative/
kv_compression.py:51-88, the second int8 consumer next to the W8A16 GEMM);
the eviction policies and draft models are not implemented here."""
from rotalabs_accel.speculative.kv_compression import QuantizedTensor

__all__ = ["QuantizedTensor"]
