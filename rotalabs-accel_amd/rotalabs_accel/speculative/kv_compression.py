"""Int8 / int4 KV-cache codec, as src/rotalabs_accel/speculative/
kv_compression.py:51-88 (``QuantizedTensor``).

Same constructor, attributes (``bits``, ``per_channel``, ``shape``,
``dtype``, ``device``, ``scale``, ``data``), ``dequantize()`` and
``memory_bytes``. Per-channel quantisation of a GPU tensor runs
``ra_quantize_rows`` (one pass over the tensor), which reproduces the CPU
arithmetic bit for bit: every step rounded to the tensor's dtype, true
division by qmax. (The reference runs the same torch ops on any device; on a
GPU, torch may divide by qmax as a multiplication by its reciprocal.)
Per-tensor quantisation runs the torch ops.
"""
from __future__ import annotations

import torch

from rotalabs_accel import _backend


class QuantizedTensor:
    """Quantized tensor for KV-cache compression (int8 storage for 8 and 4 bits)."""

    def __init__(self, tensor: torch.Tensor, bits: int = 8, per_channel: bool = True):
        self.bits = bits
        self.per_channel = per_channel
        self.shape = tensor.shape
        self.dtype = tensor.dtype
        self.device = tensor.device
        if bits not in (8, 4):
            raise ValueError(f"Unsupported bits: {bits}")
        qmax = 2 ** (bits - 1) - 1
        if per_channel and tensor.is_cuda and tensor.dtype in (torch.float16, torch.bfloat16, torch.float32) \
                and tensor.dim() > 0:
            self.data, self.scale = self._quantize_rows_hip(tensor, bits)
            return
        if per_channel:
            self.scale = tensor.abs().amax(dim=-1, keepdim=True) / qmax
            self.scale = self.scale.clamp(min=1e-8)
        else:
            self.scale = tensor.abs().max() / qmax
            self.scale = max(self.scale.item(), 1e-8)
        lo = -128 if bits == 8 else -8
        self.data = (tensor / self.scale).round().clamp(lo, qmax).to(torch.int8)

    @staticmethod
    def _quantize_rows_hip(tensor: torch.Tensor, bits: int):
        lib = _backend.load()
        cols = tensor.shape[-1]
        t2 = tensor.reshape(-1, cols)
        if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < cols):
            t2 = t2.contiguous()
        rows = t2.shape[0]
        ldt = t2.stride(0) if rows > 1 else cols
        q = torch.empty((rows, cols), dtype=torch.int8, device=tensor.device)
        scale = torch.empty((rows, 1), dtype=tensor.dtype, device=tensor.device)
        with _backend.on_device(tensor.device):
            _backend.check(lib.ra_quantize_rows(
                t2.data_ptr(), ldt, _backend.dtype_code(tensor.dtype), rows, cols, bits, q.data_ptr(), cols,
                scale.data_ptr(), _backend.stream_handle(tensor.device)))
        return q.view(tensor.shape), scale.view(tensor.shape[:-1] + (1,))

    def dequantize(self) -> torch.Tensor:
        return self.data.to(self.dtype) * self.scale

    @property
    def memory_bytes(self) -> int:
        data_bytes = self.data.numel() * (1 if self.bits == 8 else 0.5)
        scale_bytes = self.scale.numel() * 4 if isinstance(self.scale, torch.Tensor) else 4
        return int(data_bytes + scale_bytes)
