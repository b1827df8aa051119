"""Config 1, the reference's CPU plumbing workload, on the GPU machine.

x fp16 [16,4096] ~N(0,1), W fp32 [4096,4096] ~N(0,0.02) quantized per
channel, seed 0 (src/rotalabs_accel/kernels/gemm.py:31-48, the fallback).

* The recipe's inputs (x, q, s) are bit-identical to the reference's on this
  host (sha256 digests written where the reference ran).
* The CPU path on this host: equal to the reference's output bits where the
  host's CPU GEMM rounds as the reference's host did, and within
  rtol = atol = 1e-2 of them in any case (the fp16 GEMM of torch's CPU
  backend may accumulate in another order on another CPU).
* The HIP path on the same workload: within rtol = atol = 1e-2 of the
  reference's output and of the float64 oracle.
"""
import hashlib
import os

import numpy as np
import pytest
import torch

import rotalabs_accel as ra
from oracle import fallback
from workloads import PLUMBING_SHAPE, gemm_case

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _sha(t):
    a = t.contiguous()
    if a.dtype in (torch.float16, torch.bfloat16):
        a = a.view(torch.int16)
    return hashlib.sha256(a.numpy().tobytes()).hexdigest()


def test_plumbing_workload_on_gpu_host(gpu, golden_digests):
    M, K, N, seed = PLUMBING_SHAPE
    print(f"  plumbing M={M} K={K} N={N} seed={seed}", flush=True)
    c = gemm_case(M, K, N, seed)
    assert _sha(c.x) == golden_digests["x_f16"]
    assert _sha(c.q) == golden_digests["q"] and _sha(c.s) == golden_digests["s"]
    y_ref = torch.from_numpy(np.load(os.path.join(GOLDEN, "plumbing_y_f16.npy"))).view(torch.float16)
    assert _sha(y_ref) == golden_digests["y_f16"]
    # CPU path on this host
    y_cpu = ra.int8_gemm(c.x, c.q, c.s)
    assert y_cpu.dtype == torch.float16 and y_cpu.shape == (M, N)
    same = _sha(y_cpu) == golden_digests["y_f16"]
    neq = int((y_cpu != y_ref).sum())
    print(f"  CPU path: reference bits {'reproduced' if same else 'not reproduced'} "
          f"({neq} of {y_ref.numel()} fp16 values differ)", flush=True)
    torch.testing.assert_close(y_cpu.float(), y_ref.float(), rtol=1e-2, atol=1e-2)
    # HIP path
    y_gpu = ra.int8_gemm(c.x.to(gpu), c.q.to(gpu), c.s.to(gpu)).cpu()
    assert y_gpu.dtype == torch.float16 and y_gpu.shape == (M, N)
    torch.testing.assert_close(y_gpu.float(), y_ref.float(), rtol=1e-2, atol=1e-2)
    y64 = torch.from_numpy(fallback.gemm_f64(c.x.float().numpy(), c.q.numpy(), c.s.numpy()))
    torch.testing.assert_close(y_gpu.double(), y64, rtol=1e-2, atol=1e-2)
    # the kernel is the more accurate of the two (it scales the exact fp32
    # accumulator; the fallback rounds each dequantized weight to fp16 first)
    err_gpu = (y_gpu.double() - y64).abs().max().item()
    err_ref = (y_ref.double() - y64).abs().max().item()
    print(f"  max |y - y64|: HIP {err_gpu:.3g}, reference fallback {err_ref:.3g}", flush=True)
    assert err_gpu <= err_ref
