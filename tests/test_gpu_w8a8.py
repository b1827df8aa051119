"""GPU parity of the opt-in W8A8 route (int8 activations x int8 weights on
the int8 MFMA), through the C ABI (ra_quantize_act_rows, ra_w8a8_gemm).

Everything here is integer work followed by fp32 scaling with a fixed op
order, so the bar is bit-exact:

* activation quantisation vs the numpy restatement of quantized_matmul.py:
  85-87 (edge rows: zeros, NaN, inf, values below the 1e-5 floor);
* the GEMM vs the numpy restatement (exact int64 sums) on ragged shapes that
  run every tile shape and the any-K kernel, with every bias dtype;
* full-size workloads vs torch._int_mm (hipBLASLt's exact int32 sums) scaled
  by torch in fp32 on the GPU, plus rows re-checked against the oracle;
* strided, misaligned and > 2 GiB operands; determinism; the
  ``int8_gemm(..., use_cublas=True)`` dispatch.
"""
import numpy as np
import pytest
import torch

import rotalabs_accel as ra
from oracle import quant as oq
from rotalabs_accel.kernels import quantized_matmul as qm

pytestmark = pytest.mark.gpu

DT = {torch.float16: "f16", torch.bfloat16: "bf16"}


def _acts(M, K, dt, seed, edges=True):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * (torch.rand(M, 1, generator=g) * 8 + 0.01)).to(dt)
    if edges and M >= 8:
        x[0] = 0
        x[1, K // 2] = float("nan")
        x[2, K - 1] = float("inf")
        x[3] = 1e-7
        x[4] = 3e-5
        x[5] = -2.0
        x[7] = 60000.0 if dt == torch.float16 else 3e38
    return x


def _weights(N, K, seed):
    g = torch.Generator().manual_seed(seed + 1000)
    return ra.quantize_weight_per_channel(torch.randn(N, K, generator=g) * 0.05)


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K", [(1, 128), (5, 7), (17, 4096), (300, 200), (64, 11008), (9, 8192), (3, 16392)])
def test_quantize_activations_bit_exact(gpu, dt, M, K):
    print(f"  act-quant M={M} K={K} dt={dt}", flush=True)
    x = _acts(M, K, dt, seed=M + K)
    q, xs = qm.quantize_activations(x.to(gpu))
    torch.cuda.synchronize()
    q_ref, xs_ref = oq.quantize_activations_rows(x.float().numpy(), DT[dt])
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(_np(xs), xs_ref)
    assert xs.dtype == dt and q.shape == (M, K)


@pytest.mark.parametrize("c", [100.0, 63.5])
@pytest.mark.parametrize("M,K", [(5, 7), (17, 4096), (3, 16392)])
def test_quantize_activations_other_act_scale(gpu, c, M, K):
    """act_scale other than 127 (quantized_matmul.py:48): bit-exact with the
    oracle, which follows torch's CPU evaluation of the reference's ops."""
    for dt in (torch.float16, torch.bfloat16):
        print(f"  act-quant M={M} K={K} dt={dt} act_scale={c}", flush=True)
        x = _acts(M, K, dt, seed=M + K + 1)
        q, xs = qm.quantize_activations(x.to(gpu), act_scale=c)
        torch.cuda.synchronize()
        q_ref, xs_ref = oq.quantize_activations_rows(x.float().numpy(), DT[dt], act_scale=c)
        np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
        np.testing.assert_array_equal(_np(xs), xs_ref)


def test_quantize_activations_strided_rows(gpu):
    x = _acts(40, 512, torch.float16, seed=5)
    store = torch.zeros(40, 520, dtype=torch.float16, device=gpu)
    store[:, :512] = x.to(gpu)
    print("  act-quant strided M=40 K=512 ld=520", flush=True)
    q, xs = qm.quantize_activations(store[:, :512])
    torch.cuda.synchronize()
    q_ref, xs_ref = oq.quantize_activations_rows(x.float().numpy(), "f16")
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(_np(xs), xs_ref)


# (M, N, K): K % 64 == 0 runs the MFMA kernel (ragged M / N, every tile
# shape; K % 128 == 64 the 64-k stages), the others the any-K kernel.
GEMM_SHAPES = [(17, 128, 128), (64, 256, 96), (300, 320, 256), (256, 192, 512), (513, 129, 1024),
               (1000, 64, 128), (256, 256, 384), (1024, 1024, 256), (300, 200, 192), (64, 256, 320), (252, 192, 256),
               (33, 50, 200), (40, 70, 136)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_w8a8_gemm_bit_exact(gpu, dt, M, N, K):
    print(f"  w8a8 M={M} N={N} K={K} dt={dt}", flush=True)
    x = _acts(M, K, dt, seed=M * 7 + N, edges=False)
    q, s = _weights(N, K, seed=N)
    xq_ref, xs_ref = oq.quantize_activations_rows(x.float().numpy(), DT[dt])
    xq, xs = qm.quantize_activations(x.to(gpu))
    y = qm.w8a8_gemm(xq, xs, q.to(gpu), s.to(gpu))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)
    ref = oq.w8a8_gemm_rows(xq_ref, xs_ref, q.numpy(), s.numpy(), DT[dt])
    np.testing.assert_array_equal(_np(y), ref)


@pytest.mark.parametrize("bias_dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(300, 320, 256), (40, 70, 136)])
def test_w8a8_gemm_bias_bit_exact(gpu, bias_dt, M, N, K):
    print(f"  w8a8 bias={bias_dt} M={M} N={N} K={K}", flush=True)
    x = _acts(M, K, torch.bfloat16, seed=3, edges=False)
    q, s = _weights(N, K, seed=4)
    b = torch.randn(N, generator=torch.Generator().manual_seed(9)).to(bias_dt)
    xq, xs = qm.quantize_activations(x.to(gpu))
    y = qm.w8a8_gemm(xq, xs, q.to(gpu), s.to(gpu), b.to(gpu))
    torch.cuda.synchronize()
    ref = oq.w8a8_gemm_rows(xq.cpu().numpy(), _np(xs), q.numpy(), s.numpy(), "bf16", b.float().numpy())
    np.testing.assert_array_equal(_np(y), ref)


@pytest.mark.parametrize("M,N,K", [(2048, 11008, 4096), (4096, 4096, 512), (8192, 4096, 4096)])
def test_w8a8_full_size_vs_int_mm(gpu, M, N, K):
    """Prefill shapes: bit-exact vs torch._int_mm sums scaled by torch in
    fp32 (separate elementwise kernels, no fused multiply-add), and rows
    against the oracle."""
    print(f"  w8a8 full M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(M + N)
    x = torch.randn(M, K, device=gpu, generator=g).half()
    q = torch.randint(-127, 128, (N, K), device=gpu, generator=g, dtype=torch.int8)
    s = torch.rand(N, device=gpu, generator=g) * 1e-3 + 1e-4
    xq, xs = qm.quantize_activations(x)
    y = qm.w8a8_gemm(xq, xs, q, s)
    acc = torch._int_mm(xq, q.t())
    ref = ((acc.float() * xs.float()[:, None]) * s[None, :]).half()
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    rows = [0, 1, M // 2, M - 1]
    xq_ref, xs_ref = oq.quantize_activations_rows(x[rows].float().cpu().numpy(), "f16")
    np.testing.assert_array_equal(xq[rows].cpu().numpy(), xq_ref)
    np.testing.assert_array_equal(_np(y[rows]),
                                  oq.w8a8_gemm_rows(xq_ref, xs_ref, q.cpu().numpy(), s.cpu().numpy(), "f16"))


def test_w8a8_strided_and_misaligned(gpu):
    """Row strides that keep 16-byte alignment run the MFMA kernel; odd
    strides run the any-K kernel; both equal the contiguous result."""
    M, N, K = 200, 160, 256
    x = _acts(M, K, torch.float16, seed=21, edges=False)
    q, s = _weights(N, K, seed=22)
    xq, xs = qm.quantize_activations(x.to(gpu))
    y0 = qm.w8a8_gemm(xq, xs, q.to(gpu), s.to(gpu))
    for ldx, ldw in ((K + 16, K + 32), (K + 1, K + 3)):
        print(f"  w8a8 strided ldx={ldx} ldw={ldw}", flush=True)
        xs_store = torch.zeros(M, ldx, dtype=torch.int8, device=gpu)
        xs_store[:, :K] = xq
        w_store = torch.zeros(N, ldw, dtype=torch.int8, device=gpu)
        w_store[:, :K] = q.to(gpu)
        y = qm.w8a8_gemm(xs_store[:, :K], xs, w_store[:, :K], s.to(gpu))
        torch.cuda.synchronize()
        assert torch.equal(y, y0)


def _strided_on(gpu, t, ld):
    rows, cols = t.shape
    store = torch.empty((rows - 1) * ld + cols, dtype=t.dtype, device=gpu)
    v = store.as_strided((rows, cols), (ld, 1))
    v.copy_(t.to(gpu))
    return v


def test_w8a8_operands_spanning_more_than_2gib(gpu):
    """Operands whose rows span more than 2^31 bytes are split into row
    chunks (31-bit copy offsets): xq 512 + 88 rows, w 256 + 256 + 88 rows."""
    M, N, K = 600, 600, 256
    x = _acts(M, K, torch.float16, seed=31, edges=False)
    q, s = _weights(N, K, seed=32)
    xq_ref, xs_ref = oq.quantize_activations_rows(x.float().numpy(), "f16")
    print("  w8a8 spanning xq ld=2^22+16 w ld=2^23+16", flush=True)
    xq = _strided_on(gpu, torch.from_numpy(xq_ref), (1 << 22) + 16)
    w = _strided_on(gpu, q, (1 << 23) + 16)
    xs = torch.from_numpy(xs_ref).half().to(gpu)
    y = qm.w8a8_gemm(xq, xs, w, s.to(gpu)).cpu()
    del xq, w
    torch.cuda.empty_cache()
    np.testing.assert_array_equal(_np(y), oq.w8a8_gemm_rows(xq_ref, xs_ref, q.numpy(), s.numpy(), "f16"))


def test_w8a8_deterministic(gpu):
    M, N, K = 2048, 1024, 1024
    print(f"  w8a8 determinism M={M} N={N} K={K}", flush=True)
    x = _acts(M, K, torch.bfloat16, seed=41, edges=False).to(gpu)
    q, s = _weights(N, K, seed=42)
    q, s = q.to(gpu), s.to(gpu)
    ys = [qm.int8_gemm(x, q, s, use_cublas=True) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(ys[0], y) for y in ys[1:])


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_int8_gemm_use_cublas_dispatch(gpu, dt):
    """use_cublas=True with M > 16 is the W8A8 route (bit-exact vs the
    oracle, error near the W8A16 result); M <= 16 or use_cublas=None is the
    W8A16 GEMM."""
    B, S, K, N = 2, 40, 512, 384
    x = _acts(B * S, K, dt, seed=51, edges=False).reshape(B, S, K)
    q, s = _weights(N, K, seed=52)
    b = torch.randn(N, generator=torch.Generator().manual_seed(53)).half()
    print(f"  int8_gemm use_cublas dt={dt}", flush=True)
    xg, qg, sg, bg = x.to(gpu), q.to(gpu), s.to(gpu), b.to(gpu)
    y = qm.int8_gemm(xg, qg, sg, bg, use_cublas=True)
    y16 = qm.int8_gemm(xg, qg, sg, bg)
    small = qm.int8_gemm(xg[:, :8], qg, sg, bg, use_cublas=True)
    torch.cuda.synchronize()
    assert y.shape == (B, S, N) and y.dtype == dt
    xq_ref, xs_ref = oq.quantize_activations_rows(x.reshape(-1, K).float().numpy(), DT[dt])
    ref = oq.w8a8_gemm_rows(xq_ref, xs_ref, q.numpy(), s.numpy(), DT[dt], b.float().numpy())
    np.testing.assert_array_equal(_np(y).reshape(-1, N), ref)
    assert torch.equal(y16, ra.int8_gemm(xg, qg, sg, bg))
    assert torch.equal(small, ra.int8_gemm(xg[:, :8], qg, sg, bg))
    rel = ((y.float() - y16.float()).norm() / y16.float().norm()).item()
    assert rel < 0.05, rel
