"""Seeded synthetic inputs for the W8A16 workloads (tests and bench.py).

Recipe: every tensor is drawn on the CPU from
``g = torch.Generator().manual_seed(seed)`` in a fixed order (activations
first, then weights), then moved to the target device; weights are quantized
per output channel with ``quantize_weight_per_channel`` (bit-exact on CPU and
GPU).

Workloads
---------
plumbing    x fp16 [16,4096] ~N(0,1), W fp32 [4096,4096] ~N(0,0.02), seed 0;
            runs the CPU path (int8_gemm_torch).
decode      M=1, (K,N) in {(4096,4096), (4096,11008), (11008,4096)}, seeds 1-3;
            fp16 x ~N(0,1), W ~N(0,0.02).
smallbatch  M in {4,16,64}, K=4096, N=11008, seeds 4-6; fp16 x ~N(0,1) with
            max(1, round(0.01*M)) randomly chosen rows scaled x20 (outliers).
prefill     (M,K,N) in {(2048,4096,11008), (8192,4096,4096)}, seeds 7-8, fp16.
mlp         bf16 decoder MLP, H=8192, I=28672, M in {1,17,4096}, seeds 9-11:
            x ~N(0,1); RMSNorm weight 1+0.01*N(0,1) (bf16), eps 1e-6;
            Wg, Wu [I,H] and Wd [H,I] ~N(0,0.02), quantized separately;
            [Wg; Wu] concatenated row-wise.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

DECODE_SHAPES = [(1, 4096, 4096, 1), (1, 4096, 11008, 2), (1, 11008, 4096, 3)]   # (M, K, N, seed)
SMALLBATCH_SHAPES = [(4, 4096, 11008, 4), (16, 4096, 11008, 5), (64, 4096, 11008, 6)]
PREFILL_SHAPES = [(2048, 4096, 11008, 7), (8192, 4096, 4096, 8)]
MLP_SHAPES = [(1, 8192, 28672, 9), (17, 8192, 28672, 10), (4096, 8192, 28672, 11)]  # (M, H, I, seed)
PLUMBING_SHAPE = (16, 4096, 4096, 0)

W_STD = 0.02


def _quantize(w: torch.Tensor):
    from rotalabs_accel import quantize_weight_per_channel
    return quantize_weight_per_channel(w)


@dataclass
class GemmCase:
    name: str
    M: int
    K: int
    N: int
    seed: int
    x: torch.Tensor
    q: torch.Tensor
    s: torch.Tensor
    meta: dict = field(default_factory=dict)


def gemm_case(M: int, K: int, N: int, seed: int, device="cpu", dtype=torch.float16,
              outlier_rows: bool = False, name: str = "") -> GemmCase:
    """x ~N(0,1) [M,K] (optionally with 1% outlier rows x20), W ~N(0,0.02) [N,K]
    quantized per channel. Weight is drawn and quantized on ``device``'s side
    of the recipe: generated on CPU, quantized where it lives."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    meta = {}
    if outlier_rows:
        n_out = max(1, round(0.01 * M))
        rows = torch.randperm(M, generator=g)[:n_out]
        x[rows] *= 20.0
        meta["outlier_rows"] = rows.tolist()
    w = torch.randn(N, K, generator=g) * W_STD
    x = x.to(dtype).to(device)
    q, s = _quantize(w.to(device))
    return GemmCase(name or f"M{M}_K{K}_N{N}", M, K, N, seed, x, q, s, meta)


@dataclass
class MlpCase:
    M: int
    H: int
    I: int
    seed: int
    x: torch.Tensor
    norm_w: torch.Tensor
    q_gu: torch.Tensor
    s_gu: torch.Tensor
    q_d: torch.Tensor
    s_d: torch.Tensor


def mlp_case(M: int, H: int, I: int, seed: int, device="cpu", dtype=torch.bfloat16) -> MlpCase:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, H, generator=g).to(dtype).to(device)
    norm_w = (1.0 + 0.01 * torch.randn(H, generator=g)).to(dtype).to(device)
    qg, sg = _quantize((torch.randn(I, H, generator=g) * W_STD).to(device))
    qu, su = _quantize((torch.randn(I, H, generator=g) * W_STD).to(device))
    q_gu = torch.cat([qg, qu], 0)
    s_gu = torch.cat([sg, su], 0)
    del qg, qu
    qd, sd = _quantize((torch.randn(H, I, generator=g) * W_STD).to(device))
    return MlpCase(M, H, I, seed, x, norm_w, q_gu, s_gu, qd, sd)


def gemm_bytes(M: int, K: int, N: int, x_bytes: int = 2, bias: bool = False) -> int:
    """Algorithmic HBM bytes of one W8A16 GEMM: int8 W, fp32 scale, x in, y out."""
    return N * K + 4 * N + x_bytes * M * K + x_bytes * M * N + (x_bytes * N if bias else 0)


def gemm_flops(M: int, K: int, N: int) -> int:
    return 2 * M * N * K


def mlp_bytes(M: int, H: int, I: int, x_bytes: int = 2) -> int:
    """RMSNorm (x in, h out, weight) + gate/up (W, scales, h in, act out) +
    down (W, scales, act in, y out)."""
    norm = 2 * x_bytes * M * H + x_bytes * H
    gateup = 2 * I * H + 8 * I + x_bytes * M * H + x_bytes * M * I
    down = H * I + 4 * H + x_bytes * M * I + x_bytes * M * H
    return norm + gateup + down


def mlp_flops(M: int, H: int, I: int) -> int:
    return 2 * M * H * (2 * I) + 2 * M * I * H
