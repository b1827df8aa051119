"""GPU parity of the W8A16 GEMM kernels (through the C ABI).

* Exact known answers: integer activations and weights with small sums, so
  every partial sum and the rounded output are exact and any indexing
  mistake shows up as a mismatch -- for every kernel variant.
* Tolerance vs the oracle (the reference fallback restated on the CPU,
  rtol = atol = 1e-2) and vs a float64 reference (tighter, per dtype).
* Full-size workloads vs an fp32 torch reference on the GPU, plus rows
  re-checked against the float64 oracle on the CPU.
* Determinism, bias dtypes, strides / misalignment, K tails, graph replay.
"""
import numpy as np
import pytest
import torch

import rotalabs_accel as ra
from oracle import fallback
from rotalabs_accel import _backend
from rotalabs_accel.kernels.gemm import _int8_gemm_hip
from workloads import DECODE_SHAPES, PREFILL_SHAPES, SMALLBATCH_SHAPES, gemm_case

pytestmark = pytest.mark.gpu

SKINNY, TILED, GENERIC, GEMV, ROWS, BATCH, SPLITK = (_backend.VARIANT_SKINNY, _backend.VARIANT_TILED,
                                                     _backend.VARIANT_GENERIC, _backend.VARIANT_GEMV,
                                                     _backend.VARIANT_ROWS, _backend.VARIANT_BATCH,
                                                     _backend.VARIANT_SPLITK)
ALL_VARIANTS = (ROWS, GEMV, BATCH, SPLITK, SKINNY, TILED, GENERIC)


def _may_refuse(v, M, K):
    """The variants that cover only part of the shape space (RA_ERR_VARIANT)."""
    return ((v == GEMV and M > 4) or (v == ROWS and M > 2) or
            (v in (BATCH, SPLITK) and (M > 64 or K % 128 != 0)))

# fp64 tolerance per output dtype: ~2 ulp relative + accumulation noise
TOL64 = {torch.float16: (2e-3, 2e-3), torch.bfloat16: (8e-3, 8e-3), torch.float32: (1e-5, 1e-4)}


def _run(x, q, s, bias=None, variant=_backend.VARIANT_AUTO):
    """One GEMM through the C ABI; None if a forced variant reports that it
    cannot run this shape (RA_ERR_VARIANT)."""
    print(f"  gemm M={x.reshape(-1, x.shape[-1]).shape[0]} K={x.shape[-1]} N={q.shape[0]} "
          f"dt={x.dtype} variant={variant}", flush=True)
    try:
        y = _int8_gemm_hip(x, q, s, bias, variant)
    except RuntimeError as e:
        if variant != _backend.VARIANT_AUTO and "variant cannot run" in str(e):
            return None
        raise
    torch.cuda.synchronize()
    return y


def _exact_case(M, K, N, dt, seed, dev, bias=False):
    """Integer x in {-1,0,1}, q in [-lim, lim], scale 2^-4 (exact), optional
    integer bias * 2^-4: |sum| stays small enough to be exact in dt."""
    g = torch.Generator().manual_seed(seed)
    lim = 3 if dt == torch.float16 else 1
    x = torch.randint(-1, 2, (M, K), generator=g).float()
    if dt == torch.bfloat16:   # keep |sum| <= 255: at most 127 nonzeros per row
        keep = torch.rand(M, K, generator=g) < min(1.0, 127.0 / K)
        x = x * keep
    q = torch.randint(-lim, lim + 1, (N, K), generator=g).to(torch.int8)
    s = torch.full((N,), 2.0 ** -4)
    b = (torch.randint(-8, 9, (N,), generator=g).float() * 2.0 ** -4) if bias else None
    exact = (x.double() @ q.double().T) * 2.0 ** -4
    if b is not None:
        exact = exact + b.double()
    return (x.to(dt).to(dev), q.to(dev), s.to(dev), None if b is None else b.to(dt).to(dev), exact)


EXACT_SHAPES = [
    (1, 64, 16), (1, 48, 43), (2, 4096, 64), (2, 1008, 8202), (2, 2048, 4100), (1, 11008, 40), (3, 128, 77),
    (1, 4096, 4101), (1, 5120, 37), (1, 16400, 300), (1, 6144, 11003),
    (16, 1040, 33),
    (17, 64, 130), (33, 96, 50), (64, 256, 96), (65, 256, 300), (256, 128, 128), (300, 320, 200),
    (513, 1024, 129), (1000, 64, 17),
]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", EXACT_SHAPES)
def test_exact_known_answer_all_variants(gpu, M, K, N, dt):
    x, q, s, b, exact = _exact_case(M, K, N, dt, seed=M * 7 + K + N, dev=gpu, bias=(M % 2 == 1))
    want = exact.to(dt)
    ran = 0
    for v in ALL_VARIANTS:
        y = _run(x, q, s, b, v)
        if y is None:
            assert _may_refuse(v, M, K), f"variant {v} refused M={M} K={K}"
            continue
        y = y.cpu()
        ran += 1
        assert y.dtype == dt
        assert torch.equal(y, want), f"variant {v}: {(y.double() - exact).abs().max()}"
    assert ran >= 3
    # every variant that covers the shape ran (none refused it wrongly)
    assert ran == sum(not _may_refuse(v, M, K) for v in ALL_VARIANTS)


# Wide N: the small-batch kernel takes 32 or 48 weight rows per workgroup
# (RT = 2, 3) and splits K over 8 waves, K slices of 128 to 640; K = 1152
# leaves three of the eight waves without a slice, K = 128 all but one.
WIDE_BATCH_SHAPES = [(4, 1152, 11008), (16, 128, 8000), (33, 4096, 11008), (64, 1024, 6000), (20, 640, 9000)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", WIDE_BATCH_SHAPES)
def test_exact_known_answer_wide_batch(gpu, M, K, N, dt):
    x, q, s, b, exact = _exact_case(M, K, N, dt, seed=M + K + N, dev=gpu, bias=(K % 256 == 128))
    print(f"  wide batch M={M} K={K} N={N} {dt}", flush=True)
    want = exact.to(dt)
    for v in (_backend.VARIANT_AUTO, BATCH, SPLITK):
        y = _run(x, q, s, b, v).cpu()
        assert torch.equal(y, want), f"variant {v}: {(y.double() - exact).abs().max()}"


# Shapes the small-batch kernel with the activation rows resident in LDS
# takes (M <= 16, K = 2048 .. 4096 in steps of 512, K / 512 waves shared
# equally by the workgroup's 16-row weight tiles, at most one workgroup per
# CU): 1, 2, 3, 4, 6 or 8 tiles per workgroup, 1 to 7 K parts per tile (a
# single part at 6 and 8 tiles), 2 or 4 stages in flight, M from 1 to 16, N
# tails inside a tile and a half-filled last tile.
XLDS_SHAPES = [(1, 2048, 16), (2, 4096, 64), (3, 3072, 77), (5, 4096, 11008), (8, 2560, 4000), (13, 2048, 300),
               (16, 4096, 11008), (16, 3584, 4096), (11, 2048, 8193), (16, 2048, 14000), (7, 3072, 12000),
               (6, 4096, 6000), (16, 3072, 9000), (2, 4096, 28672), (16, 4096, 20000), (9, 3072, 24000)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", XLDS_SHAPES)
def test_exact_known_answer_xlds(gpu, M, K, N, dt):
    x, q, s, b, exact = _exact_case(M, K, N, dt, seed=3 * M + K + N, dev=gpu, bias=(N % 2 == 0))
    print(f"  activation-resident batch M={M} K={K} N={N} {dt}", flush=True)
    want = exact.to(dt)
    y = _run(x, q, s, b, BATCH).cpu()
    assert torch.equal(y, want), f"max err {(y.double() - exact).abs().max()}"
    # twice in a row: nothing carried over between launches
    y2 = _run(x, q, s, b, BATCH).cpu()
    assert torch.equal(y2, y)


@pytest.mark.parametrize("bdt", [torch.float16, torch.bfloat16, torch.float32])
def test_xlds_strides_and_bias_dtypes(gpu, bdt):
    """The activation-resident kernel with row strides on both operands
    (ldx = K + 8, ldw = K + 48: the copies and loads address each row), a
    bias in each dtype, and a 2-byte-misaligned activation base."""
    M, K, N = 16, 4096, 4100
    x, q, s, _, exact = _exact_case(M, K, N, torch.float16, seed=41, dev="cpu")
    g = torch.Generator().manual_seed(42)
    b = torch.randint(-8, 9, (N,), generator=g).float() * 2.0 ** -4      # exact in every bias dtype
    want = (exact + b.double()).to(torch.float16)
    xs = _strided_on(gpu, x, K + 8)
    ws = _strided_on(gpu, q, K + 48)
    y = _run(xs, ws, s.to(gpu), b.to(bdt).to(gpu), BATCH).cpu()
    assert torch.equal(y, want), f"max err {(y.double() - exact - b.double()).abs().max()}"
    flat = torch.zeros(M * K + 1, dtype=torch.float16, device=gpu)
    flat[1:] = x.reshape(-1).to(gpu)
    x_mis = flat[1:].view(M, K)
    for v in (BATCH, _backend.VARIANT_AUTO):
        y2 = _run(x_mis, q.to(gpu), s.to(gpu), b.to(bdt).to(gpu), v).cpu()
        assert torch.equal(y2, want)


# The tiled kernel's 64 x 64 tile (M <= 64; chosen automatically for
# M = 33..64 with >= 8192 weight rows): M tails inside the tile, N tails,
# short and long K, bias.
SMALL_TILE_SHAPES = [(33, 4096, 11008), (64, 4096, 11008), (50, 2048, 8200), (64, 128, 8192), (40, 576, 9000),
                     (17, 1024, 300), (1, 64, 64)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", SMALL_TILE_SHAPES)
def test_exact_known_answer_small_tile(gpu, M, K, N, dt):
    x, q, s, b, exact = _exact_case(M, K, N, dt, seed=5 * M + K + N, dev=gpu, bias=(M % 2 == 0))
    print(f"  64x64 tiles M={M} K={K} N={N} {dt}", flush=True)
    want = exact.to(dt)
    for v in (TILED, _backend.VARIANT_AUTO):
        y = _run(x, q, s, b, v).cpu()
        assert torch.equal(y, want), f"variant {v}: {(y.double() - exact).abs().max()}"


# M = 33..64 shapes whose plan splits K over workgroups or widens the tile
# (64 x 64*bnb tiles, nsplit splits; bnb/nsplit from the plan at 256 CUs):
# 2/4, 2/3, 3/4, 3/2, 3/1, 2/2, 2/1, 1/2 -- K tiles not a multiple of the
# split count, N tails, the partial sums of up to four splits combined.
SPLIT_TILE_SHAPES = [(57, 9216, 8192), (64, 8192, 9000), (50, 6144, 12000), (64, 4096, 16500), (56, 1024, 40000),
                     (60, 4096, 16384), (40, 2048, 24000), (64, 6144, 8192),
                     # M = 65..128: two rows of 64-row tiles or one row of 128-row tiles (ragged M
                     # and N; 128 x 128 and 128 x 192 tiles with and without K splits)
                     (65, 2048, 4096), (100, 11008, 4096), (128, 4096, 8200), (80, 6144, 9000), (97, 1024, 3000),
                     (65, 8192, 16000), (90, 12288, 7000), (65, 1024, 32000), (128, 12288, 12000),
                     # M = 129..1024, where the large tiles leave CUs idle
                     (129, 8192, 5000), (200, 4096, 4096), (256, 2048, 8192), (250, 11008, 4100),
                     (300, 2048, 8192), (384, 8192, 8200), (700, 4096, 4096), (1000, 2048, 4000)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", SPLIT_TILE_SHAPES)
def test_exact_known_answer_split_tile(gpu, M, K, N, dt):
    """The small tile with K split over workgroups, their fp32 partial sums
    combined in the workspace: exact known answers, forced and automatic
    (two calls in a row: a tile counter left non-zero would leave the second
    call's tiles unwritten)."""
    lib = _backend.load()
    assert lib.ra_w8a16_gemm_select(M, N, K, _backend.dtype_code(dt)) == TILED
    x, q, s, b, exact = _exact_case(M, K, N, dt, seed=7 * M + K + N, dev=gpu, bias=(N % 2 == 0))
    print(f"  split tiles M={M} K={K} N={N} {dt} workspace "
          f"{lib.ra_w8a16_gemm_workspace_size(M, N, K, _backend.dtype_code(dt))} B", flush=True)
    want = exact.to(dt)
    for v in (TILED, _backend.VARIANT_AUTO):
        y = _run(x, q, s, b, v).cpu()
        assert torch.equal(y, want), f"variant {v}: {(y.double() - exact).abs().max()}"


def test_exact_fp32_activations(gpu):
    x, q, s, b, exact = _exact_case(9, 200, 70, torch.float32, seed=5, dev=gpu, bias=True)
    y = _run(x, q, s, b).cpu()
    assert y.dtype == torch.float32 and torch.equal(y.double(), exact)


UNIT_ROUNDOFF = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -24}


def _oracle_check(y, x_cpu, q_cpu, s_cpu, b_cpu=None):
    """Parity of a kernel output y (CPU tensor) on CPU-sized problems.

    1. Against the fp32-accumulated dequantize-then-matmul reference (float64
       here; weights = the fp32 products q*s that dequantize forms before its
       final cast): rtol = atol = 1e-2, and a tighter per-dtype bound.
    2. Against the reference fallback's exact bits (oracle): the same
       rtol = atol = 1e-2 plus the fallback's own provable error from rounding
       the dequantized weights to x.dtype, u * (|x| @ |w|^T).
    """
    xn = x_cpu.float().numpy()
    y64 = fallback.gemm_f64(xn, q_cpu.numpy(), s_cpu.numpy(), None if b_cpu is None else b_cpu.float().numpy())
    yd = y.double().numpy()
    err = np.abs(yd - y64)
    assert (err <= 1e-2 + 1e-2 * np.abs(y64)).all(), f"max err {err.max()} vs fp32-accumulated reference"
    rtol, atol = TOL64[y.dtype]
    assert (err <= atol + rtol * np.abs(y64)).all(), f"max err {err.max()} above the {y.dtype} bound"
    y_fb = fallback.int8_gemm_ref(x_cpu, q_cpu, s_cpu, b_cpu).double().numpy()
    w_dt = fallback.dequantize_ref(q_cpu, s_cpu, x_cpu.dtype).double().numpy()
    slack = UNIT_ROUNDOFF[x_cpu.dtype] * (np.abs(xn.astype(np.float64)) @ np.abs(w_dt).T)
    err_fb = np.abs(yd - y_fb)
    assert (err_fb <= 1e-2 + 1e-2 * np.abs(y_fb) + slack).all(), f"max err vs fallback {err_fb.max()}"


TOL_SHAPES = [(1, 1024, 512), (2, 3072, 8200), (4, 2048, 1024), (48, 1024, 13000), (20, 2048, 9000), (16, 4096, 1024), (17, 1024, 777), (64, 1024, 2048),
              (100, 512, 384), (256, 1024, 1024), (512, 2048, 640)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", TOL_SHAPES)
def test_random_vs_oracle(gpu, M, K, N, dt):
    c = gemm_case(M, K, N, seed=M + K + N, dtype=dt, outlier_rows=True)
    g = torch.Generator().manual_seed(99)
    b = (torch.randn(N, generator=g) * 0.1).to(dt)
    for v in (_backend.VARIANT_AUTO, ROWS, GEMV, BATCH, SPLITK, SKINNY, TILED):
        y = _run(c.x.to(gpu), c.q.to(gpu), c.s.to(gpu), b.to(gpu), v)
        if y is None:
            assert _may_refuse(v, M, K)
            continue
        _oracle_check(y.cpu(), c.x, c.q, c.s, b)


def _full_size_check(c, gpu):
    """Full-size parity on the GPU: the reference is a float64 torch matmul
    (at least as accurate as fp32 accumulation) of x and the fp32-dequantized
    weight; the fallback's bits are bounded as in _oracle_check; a few rows
    are re-checked against the float64 oracle on the CPU."""
    x, q, s = c.x.to(gpu), c.q.to(gpu), c.s.to(gpu)
    y = _run(x, q, s)
    w32 = q.float() * s[:, None]
    y32 = (x.double() @ w32.double().t().contiguous()).float()
    err = (y.float() - y32).abs()
    assert bool((err <= 1e-2 + 1e-2 * y32.abs()).all()), f"max err {err.max().item()}"
    rtol, atol = TOL64[x.dtype]
    assert bool((err <= atol + rtol * y32.abs()).all()), f"max err {err.max().item()} above the {x.dtype} bound"
    w_dt = w32.to(x.dtype).float()
    y_fb = (x.double() @ w_dt.double().t().contiguous()).float()   # fallback arithmetic, exact accumulation
    slack = UNIT_ROUNDOFF[x.dtype] * (x.float().abs() @ w_dt.abs().t().contiguous())
    err_fb = (y.float() - y_fb).abs()
    assert bool((err_fb <= 1e-2 + 1e-2 * y_fb.abs() + slack).all())
    del w32, w_dt
    rows = sorted(set([0, c.M - 1, c.M // 2] + c.meta.get("outlier_rows", [])))[:8]
    y64 = fallback.gemm_f64(c.x[rows].float().cpu().numpy(), c.q.cpu().numpy(), c.s.cpu().numpy())
    np.testing.assert_allclose(y[rows].double().cpu().numpy(), y64, rtol=rtol, atol=atol)


@pytest.mark.parametrize("M,K,N,seed", DECODE_SHAPES)
def test_decode_full_size(gpu, M, K, N, seed):
    _full_size_check(gemm_case(M, K, N, seed, device=gpu), gpu)


@pytest.mark.parametrize("M,K,N,seed", SMALLBATCH_SHAPES)
def test_smallbatch_full_size(gpu, M, K, N, seed):
    _full_size_check(gemm_case(M, K, N, seed, device=gpu, outlier_rows=True), gpu)


@pytest.mark.parametrize("M,K,N,seed", PREFILL_SHAPES)
def test_prefill_full_size(gpu, M, K, N, seed):
    _full_size_check(gemm_case(M, K, N, seed, device=gpu), gpu)


# Shapes for which the tiled kernel picks each of its tile geometries
# (per-wave 32x32 blocks (4,2), (4,3), (3,4), (4,4); one workgroup per CU on
# 256 CUs), with M and N tails; short K keeps them fast.
TILE_SHAPES = [(300, 192, 4096), (576, 256, 11264), (640, 128, 16384), (832, 128, 13312), (1000, 320, 13000)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", TILE_SHAPES)
def test_tiled_tile_geometries(gpu, M, K, N, dt):
    _full_size_check(gemm_case(M, K, N, seed=M + N, device=gpu, dtype=dt), gpu)


# Split-K small-batch shapes: many splits (long K, few rows), N tails, one
# stage per split, every activation-tile count (M <= 16, 32, 64), two rows,
# the small-batch (K=4096 N=11008) and MLP down-projection shapes, and
# M = 17 / 33 at K >= 16384 (the last row summed on the VALU beside the
# MFMA tiles).
SPLITK_SHAPES = [(3, 4096, 11008), (16, 4096, 11008), (64, 4096, 11008), (8, 8192, 256), (17, 8192, 300),
                 (33, 1024, 1000), (64, 128, 64), (5, 28672, 8192), (20, 2048, 77), (40, 512, 3000),
                 (2, 16384, 700), (17, 16384, 1000), (33, 16384, 520), (17, 28672, 300)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", SPLITK_SHAPES)
def test_splitk_exact_and_repeated(gpu, M, K, N, dt):
    """The split-K small-batch kernel: exact known answers (integer sums, so
    any split, order or indexing mistake is a mismatch), then two calls in a
    row on different inputs against the oracle bound (a counter left
    non-zero by the first call would leave the second's output unwritten),
    and bitwise repeatable."""
    lib = _backend.load()
    ws_need = lib.ra_w8a16_gemm_workspace_size(M, N, K, _backend.dtype_code(dt))
    print(f"  split-K M={M} K={K} N={N} {dt} workspace {ws_need} B", flush=True)
    x, q, s, b, exact = _exact_case(M, K, N, dt, seed=M + K + N, dev=gpu, bias=(N % 2 == 0))
    for v in (SPLITK, _backend.VARIANT_SPLITK_SPREAD):   # a row block's splits on one XCD / on several
        y = _run(x, q, s, b, v).cpu()
        assert torch.equal(y, exact.to(dt)), f"variant {v}: max err {(y.double() - exact).abs().max()}"
    for seed in (1, 2):
        c = gemm_case(M, K, N, seed=seed * 1000 + M, dtype=dt, outlier_rows=True)
        y1 = _run(c.x.to(gpu), c.q.to(gpu), c.s.to(gpu), None, SPLITK)
        y2 = _run(c.x.to(gpu), c.q.to(gpu), c.s.to(gpu), None, SPLITK)
        assert torch.equal(y1, y2)
        if K * N <= 4096 * 11008 and M * K * N <= 64 * 4096 * 11008:
            _oracle_check(y1.cpu(), c.x, c.q, c.s)


# Shapes where the automatic pick is not the default kernel of the M range:
# M = 1 at short K (small-batch / skinny kernels instead of the row GEMV),
# M = 33..56 at short K (small-batch kernel instead of the 64-row tiles), and
# M = 17..32 at K <= 4096 over 28672+ rows (the split-K kernel without a
# split). N tails included.
SELECTION_RULE_SHAPES = [(1, 2048, 16384), (1, 1024, 16390), (1, 512, 4100), (33, 2048, 8192), (40, 3072, 12000),
                         (48, 1024, 11008), (56, 2048, 8190), (24, 2048, 28672), (32, 4096, 28700), (17, 4096, 28672)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", SELECTION_RULE_SHAPES)
def test_selection_rule_shapes_exact_and_oracle(gpu, M, K, N, dt):
    """The automatic pick at these shapes: exact known answers (with a
    workspace and without one: the same kernel, bitwise the same output),
    then a random case against the oracle bound."""
    lib = _backend.load()
    sel = lib.ra_w8a16_gemm_select(M, N, K, _backend.dtype_code(dt))
    print(f"  rule shape M={M} K={K} N={N} {dt}: variant {sel}", flush=True)
    assert sel != _backend.VARIANT_ROWS or M == 1
    x, q, s, b, exact = _exact_case(M, K, N, dt, seed=M + K + N, dev=gpu, bias=(N % 2 == 0))
    y = _run(x, q, s, b, 0).cpu()
    assert torch.equal(y, exact.to(dt)), f"max err {(y.double() - exact).abs().max()}"
    c = gemm_case(M, K, N, seed=M + 3, dtype=dt, outlier_rows=M > 1)
    xg, qg, sg = c.x.to(gpu), c.q.to(gpu), c.s.to(gpu)
    y1 = ra.int8_gemm(xg, qg, sg)
    out = torch.empty_like(y1)
    code = lib.ra_w8a16_gemm(xg.data_ptr(), K, _backend.dtype_code(dt), qg.data_ptr(), K, sg.data_ptr(), None,
                             _backend.F32, out.data_ptr(), N, M, N, K, _backend.stream_handle(gpu))
    torch.cuda.synchronize()
    assert code == 0
    assert torch.equal(y1, out), "with and without a workspace"
    _oracle_check(y1.cpu(), c.x, c.q, c.s)


# Shapes the split-K selection rules send to the split-K kernel (M = 2..32 from
# K = 5120 over 14336+ rows, at any M from K = 11008, from 16 rows at K = 8192,
# from 24 rows, from 28 rows over at most 4096 rows from K = 3072; M = 33..48
# over many rows; M = 49..64 below 8192 rows from K = 3072 and over many rows;
# M = 33..64 up to 48 rows from K = 8192, from K = 14336, over at
# most 4096 rows from K = 4096; K >= 16384), with the plans the time model
# picks there.
SPLITK_RULE_SHAPES = [(2, 5120, 14400), (16, 11008, 6000), (24, 5120, 4000), (32, 5120, 6000), (40, 4096, 4000),
                      (48, 14336, 5000), (4, 16384, 4800), (64, 4096, 4096), (3, 11008, 2000), (16, 8192, 5000),
                      (40, 8192, 9000), (30, 3072, 4000), (33, 1024, 30000), (33, 5120, 6200), (40, 4096, 6200),
                      (36, 3072, 2000), (60, 3072, 6000), (52, 2048, 30000), (24, 4096, 16000),
                      (6, 8192, 1500)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", SPLITK_RULE_SHAPES)
def test_splitk_rule_shapes_exact_and_oracle(gpu, M, K, N, dt):
    """The automatic pick is the split-K kernel: exact known answers
    (automatic and forced), then two calls in a row on random inputs,
    bitwise repeatable and, where the oracle is quick, within its bound."""
    lib = _backend.load()
    assert lib.ra_w8a16_gemm_select(M, N, K, _backend.dtype_code(dt)) == SPLITK
    print(f"  split-K rule M={M} K={K} N={N} {dt} workspace "
          f"{lib.ra_w8a16_gemm_workspace_size(M, N, K, _backend.dtype_code(dt))} B", flush=True)
    x, q, s, b, exact = _exact_case(M, K, N, dt, seed=3 * M + K + N, dev=gpu, bias=(N % 2 == 0))
    for v in (0, SPLITK):
        y = _run(x, q, s, b, v).cpu()
        assert torch.equal(y, exact.to(dt)), f"variant {v}: max err {(y.double() - exact).abs().max()}"
    c = gemm_case(M, K, N, seed=M + 11, dtype=dt, outlier_rows=True)
    xg, qg, sg = c.x.to(gpu), c.q.to(gpu), c.s.to(gpu)
    y1 = _run(xg, qg, sg, None, 0)
    y2 = _run(xg, qg, sg, None, 0)
    assert torch.equal(y1, y2)
    if K * N <= 4096 * 11008 and M * K * N <= 64 * 4096 * 11008:
        _oracle_check(y1.cpu(), c.x, c.q, c.s)


def test_splitk_plans_share_one_workspace(gpu):
    """Calls with different split plans (58 row blocks x 4 splits, then 94 x
    2, then 4 x 16) on one stream share its workspace: the counters sit in a
    fixed region that no plan's partial sums overwrite, so every call finds
    them at zero."""
    for (M, K, N) in [(33, 4096, 11008), (64, 1024, 6000), (8, 8192, 256), (33, 4096, 11008)]:
        x, q, s, b, exact = _exact_case(M, K, N, torch.float16, seed=M + K + N, dev=gpu)
        y = _run(x, q, s, b, SPLITK).cpu()
        assert torch.equal(y, exact.to(torch.float16)), f"M={M} K={K} N={N}"


def test_splitk_selected_for_long_k():
    """M = 3..64 with K >= 16384 run the split-K kernel with S > 1 (a
    workspace): the MLP's down projection at M=17 (K=28672 N=8192)."""
    lib = _backend.load()
    assert lib.ra_w8a16_gemm_select(17, 8192, 28672, _backend.BF16) == SPLITK
    assert lib.ra_w8a16_gemm_workspace_size(17, 8192, 28672, _backend.BF16) > 0
    for M in (3, 16, 32):
        assert lib.ra_w8a16_gemm_select(M, 11008, 4096, _backend.F16) == BATCH
    # M = 33..64 with >= 8192 weight rows: the tiled kernel's 64 x 64 tile
    for M in (49, 64):
        assert lib.ra_w8a16_gemm_select(M, 11008, 4096, _backend.F16) == TILED
    # M = 33..48: split K (three 16-row tiles, or two and the extra row on the VALU)
    for M in (33, 40, 48):
        assert lib.ra_w8a16_gemm_select(M, 11008, 4096, _backend.F16) == SPLITK
    # from 24 rows over at most 4096 weight rows: split K (M = 64 from K = 4096)
    assert lib.ra_w8a16_gemm_select(64, 4096, 4096, _backend.F16) == SPLITK
    assert lib.ra_w8a16_gemm_select(24, 4096, 4096, _backend.F16) == BATCH


def test_two_rows_take_the_small_batch_kernels():
    """M = 2 runs the small-batch kernels wherever they apply (K % 128 == 0;
    split K from K = 11008, with a workspace from K = 16384), the row GEMV
    where they do not and over few weight rows; M = 1 the row GEMV."""
    lib = _backend.load()
    assert lib.ra_w8a16_gemm_select(2, 11008, 4096, _backend.F16) == BATCH
    assert lib.ra_w8a16_gemm_select(2, 4096, 2048, _backend.BF16) == BATCH
    assert lib.ra_w8a16_gemm_select(2, 4096, 8192, _backend.F16) == BATCH
    assert lib.ra_w8a16_gemm_select(2, 4096, 11008, _backend.F16) == SPLITK
    assert lib.ra_w8a16_gemm_select(2, 4096, 1024, _backend.F16) == BATCH
    assert lib.ra_w8a16_gemm_select(2, 8192, 28672, _backend.BF16) == SPLITK
    assert lib.ra_w8a16_gemm_select(2, 4096, 1040, _backend.F16) == ROWS
    assert lib.ra_w8a16_gemm_select(2, 1024, 8192, _backend.F16) == ROWS   # few rows
    assert lib.ra_w8a16_gemm_select(1, 11008, 4096, _backend.F16) == ROWS
    assert lib.ra_w8a16_gemm_select(1, 8192, 28672, _backend.F16) == ROWS
    assert lib.ra_w8a16_gemm_workspace_size(2, 8192, 28672, _backend.BF16) > 0
    assert lib.ra_w8a16_gemm_workspace_size(1, 8192, 28672, _backend.BF16) == 0


@pytest.mark.parametrize("M", [1, 16, 2048])
def test_deterministic(gpu, M):
    c = gemm_case(M, 4096, 4096, seed=21, device=gpu)
    a = _run(c.x, c.q, c.s)
    b = _run(c.x, c.q, c.s)
    assert torch.equal(a, b)


@pytest.mark.parametrize("bdt", [torch.float16, torch.bfloat16, torch.float32])
def test_bias_dtypes(gpu, bdt):
    c = gemm_case(8, 512, 256, seed=3)
    b = torch.randn(256) * 0.5
    y = _run(c.x.to(gpu), c.q.to(gpu), c.s.to(gpu), b.to(bdt).to(gpu)).cpu()
    ref = fallback.gemm_f64(c.x.float().numpy(), c.q.numpy(), c.s.numpy(), b.to(bdt).float().numpy())
    np.testing.assert_allclose(y.double().numpy(), ref, rtol=2e-3, atol=2e-3)


def test_bias_shapes(gpu):
    """Bias shapes the reference's broadcast add (y + bias, gemm.py:181-182)
    accepts: a scalar and a one-element bias are expanded to [N] for the
    kernels, (1, N) goes to the kernels, (M, N) and (M, 1) are added after
    the GEMM; a shape that does not broadcast raises (as y + bias does);
    the W8A8 route takes the same shapes."""
    from rotalabs_accel.kernels import quantized_matmul as qm
    M, K, N = 24, 512, 200
    c = gemm_case(M, K, N, seed=21)
    x, q, s = c.x.to(gpu), c.q.to(gpu), c.s.to(gpu)
    y0 = ra.int8_gemm(x, q, s).float()
    xq, xs = qm.quantize_activations(x)
    w0 = qm.w8a8_gemm(xq, xs, q, s).float()
    g = torch.Generator().manual_seed(3)
    for shape in [(), (1,), (1, N), (M, N), (M, 1)]:
        b = (torch.randn(shape, generator=g) * 0.5).half().to(gpu)
        print(f"  bias shape {shape}", flush=True)
        y = ra.int8_gemm(x, q, s, b)
        torch.cuda.synchronize()
        assert y.shape == (M, N) and y.dtype == torch.float16
        torch.testing.assert_close(y.float(), (y0 + b.float()).half().float(), rtol=2e-3, atol=2e-3)
        w = qm.w8a8_gemm(xq, xs, q, s, b)
        torch.testing.assert_close(w.float(), (w0 + b.float()).half().float(), rtol=2e-3, atol=2e-3)
    for bad in [(N + 1,), (N - 1,), (M + 1, N)]:
        b = torch.zeros(bad, dtype=torch.float16, device=gpu)
        with pytest.raises(RuntimeError):
            ra.int8_gemm(x, q, s, b)


def test_strided_and_misaligned_inputs(gpu):
    c = gemm_case(24, 512, 200, seed=8)
    xb = torch.zeros(24, 520, dtype=torch.float16)
    xb[:, 8:] = c.x
    x_strided = xb.to(gpu)[:, 8:]                      # row stride 520, 16-B aligned start
    y1 = ra.int8_gemm(x_strided, c.q.to(gpu), c.s.to(gpu)).cpu()
    flat = torch.zeros(24 * 512 + 1, dtype=torch.float16)
    flat[1:] = c.x.reshape(-1)
    x_mis = flat.to(gpu)[1:].view(24, 512)            # 2-byte misaligned base
    y2 = ra.int8_gemm(x_mis, c.q.to(gpu), c.s.to(gpu)).cpu()
    x_t = c.x.t().contiguous().to(gpu).t()              # column-major
    y3 = ra.int8_gemm(x_t, c.q.to(gpu), c.s.to(gpu)).cpu()
    ref = ra.int8_gemm(c.x.to(gpu), c.q.to(gpu), c.s.to(gpu)).cpu()
    assert torch.equal(y1, ref) and torch.equal(y2, ref) and torch.equal(y3, ref)
    # odd K (not a multiple of 16) runs the generic kernel
    c2 = gemm_case(5, 50, 37, seed=9)
    y4 = ra.int8_gemm(c2.x.to(gpu), c2.q.to(gpu), c2.s.to(gpu)).cpu()
    _oracle_check(y4, c2.x, c2.q, c2.s)


def _strided_on(gpu, t, ld):
    """A (rows, cols) view of t on the GPU with row stride ld elements."""
    rows, cols = t.shape
    store = torch.empty((rows - 1) * ld + cols, dtype=t.dtype, device=gpu)
    v = store.as_strided((rows, cols), (ld, 1))
    v.copy_(t.to(gpu))
    return v


def test_operands_spanning_more_than_2gib(gpu):
    """Activations and weights whose rows span more than 2^31 bytes: the
    prefill kernel addresses its copies through 31-bit offsets, so such
    operands are split into row chunks, one launch each (x: 512 + 88 rows,
    W: 256 + 256 + 88 rows)."""
    M, K, N = 600, 256, 600
    c = gemm_case(M, K, N, seed=11)
    x = _strided_on(gpu, c.x, (1 << 21) + 64)     # 4 MiB per activation row, ~2.5 GB
    w = _strided_on(gpu, c.q, (1 << 23) + 16)     # 8 MiB per weight row, ~5 GB
    y = _run(x, w, c.s.to(gpu)).cpu()
    del x, w
    torch.cuda.empty_cache()
    _oracle_check(y, c.x, c.q, c.s)


def test_gateup_weights_spanning_more_than_2gib(gpu):
    """A gate/up weight pair spanning more than 2^31 bytes runs the
    register-staged kernel (64-bit addresses) and matches the unfused path."""
    M, K, inter = 300, 256, 300
    g = torch.Generator().manual_seed(12)
    x = torch.randn(M, K, generator=g).half()
    q, s = ra.quantize_weight_per_channel(torch.randn(2 * inter, K, generator=g) * 0.02)
    w = _strided_on(gpu, q, (1 << 22) + 16)       # 4 MiB per weight row, ~2.5 GB
    h = ra.int8_gateup_swiglu(x.to(gpu), w, s.to(gpu)).cpu()
    del w
    torch.cuda.empty_cache()
    gu = ra.int8_gemm(x.to(gpu), q.to(gpu), s.to(gpu))
    h2 = ra.swiglu_fused(gu[:, :inter].contiguous(), gu[:, inter:].contiguous()).cpu()
    torch.testing.assert_close(h.float(), h2.float(), rtol=1e-2, atol=1e-2)


def test_batched_leading_dims_and_modules(gpu):
    g = torch.Generator().manual_seed(4)
    lin = torch.nn.Linear(256, 320, bias=True)
    m = ra.Int8Linear.from_linear(lin).to(gpu)
    x = torch.randn(2, 7, 256, generator=g).half()
    y = m(x.to(gpu)).cpu()
    assert y.shape == (2, 7, 320) and y.dtype == torch.float16
    ref = fallback.int8_gemm_ref(x.reshape(-1, 256), m.weight_int8.cpu(), m.scale.cpu(), m.bias.detach().cpu())
    torch.testing.assert_close(y.reshape(-1, 320).float(), ref.float(), rtol=1e-2, atol=1e-2)
    qm = ra.QuantizedLinear.from_linear(lin).to(gpu)
    qm._quantized = True
    # the module's fp32 bias with fp16 activations: the reference's F.linear
    # error (symmetric.py:288-291), as on the CPU
    with pytest.raises(RuntimeError, match="same dtype"):
        qm(x.to(gpu))
    qm.bias.data = qm.bias.data.half()
    yq = qm(x.to(gpu)).cpu()
    torch.testing.assert_close(yq.float(), y.float(), rtol=2e-3, atol=2e-3)
    # fp32 activations with the fp32 bias run (the generic kernel)
    qm.bias.data = qm.bias.data.float()
    y32 = qm(x.float().to(gpu)).cpu()
    torch.testing.assert_close(y32, y.float(), rtol=2e-3, atol=2e-3)


def test_empty_and_k_tail(gpu):
    x = torch.zeros(0, 64, dtype=torch.float16, device=gpu)
    q = torch.zeros(32, 64, dtype=torch.int8, device=gpu)
    assert ra.int8_gemm(x, q, torch.ones(32, device=gpu)).shape == (0, 32)
    for (M, K, N) in [(1, 4096 + 16, 128), (3, 1040, 100), (300, 4096 + 48, 256), (260, 4096 + 64, 300)]:
        c = gemm_case(M, K, N, seed=K)
        for v in (ROWS, GEMV, BATCH, SKINNY, TILED):
            y = _run(c.x.to(gpu), c.q.to(gpu), c.s.to(gpu), None, v)
            if y is None:
                assert _may_refuse(v, M, K)
                continue
            _oracle_check(y.cpu(), c.x, c.q, c.s)


def _random_exact_shapes(seed, count):
    """Seeded (gate/up, M, K, N) over the sizes the selection rules separate:
    M = 1..512, K = 512..28672 (multiples of 128 and 512 both), N from 64 to
    28672 (ragged and round)."""
    import random
    rng = random.Random(seed)
    Ms = [1, 2, 3, 4, 5, 7, 8, 12, 16, 17, 18, 24, 31, 32, 33, 40, 48, 56, 63, 64, 65, 96, 128, 200, 256, 512]
    Ks = [512, 1024, 1536, 2048, 3072, 3584, 4096, 5120, 6144, 8192, 11008, 12288, 14336, 16384, 18944, 28672]
    out = []
    while len(out) < count:
        M, K = rng.choice(Ms), rng.choice(Ks)
        N = rng.choice([rng.randrange(64, 4096), rng.randrange(4096, 16384), rng.choice([4096, 8192, 11008, 28672])])
        if M * K <= 32e6 and N * K <= 200e6:
            out.append((rng.random() < 0.3 and M <= 64, M, K, N))
    return out


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_exact_random_shapes_automatic_pick(gpu, dt):
    """Exact known answers through the automatic pick at 120 seeded shapes
    (GEMM and gate/up + SwiGLU): x in {-1, 0, 1} with ~120 non-zeros per row
    and small integer weights keep every sum an integer far below 2^11, exact
    in fp32 in any order, so the GEMM output must equal the rounded sums bit
    for bit; the gate/up output must match silu(gate) * up on the rounded
    sums (the reference composition's roundings) within rtol = atol = 1e-2
    everywhere and bit for bit at all but 0.5 % of the outputs. Inputs and
    the exact sums are formed on the GPU (fp32 products of small integers)."""
    for (gu, M, K, N) in _random_exact_shapes(7, 120):
        print(f"  random exact gu={gu} M={M} K={K} N={N} {dt}", flush=True)
        g = torch.Generator(device=gpu).manual_seed(M * 7 + K + N)
        lim = 3 if dt == torch.float16 else 1
        rows = 2 * N if gu else N
        x = torch.randint(-1, 2, (M, K), device=gpu, generator=g).float()
        x = x * (torch.rand(M, K, device=gpu, generator=g) < 120.0 / K)
        q = torch.randint(-lim, lim + 1, (rows, K), device=gpu, generator=g, dtype=torch.int8)
        s = torch.full((rows,), 2.0 ** -4, device=gpu)
        sums = (x @ q.float().T) * 2.0 ** -4
        if gu:
            h = ra.int8_gateup_swiglu(x.to(dt), q, s).float()
            gb, ub = sums[:, :N].to(dt).float(), sums[:, N:].to(dt).float()
            ref = ((gb * torch.sigmoid(gb)).to(dt).float() * ub).to(dt).float()
            assert bool(((h - ref).abs() <= 1e-2 + 1e-2 * ref.abs()).all()), f"gate/up M={M} K={K} I={N}"
            assert float((h != ref).float().mean()) < 5e-3, f"gate/up M={M} K={K} I={N}"
        else:
            y = ra.int8_gemm(x.to(dt), q, s).float()
            want = sums.to(dt).float()
            assert torch.equal(y, want), f"M={M} K={K} N={N}: {int((y != want).sum())} outputs differ"


def test_graph_replay_matches_eager(gpu):
    c = gemm_case(1, 4096, 11008, seed=2, device=gpu)
    eager = ra.int8_gemm(c.x, c.q, c.s)
    torch.cuda.synchronize()
    out = {}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ra.int8_gemm(c.x, c.q, c.s)        # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out["y"] = ra.int8_gemm(c.x, c.q, c.s)
    for i in range(3):
        out["y"].zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out["y"], eager), f"replay {i}"
