"""GPU tests of the kernels that combine K splits across workgroups through a
workspace (the split-K kernel, the gate/up split-K kernel, the tiled kernel's
split plan), through the C ABI:

* the gate/up split-K kernel (SwiGLU epilogue, K >= 16384) against exact
  answers and the oracle, two calls in a row (its counters reset);
* workspaces under HIP graph capture: graphs captured one after another on
  the same capture stream, replayed in any order (one before the other ever
  ran), between eager calls, bitwise equal to eager results every time;
* a call with a workspace runs what the automatic selection reports, and
  where the split-K plan does not split it runs what a call without a
  workspace runs.
"""
import ctypes

import numpy as np
import pytest
import torch

import rotalabs_accel as ra
from oracle import fallback
from rotalabs_accel import _backend

pytestmark = pytest.mark.gpu


def _gateup_exact_case(M, K, inter, dt, seed):
    """Integer x in {-1, 0, 1} (sparse for bf16), q in [-lim, lim], scales
    2^-4: the gate and up sums are exact in fp32 whatever the order."""
    g = torch.Generator().manual_seed(seed)
    lim = 3 if dt == torch.float16 else 1
    x = torch.randint(-1, 2, (M, K), generator=g).float()
    keep = torch.rand(M, K, generator=g) < min(1.0, 200.0 / K)
    x = x * keep
    q = torch.randint(-lim, lim + 1, (2 * inter, K), generator=g).to(torch.int8)
    s = torch.full((2 * inter,), 2.0 ** -4)
    sums = (x.double() @ q.double().T) * 2.0 ** -4   # exact gate / up values
    return x.to(dt), q, s, sums


def _rnd(v64, dt):
    """Round float64 values (torch tensor) to dt and back."""
    return v64.to(dt).double()


def _dist_to_boundary(v64, dt):
    """Distance from each float64 value to the nearest rounding boundary of
    dt (the midpoints between its rounding and the two neighbours)."""
    vb = v64.to(dt)
    bits = vb.view(torch.int16).to(torch.int32)
    up = (bits + 1).to(torch.int16).view(dt).double()
    dn = (bits - 1).to(torch.int16).view(dt).double()
    vd = vb.double()
    return torch.minimum((v64 - (vd + up) / 2).abs(), (v64 - (vd + dn) / 2).abs())


def _chain(g64, u64, dt):
    """The reference composition on exact gate / up sums: gate and up stored
    in dt (int8_gemm_torch's output, gemm.py:46), silu(gate) stored in dt, the
    product stored in dt (swiglu_torch, activations.py:45) -- the roundings
    the fused epilogue reproduces. Returns (result, silu before rounding)."""
    gb, ub = _rnd(g64, dt), _rnd(u64, dt)
    t64 = gb / (1.0 + torch.exp(-gb))
    return _rnd(_rnd(t64, dt) * ub, dt), t64


def _neighbours(vb, dt):
    """(v, next up, next down) of dt values vb, as float64."""
    bits = vb.view(torch.int16).to(torch.int32)
    return [vb.double(), (bits + 1).to(torch.int16).view(dt).double(), (bits - 1).to(torch.int16).view(dt).double()]


def _check_chain(h, g64, u64, dt, gslack, uslack):
    """h (kernel output) against the chain of the exact sums:

    * bitwise equal except for fewer than 0.5 % of the outputs (fp32
      accumulation in any order changes a gate / up value that lies within
      its error bound of a rounding boundary; tiny values, where the fp32
      sums cancel, differ by a few ulps);
    * every output within rtol = atol = 1e-2 of the chain, except where a gate
      or up value (or silu(gate)) lies within its fp32 error (gslack, uslack)
      of a rounding boundary AND the output is the chain with that value
      rounded to the other neighbour: a gate that rounds the other way moves
      the output by one gate ulp times |up|, which at long K can exceed 1e-2
      of it (the reference composition itself is that sensitive there)."""
    ref, t64 = _chain(g64, u64, dt)
    hd = h.double()
    frac = (hd != ref).double().mean().item()
    assert frac < 5e-3, frac
    out = (hd - ref).abs() > 1e-2 + 1e-2 * ref.abs()
    if out.any():
        gb, ub, tb, hb = g64[out], u64[out], t64[out], hd[out]
        near = ((_dist_to_boundary(gb, dt) <= gslack[out]) | (_dist_to_boundary(ub, dt) <= uslack[out])
                | (_dist_to_boundary(tb, dt) <= 1e-6 * tb.abs() + 1e-30))
        assert bool(near.all()), f"{int((~near).sum())} outputs beyond 1e-2 away from any rounding boundary"
        hit = torch.zeros_like(gb, dtype=torch.bool)
        for gv in _neighbours(gb.to(dt), dt):
            for uv in _neighbours(ub.to(dt), dt):
                t = gv / (1.0 + torch.exp(-gv))
                for tv in _neighbours(t.to(dt), dt):
                    hit |= hb == _rnd(tv * uv, dt)
        if not bool(hit.all()):
            miss = ~hit
            rows = [(hb[miss][i].item(), ref[out][miss][i].item(), gb[miss][i].item(), ub[miss][i].item(),
                     tb[miss][i].item()) for i in range(min(4, int(miss.sum())))]
            raise AssertionError(f"{int(miss.sum())} outputs beyond 1e-2 not explained by one rounding flip "
                                 f"(kernel, chain, gate, up, silu): {rows}")


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,inter", [(17, 16384, 3000), (3, 16384, 700), (64, 32768, 1000), (5, 16384, 48),
                                        (33, 16384, 520),
                                        # below K = 16384: M = 33..64 (from 48 rows or over 4096+ gate rows),
                                        # and at most 4096 gate rows from K = 8192
                                        (48, 4096, 3000), (33, 3584, 4200), (64, 8192, 2000), (2, 16384, 3584),
                                        (24, 12288, 1000),
                                        # M = 2..32: from 24 rows, from 16 rows at K = 8192, K not a
                                        # multiple of 1024, M = 17, few gate rows from K = 2048
                                        (24, 4096, 6000), (16, 8192, 5000), (8, 4224, 3000), (17, 2048, 3000),
                                        (8, 2048, 2000), (4, 3072, 7000),
                                        # M = 33..47 over few gate rows from K = 6144, from 40 rows at 4096
                                        (40, 6144, 2000), (44, 4096, 2000),
                                        # M = 18..23 from K = 5120
                                        (20, 5120, 3000), (21, 5120, 6000)])
def test_gateup_splitk_vs_exact_and_oracle(gpu, dt, M, K, inter):
    """The gate/up + SwiGLU GEMM through the split-K kernel (K >= 16384, M =
    33..64 (over few gate rows from K = 6144, or from 40 rows at K = 4096),
    at most 4096 gate rows from K = 8192, or M = 2..32 at M = 17,
    from 24 rows, from 16 rows at K = 8192, with K not a multiple of 1024 or
    over few gate rows from K = 2048, or from 18 rows at K >= 5120; a workspace is asked for
    and given). Exact integer sums make the fp32 gate
    and up values order-independent, so the output must be the reference
    composition's roundings of them bit for bit (up to silu's own fp32
    rounding at a boundary), with and without a workspace; a second call on
    the same inputs is bitwise equal (the counters are back at zero after
    the first); random inputs against the oracle's float64 sums."""
    lib = _backend.load()
    dcode = _backend.dtype_code(dt)
    assert lib.ra_w8a16_gateup_workspace_size(M, inter, K, dcode) > _backend.WORKSPACE_COUNTER_BYTES
    print(f"  gateup split-K exact M={M} K={K} I={inter} {dt}", flush=True)
    x, q, s, sums = _gateup_exact_case(M, K, inter, dt, seed=M + K + inter)
    xd, qd, sd = x.to(gpu), q.to(gpu), s.to(gpu)
    h1 = ra.int8_gateup_swiglu(xd, qd, sd)
    h2 = ra.int8_gateup_swiglu(xd, qd, sd)
    torch.cuda.synchronize()
    assert torch.equal(h1, h2), "second call differs: split counters not reset"
    zero = torch.zeros(M, inter, dtype=torch.float64)
    _check_chain(h1.cpu(), sums[:, :inter], sums[:, inter:], dt, zero, zero)
    # the same inputs without a workspace (the one-pass kernels, or split K where its plan does not split)
    h0 = torch.empty_like(h1)
    xc = xd.contiguous()
    _backend.check(lib.ra_w8a16_gateup_swiglu(xc.data_ptr(), K, dcode, qd.data_ptr(), K, sd.data_ptr(),
                                              h0.data_ptr(), inter, M, inter, K,
                                              _backend.stream_handle(gpu)))
    torch.cuda.synchronize()
    _check_chain(h0.cpu(), sums[:, :inter], sums[:, inter:], dt, zero, zero)
    # random inputs: the oracle's float64 sums through the same chain; a gate
    # or up value may round the other way only within K u32 sum|x w| (fp32
    # accumulation in any order) of a boundary
    print(f"  gateup split-K random M={M} K={K} I={inter} {dt}", flush=True)
    g = torch.Generator().manual_seed(7 * M + K)
    xr = torch.randn(M, K, generator=g).to(dt)
    qr, sr = ra.quantize_weight_per_channel(torch.randn(2 * inter, K, generator=g) * 0.02)
    hr = ra.int8_gateup_swiglu(xr.to(gpu), qr.to(gpu), sr.to(gpu)).cpu()
    y64 = torch.from_numpy(fallback.gemm_f64(xr.float().numpy(), qr.numpy(), sr.numpy()))
    sabs = torch.from_numpy((np.abs(xr.float().numpy()).astype(np.float64)
                             @ np.abs(qr.numpy().astype(np.float64)).T) * sr.numpy())
    slack = K * 2.0 ** -24 * sabs
    _check_chain(hr, y64[:, :inter], y64[:, inter:], dt, slack[:, :inter], slack[:, inter:])


# One problem per split-K kernel instantiation the automatic pick reaches
# (GEMM / gate-up, 16*MT-row tiles, the extra row, TW weight tiles per wave,
# 4 or 8 waves per workgroup), with the plan (NW, TW, S) the time model picks
# for it, pinned through the library's planner.
SPLITK_INSTANCES = [
    # (gate/up, M, K, N or I, NW, TW, S)
    (False, 3, 16384, 128, 4, 1, 16), (False, 5, 32768, 1600, 8, 1, 16), (False, 5, 5120, 20480, 8, 2, 3),
    (False, 3, 5120, 40960, 8, 3, 2), (False, 17, 16384, 128, 4, 1, 16), (False, 17, 16384, 2624, 8, 1, 10),
    (False, 17, 16384, 10304, 8, 2, 5), (False, 17, 24576, 10304, 8, 3, 8), (False, 24, 5120, 128, 4, 1, 8),
    (False, 18, 11008, 3136, 8, 1, 8), (False, 17, 5120, 20480, 8, 2, 3), (False, 32, 5120, 10816, 4, 3, 4),
    (False, 17, 5120, 40960, 8, 3, 2), (False, 33, 16384, 128, 4, 1, 13), (False, 33, 24576, 1600, 8, 1, 16),
    (False, 33, 16384, 10304, 8, 2, 5), (False, 33, 32768, 10304, 8, 3, 8), (False, 33, 4096, 128, 4, 1, 8),
    (False, 33, 11008, 3136, 8, 1, 8), (False, 33, 14336, 10304, 8, 2, 5), (False, 33, 8192, 40960, 8, 3, 2),
    (False, 16, 9088, 10944, 4, 3, 4), (False, 24, 2048, 29568, 4, 2, 1), (False, 33, 4096, 33344, 4, 3, 1),
    (False, 34, 4608, 64, 4, 1, 6), (False, 63, 6784, 3328, 8, 1, 8), (False, 48, 8832, 10496, 8, 2, 5),
    (False, 38, 8192, 21888, 4, 3, 2), (False, 33, 512, 28672, 4, 2, 1), (True, 3, 8192, 128, 4, 1, 11),
    (True, 8, 16384, 3136, 8, 1, 8), (True, 3, 16384, 10816, 8, 2, 5), (True, 17, 16384, 128, 4, 1, 13),
    (True, 17, 16384, 3136, 8, 1, 8), (True, 17, 16384, 10304, 8, 2, 5), (True, 17, 8192, 128, 4, 1, 8),
    (True, 24, 16384, 3136, 8, 1, 8), (True, 18, 16384, 10304, 8, 2, 5), (True, 18, 16384, 40960, 4, 3, 1),
    (True, 33, 16384, 128, 4, 1, 10), (True, 33, 16384, 3136, 8, 1, 8), (True, 33, 16384, 10304, 8, 2, 5),
    (True, 33, 16384, 11584, 4, 3, 4), (True, 48, 4096, 128, 4, 1, 4), (True, 33, 4096, 8256, 8, 1, 3),
    (True, 33, 4096, 40960, 4, 3, 1), (True, 3, 128, 16576, 4, 2, 1), (True, 13, 2304, 20928, 4, 3, 2),
    (True, 17, 128, 34688, 4, 3, 1), (True, 17, 128, 17216, 4, 2, 1), (True, 23, 1536, 64, 4, 1, 4),
    (True, 28, 128, 16576, 4, 2, 1), (True, 33, 128, 17856, 4, 2, 1), (True, 64, 3200, 8320, 8, 1, 3),
    (True, 40, 128, 17216, 4, 2, 1), (True, 60, 128, 32896, 4, 3, 1), (False, 41, 7936, 3136, 8, 1, 8),
    (False, 48, 4352, 33088, 8, 3, 2), (False, 53, 4480, 64, 4, 1, 7), (False, 59, 14336, 10432, 8, 2, 5),
    (True, 45, 2688, 8832, 8, 1, 3), (True, 45, 128, 32896, 4, 3, 1), (True, 57, 1920, 64, 4, 1, 3),
    (True, 61, 128, 17088, 4, 2, 1), (False, 38, 128, 28672, 4, 2, 1), (False, 64, 5120, 20928, 4, 3, 2)]


class _SplitkPlan(ctypes.Structure):
    """ra::SplitkPlan (rotalabs-accel_amd/csrc/ra_internal.h)."""
    _fields_ = [("ok", ctypes.c_bool), ("mt", ctypes.c_int), ("tw", ctypes.c_int), ("S", ctypes.c_int),
                ("kc", ctypes.c_int), ("nb", ctypes.c_int), ("spread", ctypes.c_bool),
                ("cnt_bytes", ctypes.c_size_t), ("ws_bytes", ctypes.c_size_t), ("x1", ctypes.c_int),
                ("nw", ctypes.c_int)]


def _splitk_plan(M, N, K, gu):
    """The library's split-K plan (its C++ planner, exported from the shared
    library under its mangled name)."""
    f = getattr(_backend.load(), "_ZN2ra11splitk_planElllbb")
    f.restype = _SplitkPlan
    f.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_bool, ctypes.c_bool]
    return f(M, N, K, gu, True)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("gu,M,K,N,nw,tw,S", SPLITK_INSTANCES)
def test_splitk_every_instantiation_exact(gpu, dt, gu, M, K, N, nw, tw, S):
    """Exact known answers from every split-K instantiation the automatic pick
    reaches (both dtypes, GEMM and gate/up): x in {-1, 0, 1} with ~120
    non-zeros per row and q in [-lim, lim] keep every sum an integer below
    2^11, exact in fp32 whatever the order, so any tile, extra-row, split or
    combine mistake is a mismatch. The inputs are generated and the exact sums
    formed on the GPU (fp32 products of small integers)."""
    lib = _backend.load()
    dcode = _backend.dtype_code(dt)
    p = _splitk_plan(M, N, K, gu)
    assert p.ok and (p.nw, p.tw, p.S) == (nw, tw, S), f"the plan is ({p.nw}, {p.tw}, {p.S})"
    print(f"  split-K instance gu={gu} M={M} K={K} N={N} nw={nw} tw={tw} S={S} {dt}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(M * 3 + K + N)
    lim = 3 if dt == torch.float16 else 1
    rows = 2 * N if gu else N
    x = torch.randint(-1, 2, (M, K), device=gpu, generator=g).float()
    x = x * (torch.rand(M, K, device=gpu, generator=g) < 120.0 / K)
    q = torch.randint(-lim, lim + 1, (rows, K), device=gpu, generator=g, dtype=torch.int8)
    s = torch.full((rows,), 2.0 ** -4, device=gpu)
    sums = ((x @ q.float().T) * 2.0 ** -4).double().cpu()
    if gu:
        assert lib.ra_w8a16_gateup_workspace_size(M, N, K, dcode) == (p.ws_bytes if S > 1 else 0)
        h = ra.int8_gateup_swiglu(x.to(dt), q, s)
        torch.cuda.synchronize()
        zero = torch.zeros(M, N, dtype=torch.float64)
        _check_chain(h.cpu(), sums[:, :N], sums[:, N:], dt, zero, zero)
        return
    assert lib.ra_w8a16_gemm_select(M, N, K, dcode) == _backend.VARIANT_SPLITK
    y = ra.int8_gemm(x.to(dt), q, s).cpu()
    assert torch.equal(y, sums.to(dt)), f"{int((y.double() != sums).sum())} outputs differ"


def _int8_case(M, K, N, dt, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(dt)
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = torch.rand(N, generator=g) * 2e-3 + 1e-4
    return x.to(dev), q.to(dev), s.to(dev)


def test_graph_capture_workspaces(gpu):
    """Graphs captured one after another on torch's default capture stream,
    each calling kernels that split K through a workspace: graph A (M=17
    K=28672 N=8192, split-K), then graph B (M=5 K=16384 N=1000 split-K, the
    tiled split plan at M=64 K=11008 N=8192 and the gate/up split-K kernel at
    M=40 I=6000 K=16384, each needing a larger workspace than the one before).
    B is replayed before A ever ran, then A, then eager calls, then both again
    in the other order; every output of every replay is bitwise equal to the
    eager result (the same kernels in the same order)."""
    dt = torch.bfloat16
    lib = _backend.load()
    a_case = _int8_case(17, 28672, 8192, dt, 1, gpu)
    b1_case = _int8_case(5, 16384, 1000, dt, 2, gpu)
    b2_case = _int8_case(64, 11008, 8192, dt, 3, gpu)
    g = torch.Generator().manual_seed(4)
    gu_x = torch.randn(40, 16384, generator=g).to(dt).to(gpu)
    gu_q, gu_s = ra.quantize_weight_per_channel(torch.randn(12000, 16384, generator=g).to(gpu) * 0.02)
    assert lib.ra_w8a16_gemm_select(17, 8192, 28672, 1) == _backend.VARIANT_SPLITK
    assert lib.ra_w8a16_gemm_select(5, 1000, 16384, 1) == _backend.VARIANT_SPLITK
    assert lib.ra_w8a16_gemm_select(64, 8192, 11008, 1) == _backend.VARIANT_TILED
    sizes = [lib.ra_w8a16_gemm_workspace_size(5, 1000, 16384, 1),
             lib.ra_w8a16_gemm_workspace_size(64, 8192, 11008, 1),
             lib.ra_w8a16_gateup_workspace_size(40, 6000, 16384, 1)]
    assert 0 < sizes[0] < sizes[1] < sizes[2], sizes

    def run_a():
        return [ra.int8_gemm(*a_case)]

    def run_b():
        return [ra.int8_gemm(*b1_case), ra.int8_gemm(*b2_case), ra.int8_gateup_swiglu(gu_x, gu_q, gu_s)]

    print("  eager references", flush=True)
    want_a, want_b = run_a(), run_b()
    torch.cuda.synchronize()
    # warm-up on a side stream, as torch's graph documentation recommends
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_a()
        run_b()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    print("  capture A, then B", flush=True)
    graph_a, graph_b = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph_a):
        out_a = run_a()
    with torch.cuda.graph(graph_b):
        out_b = run_b()
    torch.cuda.synchronize()

    def check(outs, wants, what):
        for i, (o, w) in enumerate(zip(outs, wants)):
            assert torch.equal(o, w), f"{what}: output {i} differs from eager"

    for step in range(3):
        print(f"  round {step}: replay B, A, eager", flush=True)
        for o in out_a + out_b:
            o.zero_()
        torch.cuda.synchronize()
        graph_b.replay()          # (first round: before A ever ran)
        torch.cuda.synchronize()
        check(out_b, want_b, f"round {step} B")
        graph_a.replay()
        torch.cuda.synchronize()
        check(out_a, want_a, f"round {step} A")
        check(run_b() + run_a(), want_b + want_a, f"round {step} eager")
        torch.cuda.synchronize()
        graph_a.replay()
        graph_b.replay()
        torch.cuda.synchronize()
        check(out_a, want_a, f"round {step} A again")
        check(out_b, want_b, f"round {step} B again")


@pytest.mark.parametrize("M,N,K", [(8, 65536, 16384), (2, 128256, 16384)])
def test_workspace_call_runs_the_selected_kernel(gpu, M, N, K):
    """Shapes where the split-K plan does not split (S = 1): no workspace is
    asked for and the split-K kernel runs unsplit with or without one, so
    ra_w8a16_gemm_ws with a workspace and ra_w8a16_gemm without one produce
    the same bits."""
    lib = _backend.load()
    assert lib.ra_w8a16_gemm_workspace_size(M, N, K, 0) == 0
    assert lib.ra_w8a16_gemm_select(M, N, K, 0) == _backend.VARIANT_SPLITK
    print(f"  ws vs no ws M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(M)
    x = torch.randn(M, K, device=gpu, generator=g).half()
    q = torch.randint(-127, 128, (N, K), device=gpu, generator=g, dtype=torch.int8)
    s = torch.rand(N, device=gpu, generator=g) * 1e-3
    ws = torch.zeros(1 << 24, dtype=torch.uint8, device=gpu)
    y0 = torch.empty((M, N), dtype=torch.float16, device=gpu)
    y1 = torch.empty_like(y0)
    st = _backend.stream_handle(gpu)
    _backend.check(lib.ra_w8a16_gemm(x.data_ptr(), K, 0, q.data_ptr(), K, s.data_ptr(), None, 2, y0.data_ptr(), N,
                                     M, N, K, st))
    _backend.check(lib.ra_w8a16_gemm_ws(x.data_ptr(), K, 0, q.data_ptr(), K, s.data_ptr(), None, 2, y1.data_ptr(),
                                        N, M, N, K, ws.data_ptr(), ws.numel(), st))
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    ref = (x.float() @ q.float().T) * s
    torch.testing.assert_close(y0.float(), ref, rtol=1e-2, atol=1e-2)


def _strided(gpu, t, ld):
    """A (rows, cols) copy of t on the GPU with row stride ld elements."""
    rows, cols = t.shape
    store = torch.zeros((rows - 1) * ld + cols, dtype=t.dtype, device=gpu)
    v = store.as_strided((rows, cols), (ld, 1))
    v.copy_(t.to(gpu))
    return v


@pytest.mark.parametrize("gu,M,K,N", [(False, 17, 16384, 300), (False, 40, 4096, 4000), (False, 60, 3072, 6000),
                                      (False, 5, 16384, 1000), (True, 33, 16384, 520), (True, 45, 4096, 2000),
                                      (True, 17, 8192, 700)])
def test_splitk_row_strides(gpu, gu, M, K, N):
    """The split-K kernel with row strides on both operands (ldx = K + 8,
    ldw = K + 48: every copy addresses its row through the stride) over the
    tile forms (one, two with the extra row, three and four 16-row tiles;
    GEMM and gate/up): bitwise the same output as contiguous operands (the
    same plan, so the same order of sums)."""
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(M + K + N)
    rows = 2 * N if gu else N
    x = torch.randn(M, K, generator=g).to(dt)
    q = torch.randint(-127, 128, (rows, K), generator=g, dtype=torch.int8)
    s = torch.rand(rows, generator=g) * 2e-3 + 1e-4
    lib = _backend.load()
    dcode = _backend.dtype_code(dt)
    if gu:
        assert lib.ra_w8a16_gateup_workspace_size(M, N, K, dcode) > _backend.WORKSPACE_COUNTER_BYTES
    else:
        assert lib.ra_w8a16_gemm_select(M, N, K, dcode) == _backend.VARIANT_SPLITK
    print(f"  split-K strides gu={gu} M={M} K={K} N={N}", flush=True)
    xs, qs, sd = _strided(gpu, x, K + 8), _strided(gpu, q, K + 48), s.to(gpu)
    assert xs.stride(0) == K + 8 and qs.stride(0) == K + 48
    fn = ra.int8_gateup_swiglu if gu else ra.int8_gemm
    want = fn(x.to(gpu), q.to(gpu), sd)
    got = fn(xs, qs, sd)
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"max diff {(got.float() - want.float()).abs().max().item()}"
