"""Benchmark of the W8A16 INT8 GEMM path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Metric: int8_gemm HBM GB/s at M=1 and TFLOP/s at M=2048 (K=4096, N=11008).

* Headline (``value``): decode, x fp16 [1,4096] @ int8 W [11008,4096] with
  per-channel fp32 scales. One step = one int8_gemm call through the C ABI.
  Steps cycle over 12 resident copies of the weight (541 MB > 2x the 256 MB
  Infinity Cache) so every step streams its weight from HBM. ``value`` =
  algorithmic bytes per step (N*K + 4N + 2MK + 2MN) / (timed region / K).
* ``steps``: exactly ``--steps`` launches are timed (whole graphs of 120
  launches, the remainder launched from the host), queued behind an untimed
  graph replay so that no launch latency falls inside the timed region.
* ``config.python_int8_gemm_eager_us_per_call``: the Python ``int8_gemm``
  called eagerly in a host loop at the headline shape (argument checks,
  output allocation, C ABI call and launch), beside the graph-replay figure.
* ``prefill``: x fp16 [2048,4096] @ W [11008,4096], TFLOP/s = 2MNK / time;
  ``prefill_large``: the same at M=8192 K=4096 N=4096.
* ``roofline``: the dominant kernel's achieved GB/s (TFLOP/s for prefill)
  from HIP events on the launch stream, against MI355X peaks (HBM 8 TB/s,
  dense fp16 MFMA 2516.6 TFLOP/s).
* ``w8a8``: the opt-in W8A8 route (int8 activations, int8 MFMA) at the
  prefill shape, TOPS against the dense int8 peak (5033 TOP/s), beside
  hipBLASLt's int8 GEMM (torch._int_mm).
* ``shapes``: the other decode shapes (M=1: K=4096 N=4096, K=11008 N=4096)
  and the small-batch shapes (M=4, 16, 64 at K=4096 N=11008), GB/s per
  call, timed like the headline.
* ``mlp``: the fused decoder MLP block (RMSNorm -> int8 gate/up + SwiGLU ->
  int8 down, bf16, H=8192, I=28672) per call at M=1 and M=17 (GB/s) and
  M=4096 (TFLOP/s), graph replay, each with its roofline.
* ``cpu_baseline``: the reference's CPU fallback (dequantize + F.linear per
  call), restated in oracle/, timed on this host on a bounded sample.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(HERE, "rotalabs-accel_amd"))

PEAK_HBM_GBS = 8000.0
PEAK_FP16_TFLOPS = 2516.6
METRIC = "int8_gemm HBM GB/s @M=1 + TFLOP/s @M=2048 (K=4096,N=11008)"
DECODE = (1, 4096, 11008, 2)        # M, K, N, seed
PREFILL = (2048, 4096, 11008, 7)
PREFILL_LARGE = (8192, 4096, 4096, 8)   # the second prefill shape of the workload set
N_COPIES = 12


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3000)
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--prefill-steps", type=int, default=300)
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--only", choices=("all", "decode", "prefill", "prefill_large", "mlp", "w8a8", "shapes",
                                      "ceiling", "tile-trace"),
                   default="all",
                   help="run one workload only (for profiler runs)")
    p.add_argument("--no-mlp", action="store_true", help="skip the fused-MLP timing")
    p.add_argument("--mlp-rows", default="1,17,4096",
                   help="with --only mlp: the MLP block's row counts to time (for profiler runs; any other "
                        "value than the default also skips the RMSNorm and KV-codec lines)")
    p.add_argument("--shape", default="",
                   help="with --only shapes: time this one GEMM shape M,K,N instead (for profiler runs)")
    p.add_argument("--no-graph", action="store_true",
                   help="time host-launched loops instead of HIP graph replay (for counter runs)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a plain 256 MiB device copy (torch copy_), the known-size kernel that "
                        "scales FETCH_SIZE / WRITE_SIZE counter readings to bytes")
    return p.parse_args()


TRAFFIC_FILE = os.path.join(HERE, "profiles", "hbm_traffic.md")


def measured_traffic(workload: str):
    """HBM bytes per launch of the workload's kernel (per call of the MLP
    block: its kernels summed) as measured by the rocprofv3 FETCH_SIZE +
    WRITE_SIZE runs recorded in profiles/hbm_traffic.md (table rows
    ``| workload | kernel | algorithmic B | fetch B | write B | traffic B |``);
    None when no row matches."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 6 and cells[0] == workload:
                    return int(cells[5].replace(",", ""))
    except (OSError, ValueError):
        pass
    return None


def copy_calibration():
    """A plain device copy of 256 MiB, five times: reads and writes exactly
    268,435,456 bytes per launch."""
    import torch
    n = 256 * 2**20 // 2
    src = torch.randn(n, device="cuda:0").half()
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: 5 copies of {n * 2} bytes")


class GemmLauncher:
    """Pre-bound ra_w8a16_gemm_ws calls (C ABI), one per weight copy, launched
    on torch's current stream (so they can be captured into a HIP graph),
    with a zero-filled workspace of the size the library asks for (the
    split-K small-batch kernel keeps its partial sums there)."""

    def __init__(self, x, weights, scale, y, variant=0):
        import torch
        from rotalabs_accel import _backend
        lib = _backend.load()
        M, K = x.shape
        N = weights[0].shape[0]
        xdt = _backend.dtype_code(x.dtype)
        nws = int(lib.ra_w8a16_gemm_workspace_size(M, N, K, xdt))
        self.ws = torch.zeros(max(nws, 1), dtype=torch.uint8, device=x.device)
        wsp = self.ws.data_ptr() if nws else None
        if variant:
            self.fn = lib.ra_w8a16_gemm_ex
            self.args = [(x.data_ptr(), K, xdt, w.data_ptr(), K, scale.data_ptr(), None, 0,
                          y.data_ptr(), N, M, N, K, variant, wsp, nws) for w in weights]
        else:
            self.fn = lib.ra_w8a16_gemm_ws
            self.args = [(x.data_ptr(), K, xdt, w.data_ptr(), K, scale.data_ptr(), None, 0,
                          y.data_ptr(), N, M, N, K, wsp, nws) for w in weights]
        self.keep = (x, weights, scale, y)

    def run(self, steps: int):
        import torch
        stream = torch.cuda.current_stream().cuda_stream
        fn, args, n = self.fn, self.args, len(self.args)
        for i in range(steps):
            rc = fn(*args[i % n], stream)
            if rc:
                raise RuntimeError(f"ra_w8a16_gemm_ws failed with {rc}")


def time_eager(launcher, steps: int, warmup: int):
    """Host-launched loop: per-step time including launch overhead."""
    import torch
    launcher.run(warmup)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    launcher.run(steps)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


GRAPH_LATENCY: dict = {}   # per_graph -> launch latency of one graph replay (us), last measured


def time_graph(launcher, steps: int, warmup: int, per_graph: int, warm_seconds: float = 0.2):
    """Exactly ``steps`` launches timed with HIP events on the launch stream,
    back to back on the GPU: steps // per_graph replays of a HIP graph of
    ``per_graph`` launches, then the remaining steps % per_graph launches
    issued from the host, all enqueued behind one untimed replay of the graph
    that was enqueued just before the start event. That replay keeps the GPU
    busy while the host enqueues the timed work, so no launch latency (host
    launch, or the fixed cost of starting a graph, ~5-8 us on ROCm) falls
    inside the timed region, which would otherwise be a visible share of it
    with few steps. Untimed replays run for at least ``warmup`` launches and
    ``warm_seconds`` first, so that the timed region starts at steady clocks.
    The launch latency of one graph replay from an idle stream (minus
    ``per_graph`` steady steps) is left in GRAPH_LATENCY[per_graph] (us).
    Returns (ms per step, steps timed)."""
    import torch
    steps = max(1, steps)
    full, rem = divmod(steps, per_graph)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launcher.run(2)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launcher.run(per_graph)
    t0, done = time.perf_counter(), 0
    while done < warmup or time.perf_counter() - t0 < warm_seconds:
        graph.replay()
        torch.cuda.synchronize()
        done += per_graph
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    graph.replay()                # untimed head start, not waited for
    start.record()
    for _ in range(full):
        graph.replay()
    if rem:
        launcher.run(rem)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    # launch latency of one replay from an idle stream
    lat = []
    for _ in range(3):
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        graph.replay()
        s1.record()
        torch.cuda.synchronize()
        lat.append(s0.elapsed_time(s1) - per_graph * ms)
    GRAPH_LATENCY[per_graph] = round(sorted(lat)[1] * 1e3, 2)
    return ms, steps


def time_python_int8_gemm(x, copies, scale, steps: int, warmup: int):
    """The Python ``int8_gemm`` called eagerly in a host loop (argument
    checks, output allocation, the C ABI call and its launch), cycling the
    weight copies; HIP events on torch's current stream. ms per call."""
    import torch
    import rotalabs_accel as ra
    n = len(copies)
    for i in range(warmup):
        ra.int8_gemm(x, copies[i % n], scale)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        ra.int8_gemm(x, copies[i % n], scale)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def host_info():
    """CPU model, torch version and the BLAS / oneDNN backends the CPU
    fallback's F.linear dispatches to (torch.__config__)."""
    import torch
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cfg = torch.__config__.show()
    blas = next((ln.split("=", 1)[1].strip() for ln in cfg.splitlines() if "BLAS_INFO=" in ln), "unknown")
    blas = blas.split(",")[0]
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "torch": torch.__version__,
            "blas": blas, "mkl": torch.backends.mkl.is_available(),
            "mkldnn": torch.backends.mkldnn.is_available()}


def cpu_baseline(M, K, N, seed, budget_s):
    """The reference's CPU fallback (oracle restatement) on a bounded sample."""
    import torch
    from oracle.fallback import int8_gemm_ref
    from workloads import gemm_bytes, gemm_case, gemm_flops
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    c = gemm_case(M, K, N, seed)
    int8_gemm_ref(c.x, c.q, c.s)            # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        int8_gemm_ref(c.x, c.q, c.s)
        times.append(time.perf_counter() - t0)
        if len(times) >= 200:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"med_s": med, "calls": len(times), "threads": torch.get_num_threads(),
            "gbs": gemm_bytes(M, K, N) / med / 1e9, "tflops": gemm_flops(M, K, N) / med / 1e12}


def cpu_baseline_prefill(budget_s, rows=64):
    """The reference's CPU fallback on a bounded sample of the prefill
    workload: the first ``rows`` rows of x (M=2048 K=4096 N=11008), whole
    dequantisation per call as the fallback does. TFLOP/s of the sample."""
    import torch
    from oracle.fallback import int8_gemm_ref
    from workloads import gemm_case, gemm_flops
    torch.set_num_threads(os.cpu_count() or 1)
    Mp, Kp, Np, seedp = PREFILL
    c = gemm_case(rows, Kp, Np, seedp)
    int8_gemm_ref(c.x, c.q, c.s)
    times, t_end = [], time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        int8_gemm_ref(c.x, c.q, c.s)
        times.append(time.perf_counter() - t0)
        if len(times) >= 100:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(gemm_flops(rows, Kp, Np) / med / 1e12, 4), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port", **host_info(),
            "sample": f"{len(times)} calls of the reference fallback on the first {rows} rows of the M={Mp} "
                      f"K={Kp} N={Np} fp16 workload (weights dequantised per call), median "
                      f"{med * 1e3:.1f} ms/call"}


def cpu_baseline_mlp(budget_s):
    """The reference composition on the CPU (oracle restatement: RMSNorm,
    dequantise-then-matmul gate/up, SwiGLU, down) for one bf16 row of the
    H=8192 I=28672 MLP block; GB/s of the block's bytes."""
    import torch
    from oracle.fallback import mlp_ref
    from workloads import mlp_bytes
    torch.set_num_threads(os.cpu_count() or 1)
    H, I = MLP
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, H, generator=g).to(torch.bfloat16)
    nw = (1.0 + 0.01 * torch.randn(H, generator=g)).to(torch.bfloat16)
    q_gu = torch.randint(-127, 128, (2 * I, H), generator=g, dtype=torch.int8)
    s_gu = torch.rand(2 * I, generator=g) * 1e-3
    q_d = torch.randint(-127, 128, (H, I), generator=g, dtype=torch.int8)
    s_d = torch.rand(H, generator=g) * 1e-3
    mlp_ref(x, nw, q_gu, s_gu, q_d, s_d)
    times, t_end = [], time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        mlp_ref(x, nw, q_gu, s_gu, q_d, s_d)
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(mlp_bytes(1, H, I) / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", **host_info(),
            "sample": f"{len(times)} calls of the reference MLP composition (weights dequantised per call) at "
                      f"M=1 H={H} I={I} bf16, median {med * 1e3:.1f} ms/call"}


VARIANT_NAMES = {1: "skinny", 2: "tiled", 3: "generic", 4: "gemv", 5: "rows", 6: "batch", 7: "splitk"}
# Kernel (symbol prefix in rocprofv3 traces) that each variant launches.
VARIANT_KERNELS = {1: "skinny_kernel", 2: "tiled_dma_kernel", 3: "generic_kernel", 4: "gemv_kernel",
                   5: "gemv_rows_lds_kernel", 6: "batch_kernel", 7: "splitk_kernel"}


def run_decode(args, dev):
    """Decode M=1: returns (ms/step graph or host loop, ms/step host loop,
    GB/s, timed steps, variant)."""
    import torch
    import rotalabs_accel as ra
    from rotalabs_accel import _backend
    from workloads import gemm_bytes, gemm_case
    M, K, N, seed = DECODE
    c = gemm_case(M, K, N, seed, device=dev)
    copies = [c.q] + [c.q.clone() for _ in range(N_COPIES - 1)]
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    variant = _backend.load().ra_w8a16_gemm_select(M, N, K, _backend.F16)
    launcher = GemmLauncher(c.x, copies, c.s, y)
    # correctness of what is timed (same call as the tests)
    ref = ra.int8_gemm(c.x, c.q, c.s)
    launcher.run(1)
    torch.cuda.synchronize()
    assert torch.equal(y, ref), "timed path differs from int8_gemm"
    log(f"decode M={M} K={K} N={N}: variant {variant}, {N_COPIES} weight copies "
        f"({N_COPIES * N * K / 2**20:.0f} MiB), warmup {args.warmup}, steps {args.steps}")
    ms_eager = time_eager(launcher, min(args.steps, 2000), args.warmup)
    ms_py = time_python_int8_gemm(c.x, copies, c.s, min(args.steps, 2000), args.warmup)
    if args.no_graph:
        ms, timed_steps = time_eager(launcher, args.steps, args.warmup), args.steps
    else:
        ms, timed_steps = time_graph(launcher, args.steps, args.warmup, per_graph=10 * N_COPIES)
    gbs = gemm_bytes(M, K, N) / (ms * 1e-3) / 1e9
    log(f"decode: {ms * 1e3:.2f} us/step ({'host loop' if args.no_graph else 'graph replay'}), {gbs:.0f} GB/s "
        f"({gbs / PEAK_HBM_GBS:.1%} of HBM peak); host-launched C ABI loop {ms_eager * 1e3:.2f} us/step; "
        f"eager Python int8_gemm {ms_py * 1e3:.2f} us/call")
    return ms, ms_eager, ms_py, gbs, timed_steps, variant


def run_prefill(args, dev, shape=PREFILL):
    """Prefill (M=2048 K=4096 N=11008 by default): returns (ms/step,
    TFLOP/s, variant)."""
    import torch
    import rotalabs_accel as ra
    from rotalabs_accel import _backend
    from workloads import gemm_case, gemm_flops
    Mp, Kp, Np, seedp = shape
    cp = gemm_case(Mp, Kp, Np, seedp, device=dev)
    yp = torch.empty((Mp, Np), dtype=torch.float16, device=dev)
    pcopies = [cp.q, cp.q.clone(), cp.q.clone()]
    plaunch = GemmLauncher(cp.x, pcopies, cp.s, yp)
    pref = ra.int8_gemm(cp.x, cp.q, cp.s)
    plaunch.run(1)
    torch.cuda.synchronize()
    assert torch.equal(yp, pref), "timed prefill path differs from int8_gemm"
    pvariant = _backend.load().ra_w8a16_gemm_select(Mp, Np, Kp, _backend.F16)
    if args.no_graph:
        pms = time_eager(plaunch, args.prefill_steps, 3)
    else:
        pms, _ = time_graph(plaunch, args.prefill_steps, 3, per_graph=3 * len(pcopies))
    tflops = gemm_flops(Mp, Kp, Np) / (pms * 1e-3) / 1e12
    log(f"prefill M={Mp} K={Kp} N={Np}: variant {pvariant}, {pms * 1e3:.1f} us/step, {tflops:.0f} TFLOP/s "
        f"({tflops / PEAK_FP16_TFLOPS:.1%} of dense fp16 peak)")
    return pms, tflops, pvariant


PEAK_INT8_TOPS = 5033.2   # dense int8 MFMA (v_mfma_i32_32x32x32_i8)


def run_w8a8(args, dev):
    """Opt-in W8A8 route at the prefill shape (M=2048, K=4096, N=11008, fp16):
    activation quantisation + int8 MFMA GEMM, pre-bound C ABI calls replayed
    in a HIP graph; the GEMM alone; hipBLASLt's int8 GEMM (torch._int_mm) at
    the same shape for comparison. Returns a dict for the JSON line."""
    import torch
    from rotalabs_accel import _backend
    from rotalabs_accel.kernels import quantized_matmul as qm
    from workloads import gemm_case, gemm_flops
    Mp, Kp, Np, seedp = PREFILL
    cp = gemm_case(Mp, Kp, Np, seedp, device=dev)
    lib = _backend.load()
    xq = torch.empty((Mp, Kp), dtype=torch.int8, device=dev)
    xs = torch.empty((Mp,), dtype=torch.float16, device=dev)
    y = torch.empty((Mp, Np), dtype=torch.float16, device=dev)
    wcopies = [cp.q, cp.q.clone(), cp.q.clone()]
    ref = qm.int8_gemm(cp.x, cp.q, cp.s, use_cublas=True)

    class _Route:
        def __init__(self, quant=True):
            self.quant = quant

        def run(self, n):
            st = torch.cuda.current_stream().cuda_stream
            for i in range(n):
                if self.quant:
                    _backend.check(lib.ra_quantize_act_rows(cp.x.data_ptr(), Kp, _backend.F16, Mp, Kp,
                                                            xq.data_ptr(), Kp, xs.data_ptr(), 127.0, st))
                _backend.check(lib.ra_w8a8_gemm(xq.data_ptr(), Kp, xs.data_ptr(), wcopies[i % 3].data_ptr(), Kp,
                                                cp.s.data_ptr(), None, 0, y.data_ptr(), Np, _backend.F16,
                                                Mp, Np, Kp, st))
    _Route().run(1)
    torch.cuda.synchronize()
    assert torch.equal(y, ref), "timed W8A8 path differs from int8_gemm(use_cublas=True)"
    steps = max(30, args.prefill_steps // 2)
    route_ms, _ = time_graph(_Route(True), steps, 3, per_graph=9)
    gemm_ms, _ = time_graph(_Route(False), steps, 3, per_graph=9)

    class _IntMM:
        def run(self, n):
            for i in range(n):
                torch._int_mm(xq, wcopies[i % 3].t())
    try:
        imm_ms, _ = time_graph(_IntMM(), steps, 3, per_graph=9)
    except RuntimeError as e:          # hipBLASLt refusing the shape is not fatal here
        log(f"torch._int_mm comparison skipped: {e}")
        imm_ms = float("nan")
    ops = gemm_flops(Mp, Kp, Np)
    tops = ops / (gemm_ms * 1e-3) / 1e12
    rec = {
        "workload": f"W8A8 route M={Mp} K={Kp} N={Np} fp16 (opt-in: int8_gemm(..., use_cublas=True))",
        "route_us": round(route_ms * 1e3, 2),
        "route_TOPS": round(ops / (route_ms * 1e-3) / 1e12, 1),
        "gemm_us": round(gemm_ms * 1e3, 2),
        "gemm_TOPS": round(tops, 1),
        "frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4),
        "hipblaslt_int_mm_us": round(imm_ms * 1e3, 2),
        "hipblaslt_int_mm_TOPS": round(ops / (imm_ms * 1e-3) / 1e12, 1),
    }
    log(f"w8a8: {rec}")
    return rec


MLP = (8192, 28672)   # hidden, intermediate (70B-class decoder MLP, bf16)


# The other decode (M=1) and small-batch shapes of the workload set, timed
# like the headline (graph replay, weight copies cycled past the 256 MB
# Infinity Cache): (group, M, K, N, seed).
CONFIG_SHAPES = (("decode", 1, 4096, 4096, 1), ("decode", 1, 11008, 4096, 3),
                 ("small_batch", 4, 4096, 11008, 4), ("small_batch", 16, 4096, 11008, 5),
                 ("small_batch", 64, 4096, 11008, 6))


def run_shapes(args, dev):
    """Decode and small-batch shapes beside the headline (or only the one
    --shape names): list of dicts."""
    import torch
    import rotalabs_accel as ra
    from rotalabs_accel import _backend
    from workloads import gemm_bytes, gemm_case
    rows = []
    shapes = CONFIG_SHAPES
    if args.shape:
        M, K, N = (int(v) for v in args.shape.split(","))
        shapes = (("shape", M, K, N, 5),)
    for group, M, K, N, seed in shapes:
        c = gemm_case(M, K, N, seed, device=dev, outlier_rows=M > 1)
        ncop = max(2, -(-600_000_000 // (N * K)))
        copies = [c.q] + [c.q.clone() for _ in range(ncop - 1)]
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        launcher = GemmLauncher(c.x, copies, c.s, y)
        launcher.run(1)
        torch.cuda.synchronize()
        assert torch.equal(y, ra.int8_gemm(c.x, c.q, c.s)), "timed path differs from int8_gemm"
        if args.no_graph:
            ms = time_eager(launcher, 600, 60)
        else:
            ms, _ = time_graph(launcher, 600, 60, per_graph=10 * ncop)
        gbs = gemm_bytes(M, K, N) / (ms * 1e-3) / 1e9
        variant = _backend.load().ra_w8a16_gemm_select(M, N, K, _backend.F16)
        rec = {"group": group, "M": M, "K": K, "N": N, "us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
               "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "kernel_variant": VARIANT_NAMES.get(variant, str(variant)),
               "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": round(gbs / PEAK_HBM_GBS, 4),
                            "traffic": measured_traffic(f"{group} M={M} K={K} N={N}")}}
        rows.append(rec)
        log(f"{group} M={M} K={K} N={N}: {rec['us']} us, {rec['GB/s']} GB/s ({rec['frac_hbm']:.1%} of HBM peak)")
        del copies, launcher, c, y
    return rows


PROBE_SRC = os.path.join(HERE, "bench_probe.hip")
PROBE_LIB = os.path.join(HERE, "bench_probe.so")


TRACE_LIB = os.path.join(HERE, "bench_trace.so")


def build_trace_lib(force: bool = False) -> str:
    """Compile the library's sources with -DRA_TUNING -DRA_TRACE (the tiled
    kernel then writes per-workgroup timestamps to a buffer set with
    ra_tune_trace) into bench_trace.so beside this script, unless a build
    newer than every source exists. A measurement build: never loaded by the
    package unless ROTACCEL_LIB points at it."""
    import glob
    import importlib.util
    import subprocess
    csrc = os.path.join(HERE, "rotalabs-accel_amd", "csrc")
    srcs = sorted(glob.glob(os.path.join(csrc, "*.hip")))
    newest = max(os.path.getmtime(f) for f in srcs + glob.glob(os.path.join(csrc, "*.h")))
    if not force and os.path.exists(TRACE_LIB) and os.path.getmtime(TRACE_LIB) >= newest:
        return TRACE_LIB
    spec = importlib.util.spec_from_file_location(
        "rotalabs_accel_build", os.path.join(HERE, "rotalabs-accel_amd", "rotalabs_accel", "_build.py"))
    bld = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bld)
    import concurrent.futures as cf
    import tempfile
    with tempfile.TemporaryDirectory() as td:
        def one(src):
            obj = os.path.join(td, os.path.basename(src) + ".o")
            res = subprocess.run([bld._hipcc(), *bld.compile_flags(), "-DRA_TUNING", "-DRA_TRACE", "-c", src, "-o", obj],
                                 capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError(f"trace build failed for {src}:\n{res.stderr}")
            return obj
        with cf.ThreadPoolExecutor(min(8, len(srcs))) as ex:
            objs = list(ex.map(one, srcs))
        tmp = TRACE_LIB + ".tmp"
        res = subprocess.run([bld._hipcc(), f"--offload-arch={bld.ARCH}", "-shared", "-fPIC", *objs, "-o", tmp],
                             capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"trace link failed:\n{res.stderr}")
    os.replace(tmp, TRACE_LIB)
    return TRACE_LIB


def run_tile_trace(args, dev):
    """Per-workgroup timeline of the tiled GEMM (the bench_trace.so build):
    one traced launch per run after untimed launches on cycled weight copies;
    each workgroup's entry, first K tile ready (prologue copies landed),
    end of the K loop and end of the epilogue (its stores complete) on the
    100 MHz constant clock, plus its shader-clock cycles. Returns a dict."""
    import ctypes
    import statistics as st
    import torch
    import rotalabs_accel as ra
    from workloads import gemm_case
    M, K, N = (int(v) for v in (args.shape or "64,4096,11008").split(","))
    tl = ctypes.CDLL(os.environ["ROTACCEL_LIB"])
    tl.ra_tune_trace.argtypes = [ctypes.c_void_p]
    buf = torch.zeros(1 << 20, dtype=torch.int64, device=dev)
    c = gemm_case(M, K, N, 6, device=dev, outlier_rows=M > 1)
    ncop = max(3, -(-600_000_000 // (N * K)))
    copies = [c.q] + [c.q.clone() for _ in range(ncop - 1)]
    for i in range(3 * ncop):
        ra.int8_gemm(c.x, copies[i % ncop], c.s)
    torch.cuda.synchronize()
    runs = []
    for r in range(3):
        buf.zero_()
        for i in range(4):
            ra.int8_gemm(c.x, copies[(r * 5 + i) % ncop], c.s)
        tl.ra_tune_trace(ctypes.c_void_p(buf.data_ptr()))
        ra.int8_gemm(c.x, copies[(r * 5 + 4) % ncop], c.s)
        tl.ra_tune_trace(None)
        torch.cuda.synchronize()
        recs = [x for x in buf.view(-1, 8).cpu().tolist() if x[0] != 0]
        if not recs:
            raise RuntimeError("no trace records: the shape does not run the traced tiled kernel")
        t0 = min(x[0] for x in recs)
        q = lambda a: {"min": round(min(a), 2), "median": round(st.median(a), 2), "max": round(max(a), 2)}
        rec = {"workgroups": len(recs) // 4, "span_us": round((max(x[3] for x in recs) - t0) / 100.0, 2),
               "entry_us": q([(x[0] - t0) / 100.0 for x in recs]),
               "prologue_us": q([(x[1] - x[0]) / 100.0 for x in recs]),
               "k_loop_us": q([(x[2] - x[1]) / 100.0 for x in recs]),
               "epilogue_us": q([(x[3] - x[2]) / 100.0 for x in recs]),
               "shader_clock_ghz": q([(x[6] - x[5]) / max(1, x[3] - x[0]) / 10.0 for x in recs])}
        # K loop by XCD (hardware XCC id) for the workgroups of the first round (entered within 5 us)
        # and the later ones
        for label, first in (("k_loop_us_by_xcd_round1", True), ("k_loop_us_by_xcd_later", False)):
            by = {}
            for x in recs:
                if ((x[0] - t0) / 100.0 < 5.0) == first:
                    by.setdefault(int(x[4] >> 32), []).append((x[2] - x[1]) / 100.0)
            rec[label] = {str(k): round(st.median(v), 2) for k, v in sorted(by.items())}
        log(f"tile trace M={M} K={K} N={N} run {r}: {rec}")
        runs.append(rec)
    return {"workload": f"tiled GEMM M={M} K={K} N={N} fp16, per-workgroup timeline (trace build)", "runs": runs}


def build_probe(force: bool = False) -> str:
    """Compile the measurement probe (bench_probe.hip, a plain streaming read
    with the decode kernels' access pattern; not part of the library) into
    bench_probe.so with the library's hipcc flags, unless a build newer than
    the source exists. Returns the library path."""
    if (not force and os.path.exists(PROBE_LIB)
            and os.path.getmtime(PROBE_LIB) >= os.path.getmtime(PROBE_SRC)):
        return PROBE_LIB
    import importlib.util
    import subprocess
    spec = importlib.util.spec_from_file_location(
        "rotalabs_accel_build", os.path.join(HERE, "rotalabs-accel_amd", "rotalabs_accel", "_build.py"))
    bld = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bld)
    tmp = PROBE_LIB + ".tmp"
    res = subprocess.run([bld._hipcc(), *bld.compile_flags(), "-shared", PROBE_SRC, "-o", tmp],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SRC}:\n{res.stderr}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def run_read_ceiling(args, dev):
    """Single-launch floors of the M=1 decode shapes, beside the GEMM
    (int8_gemm's kernel) on the same weight copies: a plain read of the int8
    [N, K] weight bytes with the M=1 kernels' access pattern and grid (one
    row per wave, every 1 KB window of the row in flight, non-temporal loads,
    8 rows per workgroup up to N = 8192, else 4), and the same read plus the
    GEMV's x copy into LDS and y store ("io"). Weight copies are cycled past
    the Infinity Cache; graph replay. Returns a list of dicts."""
    import ctypes
    import torch
    from workloads import gemm_bytes, gemm_case
    lib = ctypes.CDLL(build_probe())
    lib.rap_stream_rows.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p]
    lib.rap_stream_rows.restype = ctypes.c_int
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    rows = []
    for (K, N, seed) in ((4096, 4096, 1), (4096, 11008, 2), (11008, 4096, 3), (4096, 44032, 4)):
        c = gemm_case(1, K, N, seed, device=dev)
        ncop = max(2, -(-600_000_000 // (N * K)))
        copies = [c.q] + [c.q.clone() for _ in range(ncop - 1)]
        wpg = 8 if N <= 8192 else 4
        y = torch.empty((1, N), dtype=torch.float16, device=dev)

        class _Read:
            def __init__(self, io):
                self.io = io

            def run(self, n):
                st = torch.cuda.current_stream().cuda_stream
                for i in range(n):
                    rc = lib.rap_stream_rows(copies[i % ncop].data_ptr(), K, N, K, wpg, self.io, c.x.data_ptr(),
                                             y.data_ptr(), sink.data_ptr(), st)
                    if rc:
                        raise RuntimeError(f"rap_stream_rows failed with {rc}")
        read_ms, _ = time_graph(_Read(0), 600, 60, per_graph=10 * ncop)
        io_ms, _ = time_graph(_Read(1), 600, 60, per_graph=10 * ncop)
        gemm_ms, _ = time_graph(GemmLauncher(c.x, copies, c.s, y), 600, 60, per_graph=10 * ncop)
        rec = {"K": K, "N": N, "weight_bytes": N * K, "read_us": round(read_ms * 1e3, 2),
               "read_GB/s": round(N * K / (read_ms * 1e-3) / 1e9, 1), "io_us": round(io_ms * 1e3, 2),
               "gemm_us": round(gemm_ms * 1e3, 2),
               "gemm_GB/s": round(gemm_bytes(1, K, N) / (gemm_ms * 1e-3) / 1e9, 1),
               "gemm_over_read": round(gemm_ms / read_ms, 3), "gemm_over_io": round(gemm_ms / io_ms, 3)}
        rows.append(rec)
        log(f"ceiling K={K} N={N}: read {rec['read_us']} us ({rec['read_GB/s']} GB/s), read+io {rec['io_us']} us, "
            f"GEMM {rec['gemm_us']} us ({rec['gemm_over_read']}x read, {rec['gemm_over_io']}x read+io)")
        del copies, c
    return rows


def run_mlp(args, dev):
    """Fused decoder MLP block (RMSNorm -> gate/up + SwiGLU -> down, bf16,
    H=8192, I=28672) at M=1 and M=4096, random int8 weights generated on the
    GPU; returns a dict for the JSON line."""
    import torch
    import rotalabs_accel as ra
    from rotalabs_accel.kernels.mlp import int8_mlp
    from workloads import mlp_bytes, mlp_flops
    H, I = MLP
    g = torch.Generator(device=dev).manual_seed(11)
    norm_w = (1.0 + 0.01 * torch.randn(H, device=dev, generator=g)).to(torch.bfloat16)
    q_gu, s_gu = ra.quantize_weight_per_channel(torch.randn(2 * I, H, device=dev, generator=g) * 0.02)
    q_d, s_d = ra.quantize_weight_per_channel(torch.randn(H, I, device=dev, generator=g) * 0.02)
    out = {}
    rows_wanted = {int(v) for v in args.mlp_rows.split(",")}
    for M, calls in ((1, 20), (17, 20), (4096, 3)):
        x = torch.randn(M, H, device=dev, generator=g).to(torch.bfloat16)
        if M not in rows_wanted:
            continue

        class _Step:
            def run(self, n):
                for _ in range(n):
                    int8_mlp(x, norm_w, q_gu, s_gu, q_d, s_d)
        if args.no_graph:
            ms = time_eager(_Step(), calls * 3, calls)
        else:
            ms, _ = time_graph(_Step(), calls * 3, calls, per_graph=calls)
        rec = {"us_per_call": round(ms * 1e3, 2), "steps": calls * 3}
        traffic = measured_traffic(f"mlp M={M} H={H} I={I}")
        if M <= 64:   # weight-streaming (HBM-bound) sizes
            gbs = mlp_bytes(M, H, I) / (ms * 1e-3) / 1e9
            rec.update({"GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                                     "traffic": traffic}})
        else:
            tf = mlp_flops(M, H, I) / (ms * 1e-3) / 1e12
            rec.update({"TFLOP/s": round(tf, 1), "frac_mfma": round(tf / PEAK_FP16_TFLOPS, 4),
                        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_FP16_TFLOPS,
                                     "unit": "TFLOP/s", "frac": round(tf / PEAK_FP16_TFLOPS, 4),
                                     "traffic": traffic}})
        out[f"M={M}"] = rec
        log(f"mlp M={M} H={H} I={I} bf16: {rec}")
        del x
    if args.mlp_rows != "1,17,4096":
        return out
    # RMSNorm of x + residual (the block's prologue in a decoder layer), HBM-bound:
    # reads x, residual, weight, writes y; 3 input sets (384 MiB) cycled so the
    # reads come from HBM, not the 256 MB Infinity Cache.
    M = 4096
    xs = [torch.randn(M, H, device=dev, generator=g).to(torch.bfloat16) for _ in range(3)]
    rs = [torch.randn(M, H, device=dev, generator=g).to(torch.bfloat16) for _ in range(3)]

    class _Norm:
        def run(self, n):
            for i in range(n):
                ra.rmsnorm_residual_fused(xs[i % 3], rs[i % 3], norm_w)
    ms, _ = time_graph(_Norm(), 30, 9, per_graph=9)
    gbs = (6 * M * H + 2 * H) / (ms * 1e-3) / 1e9
    rec = {"us_per_call": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
    out[f"rmsnorm_residual M={M}"] = rec
    log(f"rmsnorm_residual M={M} H={H} bf16: {rec}")
    del xs, rs
    # Int8 KV-cache codec (QuantizedTensor, per channel): one bf16 K or V block
    # [batch 8, heads 32, seq 4096, head_dim 128] (256 MiB), 2 blocks cycled;
    # reads 2 B and writes 1 B per element plus a 2-byte scale per row.
    from rotalabs_accel.speculative import QuantizedTensor
    shape = (8, 32, 4096, 128)
    kvs = [torch.randn(shape, device=dev, generator=g).to(torch.bfloat16) for _ in range(2)]

    class _Codec:
        def run(self, n):
            for i in range(n):
                QuantizedTensor(kvs[i % 2], bits=8)
    ms, _ = time_graph(_Codec(), 12, 4, per_graph=4)
    elems = shape[0] * shape[1] * shape[2] * shape[3]
    gbs = (3 * elems + 2 * elems // shape[3]) / (ms * 1e-3) / 1e9
    rec = {"us_per_call": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
    out["kv_codec int8 bf16 [8,32,4096,128]"] = rec
    log(f"kv codec int8 per-channel bf16 {list(shape)}: {rec}")
    del kvs
    return out


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "multi-GPU sharding is design-only.", file=sys.stderr)
        sys.exit(2)

    if args.only == "tile-trace":  # the trace build of the library, loaded in place of the release one
        os.environ["ROTACCEL_LIB"] = build_trace_lib()
    import torch
    from rotalabs_accel import _backend
    from workloads import gemm_bytes

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        copy_calibration()
        return
    _backend.load()
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} ({getattr(props, 'gcnArchName', '?')}), {props.multi_processor_count} CUs")

    if args.only == "tile-trace":
        print(json.dumps(run_tile_trace(args, dev)), flush=True)
        return

    # ---------------- decode M=1 (headline) ----------------
    M, K, N, seed = DECODE
    ms = ms_eager = ms_py = gbs = float("nan")
    timed_steps, variant = 0, None
    if args.only in ("all", "decode"):
        ms, ms_eager, ms_py, gbs, timed_steps, variant = run_decode(args, dev)
    dbytes = gemm_bytes(M, K, N)

    # ---------------- prefill M=2048 ----------------
    Mp, Kp, Np, seedp = PREFILL
    pms = tflops = float("nan")
    pvariant = None
    if args.only in ("all", "prefill"):
        pms, tflops, pvariant = run_prefill(args, dev)
    Ml, Kl, Nl, _ = PREFILL_LARGE
    lms = ltflops = float("nan")
    lvariant = None
    if args.only in ("all", "prefill_large"):
        lms, ltflops, lvariant = run_prefill(args, dev, PREFILL_LARGE)
    w8a8 = None
    if args.only in ("all", "w8a8"):
        w8a8 = run_w8a8(args, dev)
    shapes = None
    if args.only in ("all", "shapes"):
        shapes = run_shapes(args, dev)
    ceiling = None
    if args.only in ("all", "ceiling"):
        ceiling = run_read_ceiling(args, dev)
    mlp = None
    if args.only == "mlp" or (args.only == "all" and not args.no_mlp):
        mlp = run_mlp(args, dev)
    if args.only != "all":
        return

    # ---------------- CPU baseline ----------------
    cpu = cpu_prefill = cpu_mlp = None
    if not args.no_cpu:
        log(f"CPU baseline (reference fallback restated, {os.cpu_count()} threads, ~{args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(M, K, N, seed, args.cpu_seconds)
        log(f"CPU: {cpu['med_s'] * 1e3:.2f} ms/call, {cpu['gbs']:.2f} GB/s over {cpu['calls']} calls")
        cpu_prefill = cpu_baseline_prefill(args.cpu_seconds)
        log(f"CPU prefill sample: {cpu_prefill}")
        if mlp is not None:
            cpu_mlp = cpu_baseline_mlp(args.cpu_seconds)
            log(f"CPU MLP: {cpu_mlp}")

    out = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": timed_steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"W8A16 decode GEMM M={M} K={K} N={N}: fp16 x ~N(0,1), int8 per-channel W from "
                        f"N(0,0.02) (seed {seed}), {N_COPIES} resident weight copies cycled per step",
            "M": M, "K": K, "N": N,
            "bytes_per_step": dbytes,
            "kernel_variant": VARIANT_NAMES.get(variant, str(variant)),
            "timing": ("host-launched loop" if args.no_graph else
                       f"{timed_steps // (10 * N_COPIES)} replays of a HIP graph of {10 * N_COPIES} launches and "
                       f"{timed_steps % (10 * N_COPIES)} host-launched C ABI calls, all queued behind an untimed "
                       "graph replay enqueued just before the start event") + "; HIP events on the launch stream",
            "graph_launch_latency_us": GRAPH_LATENCY.get(10 * N_COPIES),
            "host_launched_us_per_step": round(ms_eager * 1e3, 3),
            "python_int8_gemm_eager_us_per_call": round(ms_py * 1e3, 3),
            "steps_note": f"steps = launches timed, exactly --steps (whole {10 * N_COPIES}-launch graphs plus "
                          "the remainder launched from the host); graph_launch_latency_us = one replay of a "
                          f"{10 * N_COPIES}-launch graph from an idle stream minus {10 * N_COPIES} steady steps, "
                          "kept out of the timed region",
        },
        "roofline": {
            "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4),
            "traffic": measured_traffic(f"decode M={M} K={K} N={N}"),
        },
        "prefill": {
            "metric": "int8_gemm TFLOP/s @M=2048 K=4096 N=11008",
            "value": round(tflops, 1), "unit": "TFLOP/s", "ms_per_step": pms, "steps": args.prefill_steps,
            "kernel_variant": VARIANT_NAMES.get(pvariant, str(pvariant)),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": PEAK_FP16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP16_TFLOPS, 4),
                         "traffic": measured_traffic(f"prefill M={Mp} K={Kp} N={Np}")},
        },
        "prefill_large": {
            "metric": f"int8_gemm TFLOP/s @M={Ml} K={Kl} N={Nl}",
            "value": round(ltflops, 1), "unit": "TFLOP/s", "ms_per_step": lms, "steps": args.prefill_steps,
            "kernel_variant": VARIANT_NAMES.get(lvariant, str(lvariant)),
            "roofline": {"bound": "mfma", "achieved": round(ltflops, 1), "peak": PEAK_FP16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ltflops / PEAK_FP16_TFLOPS, 4),
                         "traffic": measured_traffic(f"prefill M={Ml} K={Kl} N={Nl}")},
        },
    }
    if shapes is not None:
        out["shapes"] = {"workload": "the other decode (M=1) and small-batch shapes: fp16 x ~N(0,1) (1% of "
                                     "rows x20 for M > 1), int8 per-channel W from N(0,0.02), weight copies "
                                     "cycled past the Infinity Cache, HIP graph replay", "rows": shapes}
    if ceiling is not None:
        out["decode_read_ceiling"] = {
            "workload": "single-launch floors of the M=1 shapes: a plain streaming read of the weights with "
                        "the decode kernels' pattern and grid (one row per wave, all windows in flight, "
                        "non-temporal) and the same read plus the x copy into LDS and the y store (io), beside "
                        "the GEMM on the same copies; graph replay", "rows": ceiling}
    if w8a8 is not None:
        out["w8a8"] = w8a8
    if mlp is not None:
        out["mlp"] = {"workload": "fused decoder MLP (RMSNorm -> int8 gate/up + SwiGLU -> int8 down), bf16, "
                                  "H=8192, I=28672, random int8 per-channel weights", **mlp}
    if cpu_prefill is not None:
        out["prefill"]["cpu_baseline"] = cpu_prefill
    if cpu_mlp is not None:
        out["mlp"]["cpu_baseline"] = cpu_mlp
    if cpu is not None:
        out["cpu_baseline"] = {
            "value": round(cpu["gbs"], 3), "unit": "GB/s", "cores": cpu["threads"], "kind": "port", **host_info(),
            "sample": f"{cpu['calls']} calls of the reference fallback (dequantize + F.linear) at "
                      f"M={M} K={K} N={N} fp16 on the host CPU, median {cpu['med_s'] * 1e3:.2f} ms/call",
        }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
