"""The oracle is pinned before it is trusted (CPU only).

* fp32 per-channel quantization: numpy closed form == independent C
  restatement, bit for bit; invariants; round-half-even tie rows; row
  independence; brute force on tiny inputs.
* fp16/bf16 quantization, int8_gemm_torch outputs, quantization-error
  metrics, rmsnorm_torch, swiglu_torch: golden vectors from the reference.
* GEMM: the float64 reference equals a brute-force triple loop (C) and exact
  known answers (integer inputs, power-of-two scales).
"""
import os

import numpy as np
import pytest
import torch

from oracle import cquant, fallback
from oracle import quant as oq


def _edge_rows(rng, rows=48, cols=96):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[0] = 0
    w[1] = 0
    w[1, 3] = -0.5
    w[2] = np.linspace(-1, 1, cols, dtype=np.float32)
    w[3] = 0
    w[3, 0] = 127.0
    w[3, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -125.5]
    w[4] *= 1e-30
    w[5, :] = 3.0
    return w


def test_fp32_quant_numpy_equals_c():
    rng = np.random.default_rng(0)
    for shape in [(48, 96), (7, 1), (1, 4096), (33, 1000)]:
        w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        q1, s1 = oq.quantize_weight_per_channel(w)
        q2, s2 = cquant.quantize_rows_f32(w)
        assert np.array_equal(q1, q2) and np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    w = _edge_rows(rng)
    q1, s1 = oq.quantize_weight_per_channel(w)
    q2, s2 = cquant.quantize_rows_f32(w)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


def test_fp32_quant_invariants_and_ties():
    rng = np.random.default_rng(1)
    w = _edge_rows(rng)
    q, s = oq.quantize_weight_per_channel(w)
    assert q.dtype == np.int8 and s.dtype == np.float32 and q.shape == w.shape and s.shape == (w.shape[0],)
    assert np.abs(q.astype(np.int32)).max() <= 127
    # zero row -> scale 1, q 0
    assert s[0] == 1.0 and not q[0].any()
    # scale is the single fp32 rounding of max/127
    amax = np.abs(w).max(axis=1)
    expect = (amax / np.float32(127)).astype(np.float32)
    expect[expect == 0] = 1
    assert np.array_equal(s, expect)
    # the row maximum maps to +-127
    for r in range(1, w.shape[0]):
        k = np.argmax(np.abs(w[r]))
        if amax[r] / np.float32(127) > 0:
            assert abs(int(q[r, k])) == 127
    # row 3: max 127 -> s == 1 exactly; ties round half to even
    assert s[3] == 1.0
    assert q[3, 1:9].tolist() == [0, 2, 2, 0, -2, -2, 126, -126]
    # constant row -> all 127
    assert (q[5] == 127).all()


def test_fp32_quant_row_independence():
    rng = np.random.default_rng(2)
    a = (rng.standard_normal((20, 64)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((30, 64)) * 0.02).astype(np.float32)
    qa, sa = oq.quantize_weight_per_channel(a)
    qb, sb = oq.quantize_weight_per_channel(b)
    qc, sc = oq.quantize_weight_per_channel(np.concatenate([a, b]))
    assert np.array_equal(qc, np.concatenate([qa, qb])) and np.array_equal(sc, np.concatenate([sa, sb]))


def test_fp32_quant_brute_force():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((5, 7)) * 0.1).astype(np.float32)
    q, s = oq.quantize_weight_per_channel(w)
    for r in range(5):
        m = max(abs(float(v)) for v in w[r])
        sr = float(np.float32(np.float32(m) / np.float32(127)))
        assert s[r] == np.float32(sr)
        for k in range(7):
            v = float(np.float32(w[r, k] / np.float32(sr)))
            rq = int(np.rint(v))  # numpy rint: half to even
            assert q[r, k] == max(-128, min(127, rq))


@pytest.mark.parametrize("name", ["f16", "bf16"])
def test_reduced_precision_quant_golden(golden, name):
    wb = golden[f"qpc_{name}_w"]
    w32 = wb.view(np.float16).astype(np.float32) if name == "f16" else oq.bf16_bits_to_f32(wb)
    q, s = oq.quantize_weight_per_channel(w32, name)
    assert np.array_equal(q, golden[f"qpc_{name}_q"])
    assert np.array_equal(s, golden[f"qpc_{name}_s"])
    qt, st = oq.quantize_symmetric(w32, name)
    assert np.array_equal(qt, golden[f"qpt_{name}_q"])
    assert np.array_equal(np.atleast_1d(st), golden[f"qpt_{name}_s"])


def test_quant_error_metrics_golden(golden):
    x = golden["qerr_x"]
    q, s = oq.quantize_symmetric(x)
    e = oq.calculate_quantization_error(x, q, s)
    got = [e["max_abs_error"], e["mean_abs_error"], e["relative_error_pct"], e["snr_db"]]
    np.testing.assert_allclose(got, golden["qerr_vals"], rtol=1e-5)
    q2, s2 = oq.quantize_weight_per_channel(x)
    e2 = oq.calculate_quantization_error(x, q2, s2, dim=0)
    got2 = [e2["max_abs_error"], e2["mean_abs_error"], e2["relative_error_pct"], e2["snr_db"]]
    np.testing.assert_allclose(got2, golden["qerr_pc_vals"], rtol=1e-5)


def _t16(bits, dt):
    return torch.from_numpy(bits.astype(np.int16)).view(dt)


@pytest.mark.parametrize("name,dt", [("f16", torch.float16), ("bf16", torch.bfloat16), ("f32", torch.float32)])
def test_int8_gemm_fallback_golden(golden, name, dt):
    x = torch.from_numpy(golden["gemm_x_f32"]).to(dt)
    q = torch.from_numpy(golden["gemm_q"])
    s = torch.from_numpy(golden["gemm_s"])
    b = torch.from_numpy(golden["gemm_b_f32"]).to(dt)
    y = fallback.int8_gemm_ref(x, q, s)
    yb = fallback.int8_gemm_ref(x, q, s, b)
    if dt == torch.float32:
        assert np.array_equal(y.numpy(), golden["gemm_y_f32"])
        assert np.array_equal(yb.numpy(), golden["gemm_yb_f32"])
    else:
        assert torch.equal(y, _t16(golden[f"gemm_y_{name}"], dt))
        assert torch.equal(yb, _t16(golden[f"gemm_yb_{name}"], dt))


def test_reference_unit_case_golden(golden):
    x = torch.from_numpy(golden["reftest_x"])
    w = torch.from_numpy(golden["reftest_w"])
    y = fallback.int8_gemm_ref(x, w, torch.ones(128))
    assert y.shape == (2, 8, 128)
    assert np.array_equal(y.numpy(), golden["reftest_y"])


def test_rmsnorm_swiglu_golden(golden):
    x = _t16(golden["rms_x_bf16"], torch.bfloat16)
    w = _t16(golden["rms_w_bf16"], torch.bfloat16)
    assert torch.equal(fallback.rmsnorm_ref(x, w), _t16(golden["rms_y_bf16"], torch.bfloat16))
    xh = _t16(golden["rms_x_f16"], torch.float16)
    wf = torch.from_numpy(golden["rms_w_f32"])
    y = fallback.rmsnorm_ref(xh, wf)
    assert y.dtype == torch.float32
    assert np.array_equal(y.numpy(), golden["rms_y_f16w32"])
    g = _t16(golden["swiglu_g_bf16"], torch.bfloat16)
    u = _t16(golden["swiglu_u_bf16"], torch.bfloat16)
    assert torch.equal(fallback.swiglu_ref(g, u), _t16(golden["swiglu_y_bf16"], torch.bfloat16))


def test_gemm_f64_equals_brute_force():
    rng = np.random.default_rng(4)
    for (M, K, N) in [(1, 48, 43), (17, 64, 5), (3, 16, 16)]:
        x = rng.standard_normal((M, K))
        q = rng.integers(-127, 128, (N, K)).astype(np.int8)
        s = (rng.random(N).astype(np.float32) * 0.01 + 1e-3).astype(np.float32)
        np.testing.assert_allclose(fallback.gemm_f64(x, q, s), cquant.w8a16_gemm_f64(x, q, s), rtol=1e-12, atol=1e-12)


def test_gemm_known_answer():
    # integer x, scale = 2^-e: every partial sum is an exact small integer
    rng = np.random.default_rng(5)
    M, K, N = 4, 64, 8
    x = rng.integers(-2, 3, (M, K)).astype(np.float64)
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = np.full(N, 0.25, np.float32)
    exact = (x.astype(np.int64) @ q.astype(np.int64).T) * 0.25
    assert np.array_equal(fallback.gemm_f64(x, q, s), exact)
    # scale == 1 reduces to the integer product
    assert np.array_equal(fallback.gemm_f64(x, q, np.ones(N, np.float32)), exact * 4)


def test_dequantize_closed_form():
    rng = np.random.default_rng(6)
    q = rng.integers(-128, 128, (16, 32)).astype(np.int8)
    s = (rng.random(16) * 0.05).astype(np.float32)
    ref = fallback.dequantize_ref(torch.from_numpy(q), torch.from_numpy(s), torch.float16)
    mine = oq.dequantize(q, s, "f16")
    assert np.array_equal(ref.float().numpy(), mine)
    refb = fallback.dequantize_ref(torch.from_numpy(q), torch.from_numpy(s), torch.bfloat16)
    assert np.array_equal(refb.float().numpy(), oq.dequantize(q, s, "bf16"))


@pytest.mark.parametrize("tdt,dt", [(torch.bfloat16, "bf16"), (torch.float16, "f16")])
def test_rmsnorm_exact_oracle_pinned(golden, tdt, dt):
    """rmsnorm_exact_ref (normalization.py:43-45 with exactly rounded fp32
    ops) is pinned three ways:
    * rows whose fp32 sum of squares is exact in any order (multiples of 1/8
      up to 4 in magnitude; a row of +-2^-10, where eps is half the mean):
      equal bit for bit to torch's evaluation of the fallback;
    * random rows (the golden vectors' and wider ones): equal to torch's on
      all but a sliver (torch's fp32 sum rounds in its own order) and within
      one output ulp everywhere;
    * a float64 closed form x * w / sqrt(mean(x^2) + eps) within two output
      ulps (a dropped eps, a wrong divisor or a missing rounding fails one
      of these)."""
    from oracle.quant import round_to
    g = torch.Generator().manual_seed(9)
    H = 8192
    exact = (torch.randint(-32, 33, (6, H), generator=g).float() / 8)
    exact[5] = torch.where(torch.rand(H, generator=g) < 0.5, -1.0, 1.0) * 2.0 ** -10
    x = exact.to(tdt)
    w = (1 + 0.01 * torch.randn(H, generator=g)).to(tdt)
    got = fallback.rmsnorm_exact_ref(x.float().numpy(), w.float().numpy(), 1e-6, dt)
    np.testing.assert_array_equal(got, fallback.rmsnorm_ref(x, w, 1e-6).float().numpy())
    ulp = 2.0 ** -7 if dt == "bf16" else 2.0 ** -10
    rand = [(torch.randn(64, H, generator=g) * 2).to(tdt)]
    if dt == "bf16":
        rand.append(_t16(golden["rms_x_bf16"], tdt))
    for xr in rand:
        wr = (1 + 0.01 * torch.randn(xr.shape[-1], generator=g)).to(tdt)
        got = fallback.rmsnorm_exact_ref(xr.float().numpy(), wr.float().numpy(), 1e-6, dt)
        tor = fallback.rmsnorm_ref(xr, wr, 1e-6).float().numpy()
        assert (got == tor).mean() > 0.999
        np.testing.assert_allclose(got, tor, rtol=ulp, atol=0)
        x64 = xr.double().numpy()
        closed = x64 * wr.double().numpy() / np.sqrt((x64 * x64).mean(-1, keepdims=True) + 1e-6)
        np.testing.assert_allclose(got, closed, rtol=2 * ulp, atol=2.0 ** -24)   # fp16 subnormal step
        assert np.array_equal(got, round_to(got, dt))


def test_rmsnorm_residual_oracle_pinned(golden):
    """rmsnorm_residual_ref (normalization.py:48-64) pinned by identities:
    a zero residual is rmsnorm of x; with equal dtypes it is rmsnorm of the
    rounded sum (so a dropped or mis-signed residual term, or a rounding to
    the wrong dtype, fails); mixed dtypes round the sum in the promoted type
    and the normalised value in x's dtype (float64 closed form, 1 ulp)."""
    x = _t16(golden["rms_x_bf16"], torch.bfloat16)
    w = _t16(golden["rms_w_bf16"], torch.bfloat16)
    ref = _t16(golden["rms_y_bf16"], torch.bfloat16)
    assert torch.equal(fallback.rmsnorm_residual_ref(x, torch.zeros_like(x), w), ref)
    g = torch.Generator().manual_seed(3)
    r = (torch.randn(x.shape, generator=g) * 0.5).to(torch.bfloat16)
    assert torch.equal(fallback.rmsnorm_residual_ref(x, r, w), fallback.rmsnorm_ref(x + r, w))
    assert not torch.equal(fallback.rmsnorm_residual_ref(x, r, w), fallback.rmsnorm_ref(x - r, w))
    # fp16 x + fp32 residual: the sum stays fp32, the normalised value is fp16
    xh = (torch.randn(4, 96, generator=g) * 2).half()
    rf = torch.randn(4, 96, generator=g) * 0.25
    wf = 1 + 0.01 * torch.randn(96, generator=g)
    y = fallback.rmsnorm_residual_ref(xh, rf, wf)
    assert y.dtype == torch.float32
    v = xh.double() + rf.double()
    n = (v / torch.sqrt((v * v).mean(dim=-1, keepdim=True) + 1e-6)).half().double() * wf.double()
    assert torch.allclose(y.double(), n, rtol=2 ** -10, atol=1e-6)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("bits", [8, 4])
def test_kv_codec_restatements_agree(dtype, bits):
    """The KV-cache codec (kv_compression.py:51-78) restated twice -- numpy
    closed form with explicit roundings, and the reference's torch ops on the
    CPU -- agree bit for bit, including all-zero rows (fp16's 1e-8 floor
    underflows: 0/0 -> 0), exact .5 ties and rows of one repeated value; the
    invariants |q| <= qmax and |q| = qmax at each row's |max| (fp32; >= qmax-1
    when the scale is rounded to 16 bits) hold."""
    g = torch.Generator().manual_seed(bits)
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dtype]
    t = (torch.randn(6, 40, generator=g) * 3).to(tdt)
    t[1] = 0
    t[2, :] = 2.5                                   # one repeated value
    qmax = 2 ** (bits - 1) - 1
    t[3, 0] = float(qmax)                            # scale 1 (exactly representable)
    t[3, 1:6] = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5])
    t[4] = (torch.randn(40, generator=g) * 1e-6).to(tdt)  # fp16: the floored scale rounds to 0 -> +-inf -> clamp
    qt, st = fallback.quantized_tensor_ref(t, bits)
    qn, sn = oq.quantized_tensor_rows(t.float().numpy(), dtype, bits)
    assert np.array_equal(qt.numpy(), qn)
    assert np.array_equal(st.float().numpy(), sn)
    assert qt[3, 1:6].tolist() == [0, 2, 2, 0, -2]  # round half to even
    assert (qt.int().abs() <= qmax + 1).all() and (qt[1] == 0).all()
    if dtype == "f16" and bits == 8:     # amax / 127 of a 1e-6 row underflows fp16
        nz = t[4] != 0
        assert st[4].item() == 0 and (qt[4][nz].int().abs() >= qmax).all()
    nz = t.abs().amax(dim=-1) > 0
    # the scale rounded to a 16-bit dtype can exceed amax / qmax by half an ulp
    assert (qt.abs().amax(dim=-1)[nz] >= (qmax if dtype == "f32" else qmax - 1)).all()


# ------------------------------------------------------------- W8A8 route
def _act_rows(tdt, seed=0, M=48, K=300):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * torch.rand(M, 1, generator=g) * 8).to(tdt)
    x[0] = 0                       # all-zero row: a = round(1e-5)
    x[1, 3] = float("nan")         # NaN propagates through amax: q = 0, xs = NaN
    x[2, 7] = float("inf")         # inf row: xs = inf, q = 0
    x[3] = 1e-7                    # below the 1e-5 floor
    x[4] = 3e-5
    x[5] = -2.0                    # constant row: q = -127
    x[6, :4] = torch.tensor([1.0, -1.0, 0.5, -0.5])  # tie candidates
    x[7] = 60000.0 if tdt == torch.float16 else 3e38
    return x


@pytest.mark.parametrize("tdt,dt", [(torch.float16, "f16"), (torch.bfloat16, "bf16")])
def test_w8a8_activation_quant_oracle_pinned(tdt, dt):
    """The numpy restatement of quantized_matmul.py:85-87 equals torch's CPU
    evaluation of the reference's own expression (which pins the rounding
    model: 127 / a is reciprocal(a) * 127, each op rounded to the dtype; a
    plain fp32 127 / a differs on a large share of rows), on random rows and
    edge rows."""
    x = _act_rows(tdt)
    absmax = x.abs().amax(dim=1, keepdim=True).clamp(min=1e-5)
    xs_t = (absmax / 127.0).to(tdt).reshape(-1)
    q_t = (x * (127.0 / absmax)).round().clamp(-128, 127).to(torch.int8)
    q, xs = oq.quantize_activations_rows(x.float().numpy(), dt)
    np.testing.assert_array_equal(q, q_t.numpy())
    np.testing.assert_array_equal(xs, xs_t.float().numpy())
    # invariants: |q| <= 127 and the row max lands on +-127 (or 126 for a
    # rounded multiplier) for every finite row above the floor
    fin = np.isfinite(x.float().numpy()).all(1) & (np.abs(x.float().numpy()).max(1) > 1e-4)
    assert np.abs(q.astype(int)).max() <= 128
    assert (np.abs(q[fin].astype(int)).max(1) >= 126).all()
    assert (q[1] == 0).all() and np.isnan(xs[1]) and np.isinf(xs[2]) and (q[2] == 0).all()
    assert (q[5] == -127).all()


@pytest.mark.parametrize("c", [100.0, 63.5, 200.0])
def test_w8a8_activation_quant_general_act_scale(c):
    """The restatement with another act_scale equals torch's CPU evaluation of
    the reference's expression with that constant (quantized_matmul.py:85-87,
    act_scale argument at :48)."""
    for tdt, dt in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        x = _act_rows(tdt)
        absmax = x.abs().amax(dim=1, keepdim=True).clamp(min=1e-5)
        xs_t = (absmax / c).to(tdt).reshape(-1)
        q_t = (x * (c / absmax)).round().clamp(-128, 127).to(torch.int8)
        q, xs = oq.quantize_activations_rows(x.float().numpy(), dt, act_scale=c)
        np.testing.assert_array_equal(q, q_t.numpy())
        np.testing.assert_array_equal(xs, xs_t.float().numpy())


def test_w8a8_scalar_division_forms_agree():
    """a / 127 on the CPU (true division) and on CUDA (multiply by the fp32
    reciprocal of a CPU scalar) round to the same 16-bit value for every
    finite fp16 and bf16 a, so the restatement holds for either device."""
    bits = np.arange(1 << 16, dtype=np.uint16)
    a16 = bits.view(np.float16).astype(np.float32)
    a16 = a16[np.isfinite(a16)]
    np.testing.assert_array_equal((a16 / np.float32(127)).astype(np.float16),
                                  (a16 * (np.float32(1) / np.float32(127))).astype(np.float16))
    ab = oq.bf16_bits_to_f32(bits)
    ab = ab[np.isfinite(ab)]
    np.testing.assert_array_equal(oq.round_to((ab / np.float32(127)).astype(np.float32), "bf16"),
                                  oq.round_to((ab * (np.float32(1) / np.float32(127))).astype(np.float32), "bf16"))


def test_w8a8_gemm_oracle_pinned():
    """Integer sums against a brute-force triple loop; scaling against the
    reference's fp16 dequantisation chain (quantized_matmul.py:38-40, run by
    torch on the CPU) where that chain does not overflow (|sum| <= 65504),
    and inf from that chain where it does."""
    g = np.random.default_rng(3)
    M, N, K = 5, 7, 64
    xq = g.integers(-128, 128, (M, K)).astype(np.int8)
    q = g.integers(-127, 128, (N, K)).astype(np.int8)
    xs = oq.round_to(g.uniform(1e-3, 1e-1, M).astype(np.float32), "f16")
    s = g.uniform(1e-4, 1e-2, N).astype(np.float32)
    acc = np.array([[sum(int(xq[m, k]) * int(q[n, k]) for k in range(K)) for n in range(N)] for m in range(M)])
    y = oq.w8a8_gemm_rows(xq, xs, q, s, "f16")
    ref_chain = (torch.from_numpy(acc).to(torch.int32).half() * torch.from_numpy(xs).half()[:, None]
                 * torch.from_numpy(s).half()[None, :]).float().numpy()
    small = np.abs(acc) <= 65504
    assert small.any() and (~small).any()
    np.testing.assert_allclose(y[small], ref_chain[small], rtol=1e-2, atol=1e-2)
    assert np.isinf(ref_chain[~small]).all() and np.isfinite(y).all()
    # closed form: power-of-two scales keep the scaling exact
    y2 = oq.w8a8_gemm_rows(xq, np.full(M, 2.0 ** -10, np.float32), q, np.full(N, 2.0 ** -6, np.float32), "f32")
    np.testing.assert_array_equal(y2, acc.astype(np.float32) * 2.0 ** -16)
    # bias is added after the scaling, in fp32
    b = oq.round_to(g.uniform(-1, 1, N).astype(np.float32), "bf16")
    y3 = oq.w8a8_gemm_rows(xq, xs, q, s, "f32", b)
    np.testing.assert_array_equal(y3, oq.w8a8_gemm_rows(xq, xs, q, s, "f32") + b[None, :])


@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16, torch.float32])
def test_swiglu_with_bias_oracle_pinned(tdt):
    """swiglu_with_bias_ref (swiglu.py:201-218: fp32 math, one rounding) is
    within one output rounding of the float64 closed form, with biases that
    differ per column (a bias indexed by row, or gate / up biases swapped,
    fails the same bound)."""
    g = torch.Generator().manual_seed(5)
    rows, hidden = 6, 96
    gate = (torch.randn(rows, hidden, generator=g) * 3).to(tdt)
    up = torch.randn(rows, hidden, generator=g).to(tdt)
    bg = torch.linspace(-2, 2, hidden).to(tdt)
    bu = (torch.randn(hidden, generator=g) * 0.5).to(tdt)
    ref = fallback.swiglu_with_bias_ref(gate, up, bg, bu)
    assert ref.dtype == tdt
    exact = fallback.swiglu_with_bias_f64(gate.float().numpy(), up.float().numpy(), bg.float().numpy(),
                                          bu.float().numpy())
    ulp = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -23}[tdt]
    tol = lambda e: np.abs(e) * ulp * 1.01 + 1e-30 + 8 * np.abs(e) * 2.0 ** -24   # one rounding + fp32 noise
    assert (np.abs(ref.double().numpy() - exact) <= tol(exact)).all()
    swapped = fallback.swiglu_with_bias_ref(gate, up, bu, bg).double().numpy()
    assert not (np.abs(swapped - exact) <= tol(exact)).all()
    by_row = fallback.swiglu_with_bias_ref(gate, up, bg.flip(0), bu).double().numpy()
    assert not (np.abs(by_row - exact) <= tol(exact)).all()


@pytest.mark.parametrize("tdt,dt", [(torch.float32, "f32"), (torch.float16, "f16"), (torch.bfloat16, "bf16")])
def test_nan_rows_follow_torch(tdt, dt):
    """Rows holding NaN: torch's amax propagates it (NaN scale) and the NaN
    quotients convert to 0 on the CPU; the numpy restatements of the weight
    quantiser, the KV codec and the W8A8 activation quantiser do the same."""
    from rotalabs_accel.quantization.symmetric import quantize_weight_per_channel
    g = torch.Generator().manual_seed(8)
    w = torch.randn(4, 64, generator=g).to(tdt)
    w[1, 7] = float("nan")
    q_t, s_t = quantize_weight_per_channel(w)
    q_o, s_o = oq.quantize_weight_per_channel(w.float().numpy(), dt)
    assert np.array_equal(q_t.numpy(), q_o) and (q_o[1] == 0).all()
    assert np.array_equal(s_t.numpy(), s_o, equal_nan=True) and np.isnan(s_o[1])
    for bits in (8, 4):
        qt, st = fallback.quantized_tensor_ref(w, bits)
        qn, sn = oq.quantized_tensor_rows(w.float().numpy(), dt, bits)
        assert np.array_equal(qt.numpy(), qn) and (qn[1] == 0).all()
        assert np.array_equal(st.float().numpy(), sn, equal_nan=True) and np.isnan(sn[1]).all()


def test_codec_division_correction_exhaustive(tmp_path):
    """The KV codec kernel replaces its per-element division by
    x * RN(1/s) plus one residual FMA; tests/division_check.c verifies, for
    every 16-bit x and scale in the codec's range (both formats), that this
    rounds to the same 16-bit value as the true quotient, and that amax / 127
    and amax / 7 come out bit-exact (compiled with gcc, all host threads)."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = os.path.join(os.path.dirname(os.path.abspath(__file__)), "division_check.c")
    exe = str(tmp_path / "division_check")
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", src, "-o", exe, "-lm"], check=True)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    assert " 0 mismatches" in res.stdout
