"""The product's Python API on CPU tensors: same names, results and errors as
the reference (its own tests, tests/test_imports.py:116-233, plus bit-level
checks against the oracle and the golden vectors)."""
import hashlib
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import rotalabs_accel as ra
from oracle import fallback
from oracle import quant as oq
from workloads import PLUMBING_SHAPE, gemm_case


def _t16(bits, dt):
    return torch.from_numpy(bits.astype(np.int16)).view(dt)


# ---- the reference's own unit tests, on this package -----------------------
def test_int8_gemm_torch_shape():
    x = torch.randn(2, 8, 64)
    w = torch.randint(-128, 127, (128, 64), dtype=torch.int8)
    out = ra.int8_gemm_torch(x, w, torch.ones(128))
    assert out.shape == (2, 8, 128) and not torch.isnan(out).any()


def test_quantize_dequantize_roundtrip():
    x = torch.randn(64, 128)
    q, s = ra.quantize_symmetric(x)
    assert q.dtype == torch.int8
    r = ra.dequantize(q, s)
    assert r.shape == x.shape and (x - r).abs().mean() < 0.1


def test_per_channel_shapes():
    w = torch.randn(64, 128)
    q, s = ra.quantize_weight_per_channel(w)
    assert q.dtype == torch.int8 and q.shape == w.shape and s.shape == (64,)


def test_quantization_error_keys():
    x = torch.randn(64, 128)
    q, s = ra.quantize_symmetric(x)
    e = ra.calculate_quantization_error(x, q, s)
    assert set(e) == {"max_abs_error", "mean_abs_error", "relative_error_pct", "snr_db"}
    assert e["max_abs_error"] >= 0


@pytest.mark.parametrize("cls", [ra.Int8Linear, ra.QuantizedLinear])
def test_linear_modules(cls):
    lin = cls(in_features=64, out_features=128)
    lin.quantize_weights(torch.randn(128, 64))
    out = lin(torch.randn(2, 8, 64))
    assert out.shape == (2, 8, 128) and not torch.isnan(out).any()


def test_rmsnorm_module():
    norm = ra.TritonRMSNorm(hidden_size=64, eps=1e-6)
    x = torch.randn(2, 8, 64)
    assert norm(x).shape == x.shape


# ---- bit-level agreement with the oracle / golden vectors --------------------
def test_rmsnorm_residual_cpu_path():
    """CPU tensors take rmsnorm_residual_torch (the reference's fallback):
    the oracle's bits, the reference's asserts, and the MLP composition with a
    residual stream equals the one on the rounded sum."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(3, 5, 64, generator=g).to(torch.bfloat16)
    r = torch.randn(3, 5, 64, generator=g).to(torch.bfloat16)
    w = (1 + 0.01 * torch.randn(64, generator=g)).to(torch.bfloat16)
    y = ra.rmsnorm_residual_fused(x, r, w)
    assert y.shape == x.shape and torch.equal(y, fallback.rmsnorm_residual_ref(x, r, w))
    assert torch.equal(ra.rmsnorm_residual_torch(x, r, w), y)
    with pytest.raises(AssertionError, match="Shape mismatch"):
        ra.rmsnorm_residual_fused(x, r[:, :4], w)
    with pytest.raises(AssertionError, match="Hidden dim mismatch"):
        ra.rmsnorm_residual_fused(x, r, w[:32])
    mlp = ra.Int8SwiGLUMLP(64, 96)
    mlp.quantize_weights(torch.randn(96, 64, generator=g) * 0.02, torch.randn(96, 64, generator=g) * 0.02,
                         torch.randn(64, 96, generator=g) * 0.02)
    assert torch.equal(mlp(x, r), mlp(x + r))


@pytest.mark.parametrize("bias", [False, True])
def test_swiglu_modules_cpu(bias):
    """SwiGLU keeps the reference module's structure; Int8SwiGLU.from_swiglu
    quantizes it and its CPU forward is the oracle's int8 FFN composition."""
    g = torch.Generator().manual_seed(13)
    torch.manual_seed(13)
    m = ra.SwiGLU(64, 96, bias=bias)
    assert [n for n, _ in m.named_parameters()] == (
        ["w_gate.weight", "w_gate.bias", "w_up.weight", "w_up.bias", "w_down.weight", "w_down.bias"] if bias
        else ["w_gate.weight", "w_up.weight", "w_down.weight"])
    x = torch.randn(3, 64, generator=g)
    ref = m.w_down(torch.nn.functional.silu(m.w_gate(x)) * m.w_up(x))
    assert torch.allclose(m(x), ref)
    q = ra.Int8SwiGLU.from_swiglu(m)
    xh = x.half()
    y = q(xh)
    want = fallback.swiglu_ffn_ref(xh, q.weight_gate_up, q.scale_gate_up, q.weight_down, q.scale_down,
                                   q.bias_gate_up, q.bias_down)
    assert y.dtype == torch.float16 and torch.equal(y, want)
    qg, _ = ra.quantize_weight_per_channel(m.w_gate.weight.data)
    assert torch.equal(q.weight_gate_up[:96], qg)
    with pytest.raises(RuntimeError, match="not quantized"):
        ra.Int8SwiGLU(64, 96)(xh)


def test_quantized_tensor_codec_cpu():
    """QuantizedTensor keeps the reference's attributes and runs its torch
    ops on CPU tensors (per-channel and per-tensor, 8 and 4 bits)."""
    from rotalabs_accel.speculative import QuantizedTensor
    g = torch.Generator().manual_seed(17)
    t = torch.randn(2, 4, 16, 64, generator=g).to(torch.bfloat16)
    for bits in (8, 4):
        for per_channel in (True, False):
            qt = QuantizedTensor(t, bits=bits, per_channel=per_channel)
            q, s = fallback.quantized_tensor_ref(t, bits, per_channel)
            assert torch.equal(qt.data, q)
            assert (torch.equal(qt.scale, s) if per_channel else qt.scale == s)
            assert qt.shape == t.shape and qt.dtype == t.dtype and qt.bits == bits
            assert torch.equal(qt.dequantize(), q.to(t.dtype) * s)
            n = t.numel() * (1 if bits == 8 else 0.5) + (qt.scale.numel() * 4 if per_channel else 4)
            assert qt.memory_bytes == int(n)
    with pytest.raises(ValueError, match="Unsupported bits"):
        QuantizedTensor(t, bits=2)


@pytest.mark.parametrize("cls_name", ["QuantizedLinear", "Int8Linear"])
def test_quantize_model(cls_name):
    """quantize_model replaces every nn.Linear (skip list honoured), the
    outputs follow the int8 modules, and the state_dict reloads."""
    from rotalabs_accel.quantization import quantize_model
    cls = getattr(ra, cls_name)
    torch.manual_seed(5)
    model = torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.ReLU(),
                                torch.nn.Sequential(torch.nn.Linear(128, 96, bias=False)),
                                torch.nn.Linear(96, 32))
    x = torch.randn(4, 64)
    ref = model(x)
    quantize_model(model, cls, skip=["3"])
    assert isinstance(model[0], cls) and isinstance(model[2][0], cls)
    assert type(model[3]) is torch.nn.Linear
    xin = x.half() if cls_name == "Int8Linear" else x
    if cls_name == "Int8Linear":   # fp16 activations and bias (as the reference module)
        model[3] = model[3].half()
    y = model(xin)
    assert torch.allclose(y.float(), ref, rtol=5e-2, atol=5e-2)
    sd = model.state_dict()
    assert "0.weight_int8" in sd and "2.0.weight_int8" in sd
    fresh = torch.nn.Sequential(cls(64, 128, bias=True), torch.nn.ReLU(),
                                torch.nn.Sequential(cls(128, 96)), model[3])
    fresh.load_state_dict(sd)
    for m in (fresh[0], fresh[2][0]):
        m._quantized = True
    assert torch.equal(fresh(xin), y)


def test_quantize_fp32_bit_exact():
    g = torch.Generator().manual_seed(11)
    w = torch.randn(96, 257, generator=g) * 0.02
    w[0] = 0
    w[1, :9] = torch.tensor([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -125.5])
    w[1, 9:] = 0
    q, s = ra.quantize_weight_per_channel(w)
    q_o, s_o = oq.quantize_weight_per_channel(w.numpy())
    assert np.array_equal(q.numpy(), q_o) and np.array_equal(s.numpy(), s_o)


@pytest.mark.parametrize("name,dt", [("f16", torch.float16), ("bf16", torch.bfloat16)])
def test_quantize_reduced_bit_exact(golden, name, dt):
    w = _t16(golden[f"qpc_{name}_w"], dt)
    q, s = ra.quantize_weight_per_channel(w)
    assert np.array_equal(q.numpy(), golden[f"qpc_{name}_q"])
    assert np.array_equal(s.numpy(), golden[f"qpc_{name}_s"])


@pytest.mark.parametrize("name,dt", [("f16", torch.float16), ("bf16", torch.bfloat16), ("f32", torch.float32)])
def test_int8_gemm_cpu_golden(golden, name, dt):
    x = torch.from_numpy(golden["gemm_x_f32"]).to(dt)
    q = torch.from_numpy(golden["gemm_q"])
    s = torch.from_numpy(golden["gemm_s"])
    b = torch.from_numpy(golden["gemm_b_f32"]).to(dt)
    y, yb = ra.int8_gemm(x, q, s), ra.int8_gemm(x, q, s, b)
    if dt == torch.float32:
        assert np.array_equal(y.numpy(), golden["gemm_y_f32"]) and np.array_equal(yb.numpy(), golden["gemm_yb_f32"])
    else:
        assert torch.equal(y, _t16(golden[f"gemm_y_{name}"], dt))
        assert torch.equal(yb, _t16(golden[f"gemm_yb_{name}"], dt))


def test_plumbing_workload_digest(golden_digests):
    """int8_gemm on CPU at x fp16 [16,4096], W [4096,4096], seed 0 reproduces
    the reference's output bit for bit (sha256)."""
    M, K, N, seed = PLUMBING_SHAPE
    c = gemm_case(M, K, N, seed)

    def sha(t):
        a = t.contiguous()
        if a.dtype in (torch.float16, torch.bfloat16):
            a = a.view(torch.int16)
        return hashlib.sha256(a.numpy().tobytes()).hexdigest()

    assert sha(c.x) == golden_digests["x_f16"]
    assert sha(c.q) == golden_digests["q"] and sha(c.s) == golden_digests["s"]
    y = ra.int8_gemm(c.x, c.q, c.s)
    assert y.dtype == torch.float16 and y.shape == (16, 4096)
    assert sha(y) == golden_digests["y_f16"]


def test_gateup_and_mlp_cpu_match_oracle():
    g = torch.Generator().manual_seed(3)
    H, inter, M = 64, 96, 5
    x = torch.randn(M, H, generator=g).bfloat16()
    nw = (1 + 0.01 * torch.randn(H, generator=g)).bfloat16()
    wg, wu, wd = (torch.randn(inter, H, generator=g) * 0.02, torch.randn(inter, H, generator=g) * 0.02,
                  torch.randn(H, inter, generator=g) * 0.02)
    mlp = ra.Int8SwiGLUMLP(H, inter, norm_dtype=torch.bfloat16)
    mlp.quantize_weights(wg, wu, wd)
    mlp.norm_weight.data.copy_(nw)
    y = mlp(x)
    ref = fallback.mlp_ref(x, nw, mlp.weight_gate_up, mlp.scale_gate_up, mlp.weight_down, mlp.scale_down)
    assert torch.equal(y, ref)
    # concatenated quantization == separate quantization (row independence)
    q_all, s_all = ra.quantize_weight_per_channel(torch.cat([wg, wu]))
    assert torch.equal(q_all, mlp.weight_gate_up) and torch.equal(s_all, mlp.scale_gate_up)


# ---- error behaviour ---------------------------------------------------------
def test_int8_gemm_asserts():
    x = torch.randn(4, 64)
    with pytest.raises(AssertionError, match="Weight must be INT8"):
        ra.int8_gemm(x, torch.zeros(8, 64), torch.ones(8))
    with pytest.raises(AssertionError, match="Weight shape mismatch"):
        ra.int8_gemm(x, torch.zeros(8, 32, dtype=torch.int8), torch.ones(8))
    with pytest.raises(AssertionError, match="Scale shape mismatch"):
        ra.int8_gemm(x, torch.zeros(8, 64, dtype=torch.int8), torch.ones(7))


def test_bias_dtype_mismatch_raises_on_cpu():
    x = torch.randn(2, 64).half()
    w = torch.zeros(8, 64, dtype=torch.int8)
    with pytest.raises(RuntimeError):
        ra.int8_gemm(x, w, torch.ones(8), torch.zeros(8))


def test_reexported_names():
    """The import paths of the reference's re-export lists for this path
    (src/rotalabs_accel/__init__.py:34-70, kernels/__init__.py:38-42,
    modules/__init__.py:7-11, quantization/__init__.py:6-12)."""
    import rotalabs_accel.kernels as K
    import rotalabs_accel.modules as Mo
    import rotalabs_accel.quantization as Q
    for name in ("rmsnorm", "rmsnorm_torch", "TritonRMSNorm", "swiglu_fused", "swiglu_torch", "SwiGLU",
                 "int8_gemm", "int8_gemm_torch", "Int8Linear", "quantize_symmetric", "dequantize",
                 "quantize_weight_per_channel", "calculate_quantization_error", "QuantizedLinear"):
        assert hasattr(ra, name), name
    for name in ("rmsnorm", "rmsnorm_torch", "rmsnorm_residual_fused", "TritonRMSNorm", "swiglu_fused",
                 "swiglu_torch", "SwiGLU", "int8_gemm", "int8_gemm_torch", "Int8Linear", "HAS_TRITON"):
        assert hasattr(K, name), name
    for name in ("TritonRMSNorm", "SwiGLU", "Int8Linear", "QuantizedLinear"):
        assert hasattr(Mo, name) and name in Mo.__all__, name
    assert Mo.SwiGLU is ra.SwiGLU
    for name in ("quantize_symmetric", "dequantize", "quantize_weight_per_channel",
                 "calculate_quantization_error", "QuantizedLinear"):
        assert hasattr(Q, name), name


def test_quantized_linear_bias_dtype_error():
    """QuantizedLinear keeps the reference's fp32 bias; with fp16/bf16
    activations the reference's F.linear rejects it (symmetric.py:288-291).
    The same RuntimeError on every device; fp32 activations work."""
    lin = torch.nn.Linear(32, 16, bias=True)
    m = ra.QuantizedLinear.from_linear(lin)
    for dt in (torch.float16, torch.bfloat16):
        x = torch.randn(3, 32).to(dt)
        w = ra.dequantize(m.weight_int8, m.weight_scale, dtype=dt, dim=0)
        with pytest.raises(RuntimeError) as ref_err:
            torch.nn.functional.linear(x, w, m.bias)
        with pytest.raises(RuntimeError) as err:
            m(x)
        assert str(err.value) == str(ref_err.value)
    y = m(torch.randn(3, 32))
    assert y.dtype == torch.float32 and y.shape == (3, 16)


def test_split_bias_shapes():
    """Bias shapes the reference's broadcast add accepts (gemm.py:181-182):
    (N,) and N values along the last dim go to the kernels, one value is
    expanded, other broadcastable shapes are added after the GEMM."""
    from rotalabs_accel.kernels.gemm import _split_bias
    N = 8
    for b in (torch.randn(N), torch.randn(1, N), torch.randn(N).half()):
        kb, post = _split_bias(b, N)
        assert post is None and kb.shape == (N,) and torch.equal(kb, b.reshape(N))
    for b in (torch.tensor(2.0), torch.tensor([2.0])):
        kb, post = _split_bias(b, N)
        assert post is None and kb.shape == (N,) and (kb == 2.0).all()
    for b in (torch.randn(3, N), torch.randn(3, 1), torch.randn(N).double()):
        kb, post = _split_bias(b, N)
        assert kb is None and post is b
    assert _split_bias(None, N) == (None, None)


@pytest.mark.parametrize("cls", [ra.Int8Linear, ra.QuantizedLinear])
def test_unquantized_forward_raises(cls):
    with pytest.raises(RuntimeError, match="Weights not quantized"):
        cls(16, 8)(torch.randn(2, 16))


def test_state_dict_keys_and_reload():
    lin = ra.Int8Linear(32, 16, bias=True)
    lin.quantize_weights(torch.randn(16, 32))
    sd = lin.state_dict()
    assert set(sd) == {"weight_int8", "scale", "weight_transposed", "bias"}
    assert sd["bias"].dtype == torch.float16 and sd["weight_transposed"].shape == (32, 16)
    assert torch.equal(sd["weight_transposed"], sd["weight_int8"].t())
    fresh = ra.Int8Linear(32, 16, bias=True)
    fresh.load_state_dict(sd)
    with pytest.raises(RuntimeError):          # _quantized is not part of the state
        fresh(torch.randn(2, 32))
    ql = ra.QuantizedLinear(32, 16, bias=True)
    assert set(ql.state_dict()) == {"weight_int8", "weight_scale", "bias"}


def test_from_linear():
    lin = torch.nn.Linear(32, 16, bias=True)
    a = ra.Int8Linear.from_linear(lin)
    q, s = ra.quantize_weight_per_channel(lin.weight.data)
    assert torch.equal(a.weight_int8, q) and torch.equal(a.scale, s) and a.bias.dtype == torch.float16
    b = ra.QuantizedLinear.from_linear(lin)
    assert torch.equal(b.weight_int8, q) and b.bias.dtype == torch.float32


def test_rows_helper_layouts():
    from rotalabs_accel.kernels.gemm import _rows
    t = torch.randn(6, 40).half()
    v, ld = _rows(t, 16)
    assert v.data_ptr() == t.data_ptr() and ld == 40
    sl = torch.randn(6, 48).half()[:, :40]           # row stride 48 (96 B: 16-aligned)
    v, ld = _rows(sl, 16)
    assert v.data_ptr() == sl.data_ptr() and ld == 48
    tt = torch.randn(40, 6).half().t()               # column-major -> copy
    v, ld = _rows(tt, 16)
    assert ld == 40 and v.is_contiguous() and torch.equal(v, tt)
    odd = torch.randn(1, 40).half().expand(3, 40)    # row stride 0 -> copy
    v, ld = _rows(odd, 16)
    assert ld == 40 and torch.equal(v, odd)


def test_missing_library_fails_loudly(tmp_path):
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from rotalabs_accel import _backend\n"
            "try:\n    _backend.load()\nexcept RuntimeError as e:\n    print('RAISED', e)\n") % (
        os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "rotalabs-accel_amd"))
    env = dict(os.environ, ROTACCEL_LIB=str(tmp_path / "nope.so"))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert "RAISED" in out.stdout and "Build it" in out.stdout


@pytest.mark.parametrize("tdt,dt", [(torch.float16, "f16"), (torch.bfloat16, "bf16")])
def test_w8a8_route_cpu_matches_oracle(tdt, dt):
    """quantized_matmul.int8_gemm(use_cublas=True) on CPU tensors: activation
    quantisation and the scaled int8 GEMM equal the numpy restatement bit for
    bit; M <= 16 and use_cublas=None take the W8A16 route (reference dispatch
    quantized_matmul.py:436-447)."""
    from rotalabs_accel.kernels import quantized_matmul as qm
    g = torch.Generator().manual_seed(11)
    M, K, N = 40, 256, 96
    x = torch.randn(2, M // 2, K, generator=g).to(tdt)
    q, s = ra.quantize_weight_per_channel(torch.randn(N, K, generator=g))
    b = torch.randn(N, generator=g).to(tdt)   # the CPU fallback's F.linear needs bias in x's dtype
    y = qm.int8_gemm(x, q, s, b, use_cublas=True)
    assert y.shape == (2, M // 2, N) and y.dtype == tdt
    xq, xs = oq.quantize_activations_rows(x.reshape(-1, K).float().numpy(), dt)
    ref = oq.w8a8_gemm_rows(xq, xs, q.numpy(), s.numpy(), dt, b.float().numpy())
    np.testing.assert_array_equal(y.reshape(-1, N).float().numpy(), ref)
    # the W8A8 error stays near the W8A16 result (activation quantisation)
    y16 = qm.int8_gemm(x, q, s, b)
    torch.testing.assert_close(y16, ra.int8_gemm(x, q, s, b), rtol=0, atol=0)
    rel = (y.float() - y16.float()).norm() / y16.float().norm()
    assert rel < 0.05
    small = qm.int8_gemm(x[:, :8], q, s, b, use_cublas=True)
    torch.testing.assert_close(small, ra.int8_gemm(x[:, :8], q, s, b), rtol=0, atol=0)
    # act_scale other than 127: the reference's expression with that constant
    for c in (100.0, 63.5):
        xq_c, xs_c = qm.quantize_activations(x, act_scale=c)
        q_o, xs_o = oq.quantize_activations_rows(x.reshape(-1, K).float().numpy(), dt, act_scale=c)
        np.testing.assert_array_equal(xq_c.numpy(), q_o)
        np.testing.assert_array_equal(xs_c.float().numpy(), xs_o)


def test_swiglu_module_and_bias_cpu():
    """kernels.swiglu (swiglu.py:79-260): the activation-only SwiGLU module and
    swiglu_with_bias on CPU tensors equal the oracle; the reference's asserts."""
    from rotalabs_accel.kernels import swiglu as sw
    g = torch.Generator().manual_seed(2)
    gate = torch.randn(2, 3, 64, generator=g).half()
    up = torch.randn(2, 3, 64, generator=g).half()
    assert torch.equal(sw.SwiGLU()(gate, up), fallback.swiglu_ref(gate, up))
    bg = torch.randn(64, generator=g).half()
    bu = torch.randn(64, generator=g).float()
    y = sw.swiglu_with_bias(gate, up, bg, bu)
    assert y.dtype == torch.float16 and y.shape == gate.shape
    assert torch.equal(y, fallback.swiglu_with_bias_ref(gate, up, bg, bu))
    with pytest.raises(AssertionError):
        sw.swiglu_with_bias(gate, up[..., :32], bg, bu)
    with pytest.raises(AssertionError):
        sw.swiglu_with_bias(gate, up, bg[:32], bu)


def test_plumbing_fixture_is_the_reference_output(golden_digests):
    """tests/golden/plumbing_y_f16.npy (written by make_plumbing.py) carries
    the reference's config-1 output: its sha256 is the reference's digest."""
    bits = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "plumbing_y_f16.npy"))
    assert bits.dtype == np.int16 and bits.shape == (16, 4096)
    assert hashlib.sha256(bits.tobytes()).hexdigest() == golden_digests["y_f16"]
    assert np.array_equal(bits[0, :8].view(np.float16).astype(np.float64), golden_digests["y_first8"])
