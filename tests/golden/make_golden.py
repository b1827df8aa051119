"""Write golden vectors for the W8A16 path from the reference implementation.

Run in the build container only (the reference tree does not exist on GPU
machines):   python tests/golden/make_golden.py

It imports the reference's Python package from /root/reference/src on the CPU
and records inputs and outputs of the functions whose exact bits the closed
forms in oracle/ cannot fix on their own:

  * quantize_weight_per_channel / quantize_symmetric on fp16 and bf16 input
    (intermediate roundings inside PyTorch's reduced-precision CPU kernels),
  * int8_gemm_torch output bits (CPU BLAS dispatch), incl. the reference
    test's own case (tests/test_imports.py:116-127),
  * calculate_quantization_error float outputs,
  * rmsnorm_torch / swiglu_torch (reduction order, transcendental rounding),
  * a sha256 of int8_gemm_torch's output on the CPU plumbing workload
    (x fp16 [16,4096] ~N(0,1), W fp32 [4096,4096] ~N(0,0.02), seed 0).

fp32 per-channel quantization and dequantize are pinned by closed forms and
are deliberately NOT taken from the reference.

Outputs: tests/golden/golden_small.npz and tests/golden/golden_digests.json.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, "/root/reference/src")
sys.path.insert(1, REPO)

from rotalabs_accel.kernels.gemm import int8_gemm_torch  # noqa: E402  (reference)
from rotalabs_accel.kernels.normalization import rmsnorm_torch  # noqa: E402
from rotalabs_accel.kernels.activations import swiglu_torch  # noqa: E402
from rotalabs_accel.quantization.symmetric import (  # noqa: E402
    quantize_symmetric,
    quantize_weight_per_channel,
    calculate_quantization_error,
)

assert "/root/reference/src" in os.path.abspath(sys.modules["rotalabs_accel"].__file__)

from oracle import quant as oq  # noqa: E402  (closed-form fp32 quantizer)


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit patterns of a tensor (bf16/fp16 -> uint16, others as-is)."""
    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def edge_weight(rows: int, cols: int, g: torch.Generator) -> torch.Tensor:
    w = torch.randn(rows, cols, generator=g) * 0.02
    w[0] = 0.0                                    # all-zero row -> scale 1, q 0
    w[1] = 0.0
    w[1, 5] = -0.75                               # single negative maximum
    w[2] = torch.linspace(-1.0, 1.0, cols)        # exact +-max at both ends
    # round-half-even ties: max 127 -> s = 1, entries k + 0.5
    w[3] = 0.0
    w[3, 0] = 127.0
    w[3, 1:9] = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127.5])
    w[4] = w[4] * 1e-6                            # tiny row (fp16 subnormals)
    return w


def main() -> None:
    g = torch.Generator().manual_seed(1234)
    out: dict[str, np.ndarray] = {}

    # ---- per-channel quantization on reduced-precision input -------------
    w32 = edge_weight(64, 128, g)
    for name, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        w = w32.to(dt)
        q, s = quantize_weight_per_channel(w)
        out[f"qpc_{name}_w"] = bits(w)
        out[f"qpc_{name}_q"] = q.numpy()
        out[f"qpc_{name}_s"] = s.numpy()
        qt, st = quantize_symmetric(w)            # per-tensor branch (:60-63)
        out[f"qpt_{name}_q"] = qt.numpy()
        out[f"qpt_{name}_s"] = st.reshape(1).numpy()

    # ---- int8_gemm_torch output bits -------------------------------------
    M, K, N = 16, 256, 128
    x32 = torch.randn(M, K, generator=g)
    wq32 = torch.randn(N, K, generator=g) * 0.02
    q_np, s_np = oq.quantize_weight_per_channel(wq32.numpy())
    q, s = torch.from_numpy(q_np), torch.from_numpy(s_np)
    b32 = torch.randn(N, generator=g) * 0.1
    out["gemm_x_f32"] = x32.numpy()
    out["gemm_q"] = q_np
    out["gemm_s"] = s_np
    out["gemm_b_f32"] = b32.numpy()
    for name, dt in (("f16", torch.float16), ("bf16", torch.bfloat16), ("f32", torch.float32)):
        x = x32.to(dt)
        out[f"gemm_y_{name}"] = bits(int8_gemm_torch(x, q, s))
        out[f"gemm_yb_{name}"] = bits(int8_gemm_torch(x, q, s, b32.to(dt)))

    # the reference's own unit-test case (test_imports.py:116-127)
    xt = torch.randn(2, 8, 64, generator=g)
    wt = torch.randint(-128, 127, (128, 64), dtype=torch.int8, generator=g)
    st = torch.ones(128)
    out["reftest_x"] = xt.numpy()
    out["reftest_w"] = wt.numpy()
    out["reftest_y"] = int8_gemm_torch(xt, wt, st).numpy()

    # ---- calculate_quantization_error ------------------------------------
    xe = torch.randn(64, 128, generator=g)
    qe, se = quantize_symmetric(xe)               # per-tensor, fp32: closed form
    err = calculate_quantization_error(xe, qe, se)
    out["qerr_x"] = xe.numpy()
    out["qerr_vals"] = np.array([err["max_abs_error"], err["mean_abs_error"],
                                 err["relative_error_pct"], err["snr_db"]], dtype=np.float64)
    qe2, se2 = quantize_weight_per_channel(xe)
    err2 = calculate_quantization_error(xe, qe2, se2, dim=0)
    out["qerr_pc_vals"] = np.array([err2["max_abs_error"], err2["mean_abs_error"],
                                    err2["relative_error_pct"], err2["snr_db"]], dtype=np.float64)

    # ---- rmsnorm_torch / swiglu_torch ------------------------------------
    xr = (torch.randn(17, 256, generator=g) * 2.0).to(torch.bfloat16)
    wr = (1.0 + 0.01 * torch.randn(256, generator=g)).to(torch.bfloat16)
    out["rms_x_bf16"] = bits(xr)
    out["rms_w_bf16"] = bits(wr)
    out["rms_y_bf16"] = bits(rmsnorm_torch(xr, wr, 1e-6))
    xh = torch.randn(5, 384, generator=g).to(torch.float16)
    wf = 1.0 + 0.01 * torch.randn(384, generator=g)
    out["rms_x_f16"] = bits(xh)
    out["rms_w_f32"] = wf.numpy()
    out["rms_y_f16w32"] = bits(rmsnorm_torch(xh, wf, 1e-6))   # promotes to fp32
    gt = (torch.randn(17, 256, generator=g) * 3.0).to(torch.bfloat16)
    ut = torch.randn(17, 256, generator=g).to(torch.bfloat16)
    out["swiglu_g_bf16"] = bits(gt)
    out["swiglu_u_bf16"] = bits(ut)
    out["swiglu_y_bf16"] = bits(swiglu_torch(gt, ut))

    np.savez_compressed(os.path.join(HERE, "golden_small.npz"), **out)

    # ---- CPU plumbing workload digest ------------------------------------
    g0 = torch.Generator().manual_seed(0)
    x = torch.randn(16, 4096, generator=g0).to(torch.float16)
    w = torch.randn(4096, 4096, generator=g0) * 0.02
    q_np, s_np = oq.quantize_weight_per_channel(w.numpy())
    y = int8_gemm_torch(x, torch.from_numpy(q_np), torch.from_numpy(s_np))

    def sha(a: np.ndarray) -> str:
        return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()

    digests = {
        "workload": "x fp16 [16,4096] ~N(0,1); W fp32 [4096,4096] ~N(0,0.02); seed 0; x drawn first",
        "torch": torch.__version__,
        "x_f16": sha(bits(x)),
        "q": sha(q_np),
        "s": sha(s_np),
        "y_f16": sha(bits(y)),
        "y_first8": [float(v) for v in y[0, :8].float()],
    }
    with open(os.path.join(HERE, "golden_digests.json"), "w") as f:
        json.dump(digests, f, indent=1)
    print("wrote", len(out), "arrays and digests")


if __name__ == "__main__":
    main()
