"""CPU oracle for the W8A16 INT8 GEMM path.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU, the algorithm of
the reference's W8A16 path so that the HIP kernels can be checked against it.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker (or, for ``bench.py``, as
the timed CPU baseline) -- never as the thing measured or shipped. The product
(``rotalabs-accel_amd/rotalabs_accel``) must not import anything from here.

Modules
-------
``quant``     numpy closed forms of ``quantize_symmetric`` /
              ``quantize_weight_per_channel`` / ``dequantize`` /
              ``calculate_quantization_error`` for fp32, fp16 and bf16 inputs
              (src/rotalabs_accel/quantization/symmetric.py:24-207).
``fallback``  torch-CPU restatement of ``int8_gemm_torch``
              (src/rotalabs_accel/kernels/gemm.py:31-48), ``rmsnorm_torch``
              (kernels/normalization.py:32-45), ``swiglu_torch``
              (kernels/activations.py:36-45) and the RMSNorm -> gate/up ->
              SwiGLU -> down composition, plus a float64 numpy reference.
``cquant``    ctypes wrapper of ``quant_ref.c``: an independent plain-C
              restatement of per-channel fp32 quantization, used to
              cross-check ``quant``.

How each function is pinned (what a plausible mistake would fail):

* fp32 quantization: two independent restatements (numpy, C) must agree
  bit-for-bit; invariants (|q| <= 127, q = +-127 at each row's argmax,
  zero row -> s = 1 / q = 0, s == fl32(max/127)); round-half-even tie rows;
  row independence; brute force on tiny inputs.
* fp16 / bf16 quantization, ``int8_gemm_torch`` outputs,
  ``calculate_quantization_error``, ``rmsnorm_torch``, ``swiglu_torch``:
  golden vectors written by ``tests/golden/make_golden.py`` from the
  reference itself, plus closed forms.
* ``dequantize``: closed form (int -> fp32 exact, one fp32 product, one
  rounding to the target dtype) and the golden vectors.
* GEMM tolerance: exact known-answer tests (integer x, power-of-two scales,
  |y| <= 2048 so every partial sum and the output are exact).
"""
