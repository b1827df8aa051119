"""Write tests/golden/plumbing_y_f16.npy: the output of the config-1 plumbing
workload (x fp16 [16,4096] ~N(0,1), W fp32 [4096,4096] ~N(0,0.02) quantized
per channel, seed 0) through the CPU path, int8_gemm_torch (the reference's
fallback, src/rotalabs_accel/kernels/gemm.py:31-48), as raw fp16 bits.

Runs this package's CPU path, whose output is checked bit for bit against the
sha256 digest of the reference's own output in golden_digests.json before it
is written, so the stored array is the reference's output. Other hosts' CPU
BLAS may round the fp16 GEMM differently; tests compare against this array.

    python tests/golden/make_plumbing.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "rotalabs-accel_amd"))

import torch  # noqa: E402

import rotalabs_accel as ra  # noqa: E402
from workloads import PLUMBING_SHAPE, gemm_case  # noqa: E402


def main():
    M, K, N, seed = PLUMBING_SHAPE
    c = gemm_case(M, K, N, seed)
    y = ra.int8_gemm(c.x, c.q, c.s)
    bits = y.contiguous().view(torch.int16).numpy()
    digests = json.load(open(os.path.join(HERE, "golden_digests.json")))
    got = hashlib.sha256(bits.tobytes()).hexdigest()
    if got != digests["y_f16"]:
        raise SystemExit(f"this host's CPU path does not reproduce the reference digest ({got}); not writing")
    np.save(os.path.join(HERE, "plumbing_y_f16.npy"), bits)
    print("wrote plumbing_y_f16.npy", bits.shape)


if __name__ == "__main__":
    main()
