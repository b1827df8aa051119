"""ra_w8a16_gemm_noalloc, the entry point that allocates nothing (its split-K
workspace is the library's fixed device array), through the C ABI: equal
bit for bit to ra_w8a16_gemm_ws with a caller workspace, on two calls in a
row, the second on a smaller problem, then a call whose tiled kernel splits
K over workgroups (the same array holds its partial sums); a problem needing
more than the array is refused (tests/test_abi.py)."""
import pytest
import torch

from rotalabs_accel import _backend
from workloads import gemm_case

pytestmark = pytest.mark.gpu


def _args(c, y):
    M, K = c.x.shape
    N = c.q.shape[0]
    return (c.x.data_ptr(), K, _backend.dtype_code(c.x.dtype), c.q.data_ptr(), K, c.s.data_ptr(), None, 0,
            y.data_ptr(), N, M, N, K)


def test_noalloc_matches_workspace_entry_point(gpu):
    lib = _backend.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    # (M, K, N, seed): the MLP's down projection at M=17, then a smaller split-K
    # problem, split K with three 16-row tiles, then the 64-row tiles with K
    # split over four workgroups, in one row and in two
    for (M, K, N, seed) in [(17, 28672, 8192, 1), (5, 16384, 1000, 2), (40, 8192, 6000, 5), (64, 8192, 11008, 3),
                            (128, 11008, 4096, 4)]:
        print(f"  noalloc M={M} K={K} N={N}", flush=True)
        c = gemm_case(M, K, N, seed, device=gpu, dtype=torch.bfloat16, outlier_rows=True)
        xdt = _backend.dtype_code(c.x.dtype)
        assert lib.ra_w8a16_gemm_select(M, N, K, xdt) == (_backend.VARIANT_TILED if M >= 64 else
                                                          _backend.VARIANT_SPLITK)
        need = lib.ra_w8a16_gemm_workspace_size(M, N, K, xdt)
        assert 0 < need <= 16 << 20
        ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
        y_ws = torch.full((M, N), float("nan"), dtype=c.x.dtype, device=gpu)
        _backend.check(lib.ra_w8a16_gemm_ws(*_args(c, y_ws), ws.data_ptr(), need, stream))
        y_na = torch.full((M, N), float("nan"), dtype=c.x.dtype, device=gpu)
        _backend.check(lib.ra_w8a16_gemm_noalloc(*_args(c, y_na), stream))
        torch.cuda.synchronize()
        assert not torch.isnan(y_ws).any()
        assert torch.equal(y_na, y_ws)
        # the workspace entry point left its counters at zero
        assert not ws[:16384].any()
