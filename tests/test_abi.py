"""The C ABI library loads and exports every symbol include/rotaccel.h
declares; host-side argument checks return the documented codes without any
device work (no GPU needed)."""
import ctypes
import os
import re

import pytest

from rotalabs_accel import _backend

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "rotaccel.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ra_\w+)\s*\(", src, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _backend.load()
    names = _declared()
    assert "ra_w8a16_gemm" in names and len(names) >= 8
    for n in names:
        assert hasattr(lib, n), n


def test_abi_version_matches_header():
    ver = int(re.search(r"#define RA_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert _backend.load().ra_abi_version() == ver == _backend.ABI_VERSION


def test_strerror_all_codes():
    lib = _backend.load()
    for code in range(0, 8):
        assert lib.ra_strerror(code)


def test_argument_checks_without_device_work():
    lib = _backend.load()
    n = None
    # negative / oversized sizes
    assert lib.ra_w8a16_gemm(n, 0, 0, n, 0, n, n, 0, n, 0, -1, 4, 4, n) == 1
    # unsupported activation dtype
    assert lib.ra_w8a16_gemm(n, 0, 7, n, 0, n, n, 0, n, 0, 1, 4, 4, n) == 2
    # empty problems are no-ops
    assert lib.ra_w8a16_gemm(n, 0, 0, n, 0, n, n, 0, n, 0, 0, 4, 4, n) == 0
    assert lib.ra_w8a16_gemm(n, 0, 0, n, 0, n, n, 0, n, 0, 4, 0, 4, n) == 0
    # null pointers / leading dimensions
    assert lib.ra_w8a16_gemm(n, 4, 0, n, 4, n, n, 0, n, 4, 2, 4, 4, n) == 1
    assert lib.ra_rmsnorm(n, 0, 1, n, 1, n, 0, 0, 1, 8, 1e-6, n) == 2   # y dtype != promotion
    assert lib.ra_swiglu(n, n, n, -1, 0, n) == 1
    assert lib.ra_quantize_per_channel(n, 0, 9, 1, 1, n, 0, n, n) == 2
    assert lib.ra_w8a16_gateup_swiglu(n, 0, 0, n, 0, n, n, 0, 0, 8, 8, n) == 0
    # unknown forced variant
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    assert lib.ra_w8a16_gemm_ex(p, 16, 0, p, 16, p, n, 0, p, 16, 1, 16, 16, 99, n, 0, n) == 1
    # a workspace smaller than the problem needs (the split-K plan of M=17 K=28672 N=8192): refused
    # before any launch
    need = lib.ra_w8a16_gemm_workspace_size(17, 8192, 28672, 0)
    assert need > 0
    wsa = (p + 255) // 256 * 256   # workspaces start on a 256-byte boundary
    assert lib.ra_w8a16_gemm_ws(p, 28672, 0, p, 28672, p, n, 0, p, 8192, 17, 8192, 28672, wsa, need - 1, n) == 6
    assert lib.ra_w8a16_gemm_workspace_size(1, 11008, 4096, 0) == 0      # row GEMV: none
    assert lib.ra_w8a16_gemm_workspace_size(2048, 11008, 4096, 0) == 0   # tiled: none
    assert lib.ra_w8a16_gateup_swiglu_ws(n, 0, 0, n, 0, n, n, 0, 0, 8, 8, n, 0, n) == 0
    # split-K plans keep their partial sums within the no-allocation entry point's 16 MiB
    # array: the widest problems split less (or not at all) instead of being refused there
    # (at M <= 32 the reported size is the split-K plan's; from M = 33 it also covers the
    # 64-row tiles' split plan, which runs unsplit when the array is too small)
    for (M, N, K) in [(32, 57344, 16384), (17, 57344, 32768), (32, 32768, 28672), (8, 65536, 16384),
                      (16, 128256, 16384), (5, 1000, 16384), (24, 28672, 28672)]:
        assert lib.ra_w8a16_gemm_select(M, N, K, 0) == 7
        assert 0 <= lib.ra_w8a16_gemm_workspace_size(M, N, K, 0) <= 16 << 20
    for (M, I, K) in [(64, 28672, 16384), (32, 57344, 28672), (17, 6656, 16384)]:
        assert lib.ra_w8a16_gateup_workspace_size(M, I, K, 0) <= 16 << 20
    assert lib.ra_w8a16_gemm_noalloc(n, 0, 0, n, 0, n, n, 0, n, 0, -1, 4, 4, n) == 1
    assert lib.ra_w8a16_gemm_noalloc(n, 0, 0, n, 0, n, n, 0, n, 0, 0, 4, 4, n) == 0


@pytest.mark.parametrize("M,expect", [(1, 5), (2, 6), (3, 6), (4, 6), (5, 6), (16, 6), (32, 6), (33, 7), (48, 7), (49, 2), (64, 2), (65, 2),
                                      (2048, 2)])
def test_variant_selection(M, expect):
    assert _backend.load().ra_w8a16_gemm_select(M, 11008, 4096, 0) == expect


def test_variant_selection_fallbacks():
    lib = _backend.load()
    assert lib.ra_w8a16_gemm_select(1, 8192, 28672, 1) == 5  # row GEMV: any K
    assert lib.ra_w8a16_gemm_select(3, 8192, 8192, 1) == 6   # M = 3..64, K % 128 == 0: small-batch kernel
    assert lib.ra_w8a16_gemm_select(17, 8192, 28672, 1) == 7  # ... with K >= 16384: split K over workgroups
    assert lib.ra_w8a16_gemm_select(16, 4096, 11008, 1) == 7  # ... from 16 rows, K >= 11008 over N <= 4096
    assert lib.ra_w8a16_gemm_select(15, 4096, 11008, 1) == 7  # ... at any M from K = 11008
    assert lib.ra_w8a16_gemm_select(16, 8192, 8192, 1) == 7   # ... from 16 rows at K = 8192
    assert lib.ra_w8a16_gemm_select(15, 8192, 8192, 1) == 6   # below that the small-batch kernel
    assert lib.ra_w8a16_gemm_select(64, 8192, 28672, 1) == 2  # M = 33..64, N >= 8192: 64-row tiles
    assert lib.ra_w8a16_gemm_select(4, 8192, 1040, 1) == 1   # K % 128 != 0: split-K MFMA kernel
    assert lib.ra_w8a16_gemm_select(1, 64, 50, 0) == 3     # K % 16 != 0 -> generic
    assert lib.ra_w8a16_gemm_select(1, 64, 64, 2) == 3     # fp32 activations -> generic
    assert lib.ra_w8a16_gemm_select(4, 64, 0, 0) == 3      # K == 0 -> generic (bias / zeros)


@pytest.mark.parametrize("M,N,K,expect", [
    # M = 1, K <= 2048 over 4096+ rows: the small-batch kernel (skinny at K <= 1536 over 16384+ rows)
    (1, 16384, 2048, 6), (1, 4096, 512, 6), (1, 16384, 1024, 1), (1, 2048, 1024, 5), (1, 16384, 3072, 5),
    (1, 11008, 4096, 5),
    # M = 2 over few rows: the row GEMV (up to 1024 rows, 2048 at K = 8192..16384)
    (2, 512, 8192, 5), (2, 1024, 4096, 5), (2, 2048, 16384, 5), (2, 2048, 28672, 7), (2, 2048, 4096, 6),
    # M = 33..56 at short K over at most ~12K rows: the small-batch kernel instead of the 64-row tiles
    (33, 8192, 2048, 6), (40, 12288, 3072, 6), (48, 11008, 1024, 6), (56, 8192, 2048, 6),
    (48, 9216, 2048, 2), (33, 13824, 2048, 2), (64, 8192, 2048, 2), (56, 11008, 4096, 2),
    # M = 17..32, K = 2048..4096 over 28672+ rows: the split-K kernel without a split (no workspace)
    (32, 28672, 4096, 7), (17, 28672, 4096, 7), (20, 40960, 2048, 7), (24, 24576, 4096, 6),
    (16, 28672, 4096, 6),
    # M = 2..32 from K = 5120: split K over 14336+ rows, at any M from K = 11008, from 16 rows at
    # K = 8192, from 24 rows; the small-batch kernel below that
    (32, 27648, 5120, 7), (2, 28672, 5120, 7), (8, 14336, 8192, 7), (16, 8192, 11008, 7),
    (24, 4096, 8192, 7), (32, 8192, 5120, 7), (24, 8192, 5120, 7), (2, 4096, 14336, 7), (16, 4096, 8192, 7),
    (8, 8192, 8192, 6), (16, 8192, 5120, 6), (4, 4096, 8192, 6),
    # ... and from 28 rows at K = 3072..4096 over at most 4096 rows, from 20 rows at K = 4096 over
    # 14336-20480 rows
    (32, 2048, 4096, 7), (28, 4096, 3072, 7), (24, 2048, 4096, 6), (32, 6144, 4096, 6), (32, 4096, 2048, 6),
    (20, 14336, 4096, 7), (32, 20480, 4096, 7), (19, 14336, 4096, 6), (24, 12288, 4096, 6), (24, 24576, 4096, 6),
    # ... and from K = 8192 over at most 2048 rows
    (4, 512, 8192, 7), (8, 2048, 8192, 7), (8, 2048, 4096, 6),
    # M = 33 (the extra-row form): over 28672+ rows, over 11008+ from K = 4096, over 6144+ from
    # K = 5120; the tiles or the small-batch kernel below
    (33, 28672, 3072, 7), (33, 57344, 1024, 7), (33, 11008, 4096, 7), (33, 6144, 5120, 7),
    (33, 8192, 4096, 2), (33, 16384, 2048, 2), (33, 4096, 3072, 6),
    # M = 33..64: split K up to 48 rows from K = 8192, over 32768+ rows from K = 4096, from
    # K = 14336 (not at M > 56 over 8192 rows), over at most 4096 rows from K = 4096; else the
    # 64-row tiles
    (33, 16384, 16384, 7), (48, 8192, 28672, 7), (64, 32768, 16384, 7), (40, 32768, 8192, 7),
    (64, 4096, 8192, 7), (64, 16384, 16384, 7), (40, 16384, 8192, 7), (48, 32768, 4096, 7),
    (64, 8192, 28672, 2), (56, 16384, 4096, 2), (64, 8192, 8192, 2), (56, 11008, 8192, 2),
    # M = 34..48 (three 16-row tiles): over 28672+ rows, from K = 4096 over 6144+ rows, at
    # K = 3072 over at most 2048 rows
    (40, 28672, 1024, 7), (48, 16384, 4096, 7), (36, 6144, 4096, 7), (40, 2048, 3072, 7),
    (40, 4096, 3072, 6), (48, 11008, 2048, 2),
    # M = 49..64 (four 16-row tiles): below 8192 rows from K = 4096 (below 6144 from K = 3072), over
    # 57344+ rows (from K = 3072 at M > 56), over 28672-32768 from K = 2048 (4096 at M > 56), over
    # 16384+ from K = 5120, up to M = 56 over 8192 rows from K = 8192
    (64, 6144, 4096, 7), (52, 4608, 3584, 7), (52, 6144, 3072, 6), (52, 37888, 3584, 2), (52, 57344, 1024, 7), (64, 57344, 1024, 2), (56, 28672, 2048, 7), (64, 28672, 2048, 2),
    (64, 16384, 5120, 7), (56, 8192, 8192, 7), (64, 11008, 4096, 2), (64, 16384, 4096, 2), (60, 6144, 2048, 6)])
def test_variant_selection_short_k_and_wide(M, N, K, expect):
    lib = _backend.load()
    assert lib.ra_w8a16_gemm_select(M, N, K, 1) == expect
    if expect == 7 and K <= 4096 and M <= 32 and N >= 28672:   # the unsplit split-K kernel: no workspace
        assert lib.ra_w8a16_gemm_workspace_size(M, N, K, 1) == 0


def test_workspace_of_the_tiled_split_plan():
    """M = 33..64 shapes whose tiled plan splits K (64 x 128 tiles over 4
    workgroups at M=64 K=11008 N=8192) ask for a workspace; the 64 x 64 tile
    over all of K (K=4096 N=11008) and large M need none from the tiled
    kernel (the size reported there is the split-K kernel's plan, for a forced
    RA_VARIANT_SPLITK launch)."""
    lib = _backend.load()
    assert lib.ra_w8a16_gemm_select(64, 8192, 11008, 0) == 2
    assert lib.ra_w8a16_gemm_workspace_size(64, 8192, 11008, 0) >= 16384 + 64 * 4 * 32768
    assert lib.ra_w8a16_gemm_workspace_size(2048, 11008, 4096, 0) == 0
    assert lib.ra_w8a16_gemm_workspace_size(1, 11008, 4096, 0) == 0
    # M = 65..1024: the split plans of 64- and 128-row tiles; at K=11008 N=4096
    # they split K, so they ask for a workspace; above M = 128 only where the
    # large tiles leave CUs idle (K=4096 N=28672: 224 tiles of 256 x 128 at
    # M=256); from M = 1025 none
    assert lib.ra_w8a16_gemm_select(128, 4096, 11008, 0) == 2
    assert lib.ra_w8a16_gemm_workspace_size(128, 4096, 11008, 0) > 16384
    assert lib.ra_w8a16_gemm_workspace_size(65, 4096, 11008, 0) > 16384
    assert lib.ra_w8a16_gemm_workspace_size(256, 4096, 11008, 0) > 16384
    assert lib.ra_w8a16_gemm_workspace_size(512, 4096, 11008, 0) > 16384
    assert lib.ra_w8a16_gemm_workspace_size(256, 28672, 4096, 0) == 0
    assert lib.ra_w8a16_gemm_workspace_size(1025, 4096, 11008, 0) == 0


def test_w8a8_argument_checks_without_device_work():
    lib = _backend.load()
    n = None
    buf = ctypes.create_string_buffer(256)
    p = ctypes.addressof(buf)
    # activation quantisation: fp16 / bf16 only, K = 0 rejected, M = 0 a no-op
    assert lib.ra_quantize_act_rows(p, 16, 2, 4, 16, p, 16, p, 127.0, n) == 2
    assert lib.ra_quantize_act_rows(p, 16, 0, 4, 0, p, 16, p, 127.0, n) == 1
    assert lib.ra_quantize_act_rows(n, 0, 0, 0, 16, n, 0, n, 127.0, n) == 0
    assert lib.ra_quantize_act_rows(p, 8, 0, 4, 16, p, 16, p, 127.0, n) == 1      # ldx < K
    assert lib.ra_quantize_act_rows(p, 16, 0, -1, 16, p, 16, p, 127.0, n) == 1
    # int8 GEMM: output dtype fp16 / bf16, bias dtype checked, leading dims
    assert lib.ra_w8a8_gemm(p, 16, p, p, 16, p, n, 0, p, 16, 2, 4, 4, 16, n) == 2
    assert lib.ra_w8a8_gemm(p, 16, p, p, 16, p, p, 9, p, 16, 0, 4, 4, 16, n) == 2
    assert lib.ra_w8a8_gemm(n, 0, n, n, 0, n, n, 0, n, 0, 0, 0, 4, 16, n) == 0
    assert lib.ra_w8a8_gemm(p, 8, p, p, 16, p, n, 0, p, 16, 0, 4, 4, 16, n) == 1  # ldxq < K
    assert lib.ra_w8a8_gemm(p, 16, n, p, 16, p, n, 0, p, 16, 0, 4, 4, 16, n) == 1  # no x scales
    assert lib.ra_w8a8_gemm(p, 16, p, p, 16, p, n, 0, p, 16, 0, 4, 4, -16, n) == 1


def test_workspace_constants_match_header():
    src = open(HEADER).read()
    assert int(re.search(r"#define RA_WORKSPACE_ALIGN (\d+)", src).group(1)) == _backend.WORKSPACE_ALIGN
    assert int(re.search(r"#define RA_WORKSPACE_COUNTER_BYTES (\d+)", src).group(1)) == \
        _backend.WORKSPACE_COUNTER_BYTES


def test_misaligned_workspace_refused_before_any_launch():
    """A workspace that does not start on a 256-byte boundary is RA_ERR_ARG
    (the kernels do 4-byte atomics on its counters and 16-byte stores of its
    partial sums), for the GEMM and the gate/up entry points alike; checked
    before kernel selection, so no device work happens."""
    lib = _backend.load()
    n = None
    buf = ctypes.create_string_buffer(4096)
    base = (ctypes.addressof(buf) + 255) // 256 * 256
    p = ctypes.addressof(buf)
    need = lib.ra_w8a16_gemm_workspace_size(17, 8192, 28672, 1)
    for off in (4, 16, 128):
        assert lib.ra_w8a16_gemm_ws(p, 28672, 1, p, 28672, p, n, 0, p, 8192, 17, 8192, 28672,
                                    base + off, need, n) == 1
        assert lib.ra_w8a16_gemm_ex(p, 28672, 1, p, 28672, p, n, 0, p, 8192, 17, 8192, 28672, 7,
                                    base + off, need, n) == 1
        assert lib.ra_w8a16_gateup_swiglu_ws(p, 16384, 1, p, 16384, p, p, 3000, 17, 3000, 16384,
                                             base + off, 1 << 30, n) == 1
    # an aligned but too small workspace still reports RA_ERR_WORKSPACE
    assert lib.ra_w8a16_gemm_ws(p, 28672, 1, p, 28672, p, n, 0, p, 8192, 17, 8192, 28672,
                                base, need - 1, n) == 6


def test_select_agrees_with_the_workspace_size():
    """Where the split-K plan does not split (S = 1) the problem needs no
    workspace: the split-K kernel runs unsplit with or without one given, so
    a call with a workspace runs what a call without one runs (M=8 K=16384
    N=65536, M=2 K=16384 N=128256; bitwise in tests/test_gpu_gemm.py). Where
    it does split, select reports split K and the size is non-zero."""
    lib = _backend.load()
    for (M, N, K) in ((8, 65536, 16384), (2, 128256, 16384)):
        assert lib.ra_w8a16_gemm_workspace_size(M, N, K, 1) == 0
        assert lib.ra_w8a16_gemm_select(M, N, K, 1) == 7
    for (M, N, K) in ((17, 8192, 28672), (8, 16384, 16384), (16, 4096, 11008)):
        assert lib.ra_w8a16_gemm_select(M, N, K, 1) == 7
        assert lib.ra_w8a16_gemm_workspace_size(M, N, K, 1) > _backend.WORKSPACE_COUNTER_BYTES


def test_gateup_workspace_only_where_gateup_splits():
    """The gate/up product runs the split-K kernel from K = 16384, from K = 8192
    over at most 4096 gate rows, at M = 33..64, and at M = 2..32 at M = 17,
    from 24 rows, from 16 rows at K = 8192, where K is not a multiple of
    1024, from K = 2048 over at most 4096 gate rows or from K = 3072 over at
    most 8192, and from 18 rows at K >= 5120 or over 14336+ gate rows at
    K <= 3072; elsewhere the size is 0,
    so the Python layer allocates no workspace it never uses. A plan that does
    not split K needs none either."""
    lib = _backend.load()
    assert lib.ra_w8a16_gateup_workspace_size(16, 14336, 4096, 1) == 0     # the one-pass kernels
    assert lib.ra_w8a16_gateup_workspace_size(17, 28672, 8192, 1) == 0     # a one-split plan
    assert lib.ra_w8a16_gateup_workspace_size(32, 14336, 4096, 1) > _backend.WORKSPACE_COUNTER_BYTES
    assert lib.ra_w8a16_gateup_workspace_size(8, 11008, 4096, 1) == 0
    assert lib.ra_w8a16_gateup_workspace_size(8, 4096, 1024, 1) == 0
    assert lib.ra_w8a16_gateup_workspace_size(8, 4097, 8192, 1) > _backend.WORKSPACE_COUNTER_BYTES
    assert lib.ra_w8a16_gateup_workspace_size(8, 2048, 4096, 1) > _backend.WORKSPACE_COUNTER_BYTES
    assert lib.ra_w8a16_gateup_workspace_size(20, 11008, 5120, 1) > _backend.WORKSPACE_COUNTER_BYTES
    assert lib.ra_w8a16_gateup_workspace_size(18, 11008, 4096, 1) == 0
    assert lib.ra_w8a16_gateup_workspace_size(17, 3000, 16384, 1) > _backend.WORKSPACE_COUNTER_BYTES
    assert lib.ra_w8a16_gateup_workspace_size(1, 3000, 16384, 1) == 0      # the row GEMV
    assert lib.ra_w8a16_gateup_workspace_size(48, 3000, 4096, 1) > _backend.WORKSPACE_COUNTER_BYTES
    assert lib.ra_w8a16_gateup_workspace_size(2, 3584, 16384, 1) > _backend.WORKSPACE_COUNTER_BYTES
    assert lib.ra_w8a16_gateup_workspace_size(2, 3584, 8192, 1) == 0   # M = 2, few gate rows: row GEMV
    assert lib.ra_w8a16_gateup_workspace_size(40, 3000, 4160, 1) == 0      # K % 128 != 0

