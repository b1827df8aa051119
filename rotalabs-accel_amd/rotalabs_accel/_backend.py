"""ctypes binding of librotaccel.so (C ABI declared in include/rotaccel.h).

The GPU branch of every op in this package calls into this library. There is
no silent fallback: if a CUDA/HIP tensor reaches an op and the library cannot
be loaded, the op raises ``RuntimeError`` (build it with
``python -m rotalabs_accel._build`` or ``__graft_entry__.build()``).

Set ``ROTACCEL_LIB`` to load the library from another path.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_DEFAULT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "librotaccel.so")
_lock = threading.Lock()
_lib = None
_load_error: str | None = None

ABI_VERSION = 6

# enum ra_dtype
F16, BF16, F32 = 0, 1, 2
# enum ra_variant
(VARIANT_AUTO, VARIANT_SKINNY, VARIANT_TILED, VARIANT_GENERIC, VARIANT_GEMV, VARIANT_ROWS, VARIANT_BATCH,
 VARIANT_SPLITK, VARIANT_SPLITK_SPREAD) = range(9)

_DTYPE_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}


def lib_path() -> str:
    return os.environ.get("ROTACCEL_LIB", _LIB_DEFAULT)


def _declare(lib: ctypes.CDLL) -> None:
    p, i32, i64, f32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
    sig = {
        "ra_abi_version": ([], i32),
        "ra_strerror": ([i32], ctypes.c_char_p),
        "ra_w8a16_gemm": ([p, i64, i32, p, i64, p, p, i32, p, i64, i64, i64, i64, p], i32),
        "ra_w8a16_gemm_ex": ([p, i64, i32, p, i64, p, p, i32, p, i64, i64, i64, i64, i32, p, sz, p], i32),
        "ra_w8a16_gemm_ws": ([p, i64, i32, p, i64, p, p, i32, p, i64, i64, i64, i64, p, sz, p], i32),
        "ra_w8a16_gemm_workspace_size": ([i64, i64, i64, i32], sz),
        "ra_w8a16_gemm_noalloc": ([p, i64, i32, p, i64, p, p, i32, p, i64, i64, i64, i64, p], i32),
        "ra_w8a16_gateup_swiglu_ws": ([p, i64, i32, p, i64, p, p, i64, i64, i64, i64, p, sz, p], i32),
        "ra_w8a16_gateup_workspace_size": ([i64, i64, i64, i32], sz),
        "ra_w8a16_gemm_select": ([i64, i64, i64, i32], i32),
        "ra_w8a16_gateup_swiglu": ([p, i64, i32, p, i64, p, p, i64, i64, i64, i64, p], i32),
        "ra_rmsnorm": ([p, i64, i32, p, i32, p, i64, i32, i64, i64, f32, p], i32),
        "ra_rmsnorm_residual": ([p, i64, i32, p, i64, i32, p, i32, p, i64, i32, i64, i64, f32, p], i32),
        "ra_swiglu": ([p, p, p, i64, i32, p], i32),
        "ra_swiglu_bias": ([p, p, p, p, i32, p, i64, i64, i32, p], i32),
        "ra_quantize_per_channel": ([p, i64, i32, i64, i64, p, i64, p, p], i32),
        "ra_quantize_rows": ([p, i64, i32, i64, i64, i32, p, i64, p, p], i32),
        "ra_quantize_act_rows": ([p, i64, i32, i64, i64, p, i64, p, f32, p], i32),
        "ra_w8a8_gemm": ([p, i64, p, p, i64, p, p, i32, p, i64, i32, i64, i64, i64, p], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res


def load():
    """Load (once) and return the library; raise RuntimeError if impossible."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        try:
            lib = ctypes.CDLL(path)
            _declare(lib)
        except (OSError, AttributeError) as e:  # AttributeError: a symbol of this ABI is missing
            _load_error = f"cannot load {path}: {e}"
            raise RuntimeError(
                f"rotalabs_accel: the HIP library is required for GPU tensors but {_load_error}. "
                "Build it with `python -m rotalabs_accel._build`."
            ) from e
        ver = lib.ra_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"rotalabs_accel: {path} has ABI {ver}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def check(code: int) -> None:
    if code != 0:
        raise RuntimeError(load().ra_strerror(code).decode())


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"rotalabs_accel: unsupported dtype {dtype} on the GPU path "
                        "(float16, bfloat16 and float32 are supported)") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (as an integer).
    Read without building a Stream object where torch offers that (the
    object costs ~1.7 us of host time per call)."""
    if _raw_stream is not None:
        return _raw_stream(_device_index(device))
    return torch.cuda.current_stream(device).cuda_stream


_workspaces: dict = {}
_WS_ROUND = 1 << 20


def workspace(device: torch.device, nbytes: int):
    """(pointer, bytes) of a zero-filled device workspace of at least
    ``nbytes`` for launches on torch's current stream of ``device``, or
    (None, 0) when ``nbytes`` is 0.

    The kernels that use a workspace leave it as they found it (their
    counters back at zero), so one buffer serves every call issued on a
    stream; each stream gets its own, as calls on different streams may
    overlap. The buffer comes from torch's allocator (also during graph
    capture, where its zero fill is recorded as a kernel) and grows in 1 MiB
    steps when a larger problem needs more."""
    if nbytes <= 0:
        return None, 0
    key = (_device_index(device), stream_handle(device))
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        size = -(-nbytes // _WS_ROUND) * _WS_ROUND
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws.data_ptr(), ws.numel()


class on_device:
    """Make ``device`` current for the duration of a launch (kernels launch on
    the current HIP device); a no-op when it already is."""

    __slots__ = ("idx", "prev")

    def __init__(self, device: torch.device):
        self.idx = device.index if device.index is not None else torch.cuda.current_device()
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False
