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

ABI_VERSION = 7

# include/rotaccel.h: workspace alignment and the bytes of its counter block
WORKSPACE_ALIGN = 256
WORKSPACE_COUNTER_BYTES = 16384

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
        "ra_stream_capture_info": ([p, ctypes.POINTER(i32), ctypes.POINTER(ctypes.c_ulonglong)], i32),
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


_workspaces: dict = {}   # (device, stream) -> buffer of the eager calls on that stream
_captured: dict = {}     # (device, stream, capture id) -> buffer of one graph capture
_held: list = []         # every buffer a captured graph may use: never released
_WS_ROUND = 1 << 20


def capture_info(stream: int) -> tuple[bool, int]:
    """(capturing, capture id) of a hipStream_t (the id is 0 when not capturing)."""
    cap, cid = ctypes.c_int(0), ctypes.c_ulonglong(0)
    check(load().ra_stream_capture_info(stream, ctypes.byref(cap), ctypes.byref(cid)))
    return bool(cap.value), int(cid.value)


def workspace(device: torch.device, nbytes: int):
    """(pointer, bytes) of a device workspace of at least ``nbytes`` whose
    counter block is zero when the next launch on torch's current stream of
    ``device`` reads it, or (None, 0) when ``nbytes`` is 0.

    The kernels that use a workspace leave its counters at zero, so one buffer
    serves a sequence of calls that run one after another:

    * Eager calls: one buffer per (device, stream), zero-filled when it is
      allocated (calls on different streams may overlap, so each stream has
      its own). A larger problem replaces it; the old buffer goes back to
      torch's allocator, which reuses its memory only for work ordered after
      the calls on that stream.
    * Calls under HIP graph capture: one buffer per capture (and capturing
      stream), allocated from the graph's memory pool when the capture first
      needs it, with the fill of its counter block recorded into the graph
      just before that call, so every replay clears the counters before the
      first kernel reads them -- whatever ran before the replay (another
      graph, eager calls) and whether or not this graph ever ran. Graphs never
      share a buffer, and no buffer a graph was captured with is released
      (they are held until the process ends), so a replay never reads memory
      that was handed to another tensor.

    Buffers are 256-byte aligned (torch's allocator aligns every block to at
    least 512 bytes) and grow in 1 MiB steps."""
    if nbytes <= 0:
        return None, 0
    dev = _device_index(device)
    stream = stream_handle(device)
    capturing, cid = capture_info(stream)
    size = -(-nbytes // _WS_ROUND) * _WS_ROUND
    if not capturing:
        key = (dev, stream)
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(size, dtype=torch.uint8, device=device)
            _workspaces[key] = ws
    else:
        key = (dev, stream, cid)
        ws = _captured.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(size, dtype=torch.uint8, device=device)
            ws[:WORKSPACE_COUNTER_BYTES].zero_()  # a fill kernel, recorded into the graph
            _captured[key] = ws
            _held.append(ws)
    assert ws.data_ptr() % WORKSPACE_ALIGN == 0
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
