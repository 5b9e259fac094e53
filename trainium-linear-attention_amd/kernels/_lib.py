"""ctypes binding of libbased_la.so (the C ABI declared in include/based_la.h).

The library is loaded lazily, after ``import torch`` so that its HIP runtime dependency
resolves to the runtime torch has already mapped; launches go on torch's current stream.
There is no fallback: if the library is missing or fails to load, every call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("BASED_LA_LIB", os.path.join(_PKG, "libbased_la.so"))

LA_F32 = 0
LA_BF16 = 1

_lib = None
_lock = threading.Lock()

_c_void = ctypes.c_void_p
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_size = ctypes.c_size_t

_SIGNATURES = {
    "la_abi_version": (_c_int, []),
    "la_status_string": (ctypes.c_char_p, [_c_int]),
    "la_based_parallel_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "la_based_parallel_fwd": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_int, _c_void,
                                       _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_float, _c_int,
                                       _c_void, _c_size, _c_void]),
    "la_based_parallel_pack": (_c_int, [_c_void, _c_void, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void,
                                        _c_size, _c_void]),
    "la_based_parallel_fwd_packed": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_int, _c_void,
                                              _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_float, _c_int,
                                              _c_void, _c_size, _c_void]),
    "la_based_chunked_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "la_based_chunked_workspace_bytes_dt": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "la_based_chunked_chunk_used": (_c_int, [_c_int]),
    "la_based_chunked_fwd": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_int, _c_int, _c_int,
                                      _c_int, _c_int, _c_int, _c_int, _c_float, _c_float, _c_int, _c_void,
                                      _c_size, _c_void, _c_void]),
    "la_based_chunked_fwd_num_den": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_void, _c_int, _c_int,
                                              _c_int, _c_int, _c_int, _c_int, _c_float, _c_void, _c_size, _c_void]),
    "la_based_chunked_fwd_noalloc": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_int, _c_int, _c_int,
                                              _c_int, _c_int, _c_int, _c_int, _c_float, _c_float, _c_int, _c_void,
                                              _c_void]),
    "la_sliding_window_fwd": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_int, _c_int, _c_int,
                                       _c_int, _c_int, _c_int, _c_int, _c_float, _c_void]),
    "la_sliding_window_fwd_add": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_void, _c_int, _c_int,
                                           _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_void]),
    "la_based_chunked_fwd_continue": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_int, _c_int, _c_int,
                                               _c_int, _c_int, _c_int, _c_int, _c_float, _c_float, _c_int, _c_void,
                                               _c_size, _c_void, ctypes.c_longlong, _c_void, _c_void]),
    "la_based_layer_fwd": (_c_int, [_c_void, _c_void, _c_void, _c_void, _c_void, _c_int, _c_void, _c_int, _c_int,
                                    _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_float, _c_float,
                                    _c_void, _c_size, _c_void]),
    "la_based_decode_step": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_void, _c_int, _c_int, _c_int,
                                      _c_int, _c_int, _c_float, _c_int, _c_void]),
    "la_based_decode_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "la_based_decode_step_ws": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_void, _c_int, _c_int,
                                         _c_int, _c_int, _c_int, _c_float, _c_int, _c_void, _c_size, _c_void]),
    "la_identity_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "la_identity_linear_fwd": (_c_int, [_c_void, _c_void, _c_void, _c_int, _c_void, _c_int, _c_int, _c_int, _c_int,
                                        _c_int, _c_int, _c_float, _c_void, _c_size, _c_void]),
    "la_taylor_feature_map": (_c_int, [_c_void, _c_int, _c_void, _c_int, ctypes.c_longlong, _c_int, _c_void]),
}

EXPECTED_ABI = 10


class BasedLAError(RuntimeError):
    """Raised when a libbased_la call returns a non-zero status."""


def lib():
    """Return the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise BasedLAError(
                    f"libbased_la.so not found at {LIB_PATH}; build it with "
                    "`python trainium-linear-attention_amd/build.py` (hipcc, gfx950)")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            abi = handle.la_abi_version()
            if abi != EXPECTED_ABI:
                raise BasedLAError(f"libbased_la ABI {abi}, expected {EXPECTED_ABI}")
            _lib = handle
    return _lib


def status_string(rc: int) -> str:
    return lib().la_status_string(rc).decode()


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise BasedLAError(f"{what} failed: {status_string(rc)} (status {rc})")


def hip_runtimes_loaded():
    """Paths of every libamdhip64 mapped into this process (one is expected)."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64" in parts[-1]:
                paths.add(os.path.realpath(parts[-1]))
    return sorted(paths)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return LA_F32
    if dt == torch.bfloat16:
        return LA_BF16
    raise BasedLAError(f"unsupported dtype {dt}")


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> None:
    """The HIP path only: CPU tensors are an error, never silently computed on the host."""
    dev = tensors[0].device
    for t in tensors:
        if not t.is_cuda:
            raise BasedLAError("tensors must be on a ROCm (cuda) device; there is no CPU path")
        if t.device != dev:
            raise BasedLAError("all tensors must be on the same device")
