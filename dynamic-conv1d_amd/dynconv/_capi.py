"""ctypes binding of libdynconv.so (C ABI declared in include/dynconv.h).

The library is loaded lazily after `import torch`, so it binds to the HIP
runtime torch has already mapped (both carry SONAME libamdhip64.so.7).
There is no fallback: if the library is missing or a call fails, a
RuntimeError is raised.
"""

import ctypes
import functools
import os
import threading

import torch

# DYNCONV_LIB selects another build of the library (the host-sanitizer build in
# tests/test_host_sanitize.py); by default the in-tree libdynconv.so.
LIB_PATH = os.environ.get("DYNCONV_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdynconv.so")
ABI_VERSION = 7

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_c_vp = ctypes.c_void_p
_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_pp = ctypes.POINTER(ctypes.c_void_p)  # host array of device pointers

# name -> (restype, argtypes); mirrors include/dynconv.h.
SIGNATURES = {
    "dc_abi_version": (_c_int, []),
    "dc_status_string": (ctypes.c_char_p, [_c_int]),
    "dc_headwise_fwd": (_c_int, [_c_vp] * 4 + [_c_i64] * 5 + [_c_int, _c_int, _c_vp]),
    "dc_headwise_path": (_c_int, [_c_i64] * 5 + [_c_int] * 3),
    "dc_lowrank_path": (_c_int, [_c_i64] * 5 + [_c_int] * 3),
    "dc_headwise_bwd_ws_bytes": (_c_i64, [_c_i64] * 5 + [_c_int, _c_int]),
    "dc_headwise_bwd": (_c_int, [_c_vp] * 8 + [_c_i64] + [_c_i64] * 5 + [_c_int, _c_int, _c_vp]),
    "dc_headwise_bwd_noalloc": (_c_int, [_c_vp] * 7 + [_c_i64] * 5 + [_c_int, _c_int, _c_vp]),
    "dc_lowrank_zeff_bytes": (_c_i64, [_c_i64] * 5 + [_c_int, _c_int]),
    "dc_lowrank_fwd": (_c_int, [_c_vp] * 6 + [_c_i64] + [_c_i64] * 5 + [_c_int, _c_int, _c_vp]),
    "dc_lowrank_bwd_ws_bytes": (_c_i64, [_c_i64] * 5 + [_c_int, _c_int]),
    "dc_lowrank_plan_ranges": (_c_i64, [_c_i64] * 5 + [_c_int] * 3 + [ctypes.POINTER(_c_i64), _c_i64]),
    "dc_lowrank_bwd": (_c_int, [_c_vp] * 5 + [_c_i64] + [_c_vp] * 6 + [_c_i64] + [_c_i64] * 5
                       + [_c_int, _c_int, _c_vp]),
    "dc_lowrank_fwd_grouped": (_c_int, [_c_i64, _c_vp, _c_i64] + [_c_pp] * 5 + [_c_i64] * 7 + [_c_int, _c_int, _c_vp]),
    "dc_lowrank_bwd_grouped_ws_bytes": (_c_i64, [_c_i64] * 6 + [_c_int, _c_int]),
    "dc_proj_in_fwd": (_c_int, [_c_vp, _c_vp, _c_pp] + [_c_i64] * 4 + [_c_int, _c_vp]),
    "dc_proj_in_bwd_ws_bytes": (_c_i64, [_c_i64] * 4 + [_c_int]),
    "dc_proj_in_bwd": (_c_int, [_c_vp, _c_vp, _c_pp, _c_vp, _c_vp, _c_vp, _c_i64] + [_c_i64] * 4 + [_c_int, _c_vp]),
    "dc_lowrank_bwd_grouped": (_c_int, [_c_i64, _c_vp, _c_i64] + [_c_pp] * 4 + [_c_i64] + [_c_pp]
                               + [_c_i64, _c_vp, _c_i64] + [_c_pp] * 3
                               + [_c_vp, _c_i64] + [_c_i64] * 5 + [_c_int, _c_int, _c_vp]),
}

_lib = None
_lock = threading.Lock()


def load(path: str = LIB_PATH):
    """Load (once) and return the ctypes handle of libdynconv.so."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"libdynconv.so not found at {path}; build it with "
                "`python dynamic-conv1d_amd/build.py` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.dc_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"libdynconv.so ABI version {ver}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


# dc_path codes (include/dynconv.h): which kernel family a shape runs on
PATHS = {0: "generic", 1: "vector", 2: "mfma", 3: "f32_mfma", 4: "f32_valu", 5: "wide", 6: "head_mfma"}


def status_string(status: int) -> str:
    return load().dc_status_string(status).decode()


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"dynconv {what} failed: {status_string(status)} (status {status})")


def ptr(t):
    return None if t is None else t.data_ptr()


def ptr_array(ts):
    """A host array of the tensors' device pointers (a `const void* const*` argument), or None."""
    if ts is None:
        return None
    return (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])


# torch's current-stream handle without building a Stream object (2 us -> 0.1 us per call)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None)


def on_tensor_device(fn):
    """Run an autograd Function's forward / backward with the device of its first tensor argument
    current: the C ABI launches on the current device (the stream handle is that device's), so a
    call on tensors of another GPU than the current one switches to theirs, as torch's own ops do.
    A no-op (one device query) when that device is current already."""

    @functools.wraps(fn)
    def wrapper(ctx, *args):
        t = next((a for a in args if isinstance(a, torch.Tensor)), None)
        if t is None or not t.is_cuda:
            return fn(ctx, *args)
        dev = t.get_device()
        cur = _get_device() if _get_device is not None else torch.cuda.current_device()
        if dev == cur:
            return fn(ctx, *args)
        with torch.cuda.device(dev):
            return fn(ctx, *args)

    return wrapper


def stream_of(t: torch.Tensor):
    """hipStream_t of torch's current stream on t's device."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dt]
    except KeyError:
        raise AssertionError(f"unsupported dtype {dt}; expected one of bfloat16, float16, float32") from None
