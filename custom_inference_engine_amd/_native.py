"""ctypes binding of ``libcie_paged.so`` (declared in include/cie_paged_attention.h).

The library is loaded after ``torch`` so it binds to the HIP runtime torch
already mapped (same soname, one runtime per process): the stream handles and
device pointers handed across the boundary are torch's own.  There is no CPU
or Python fallback: if the library is missing or the tensors are not on a HIP
device, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

from ._build import LIB_PATH as _BUILT_LIB

# The in-tree build.  (bench.py --lib times a trace or tuning build by pointing
# this at it before the first load; nothing in the package reads another path.)
LIB_PATH = _BUILT_LIB

_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p
_c_i64p = ctypes.c_void_p  # int64_t* passed as a raw device address

# name -> (restype, argtypes); mirrors include/cie_paged_attention.h
_SIGNATURES = {
    "cie_abi_version": (ctypes.c_int, []),
    "cie_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "cie_kv_append_decode": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64p, _c_i64p,
         _c_i64p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_kv_append_tokens": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64p, _c_i64p,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_paged_decode_partials_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "cie_paged_decode_max_splits": (ctypes.c_int, []),
    "cie_paged_decode": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64p, _c_i64p, _c_i64p, _c_ptr, _c_ptr, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_ptr, _c_ptr],
    ),
    "cie_paged_decode_append": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64p,
         _c_i64p, _c_i64p, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_paged_decode_noalloc_limit": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "cie_paged_decode_append_noalloc": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64p,
         _c_i64p, _c_i64p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_paged_decode_qkv_rope": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64p, _c_i64p, _c_i64p,
         _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_kv_append_tokens_qkv_rope": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64p, _c_i64p, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_paged_decode_plan_workgroups": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "cie_paged_decode_plan_bytes": (_c_i64, [_c_i64]),
    "cie_paged_decode_planned_partials_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "cie_paged_decode_plan": (
        ctypes.c_int,
        [_c_ptr, _c_i64p, _c_i64p, _c_i64p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_paged_decode_planned": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64p, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_paged_decode_append_planned": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr,
         _c_i64p, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_paged_decode_qkv_rope_planned": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_i64p, _c_ptr,
         _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_mixed_partials_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "cie_mixed_plan_bytes": (_c_i64, [_c_i64, _c_i64]),
    "cie_mixed_plan": (
        ctypes.c_int,
        [_c_ptr, _c_i64, _c_i64p, _c_i64p, _c_i64p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_mixed_attention_planned": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64p, _c_ptr, _c_i64, _c_ptr,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "cie_mixed_counters": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "cie_mixed_attention": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64p, _c_i64p, _c_i64p, _c_i64p, _c_ptr, _c_i64, _c_ptr,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
}

ABI_VERSION = 10

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NativeLibraryMissing(RuntimeError):
    pass


def lib_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(
                f"{LIB_PATH} is not built; run custom_inference_engine_amd._build.build()"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.cie_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().cie_status_string(status)
        raise RuntimeError(f"{what} failed: status {status} ({msg.decode() if msg else '?'})")


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one HIP device; the kernels have no CPU path."""
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            f"paged attention kernels run on a HIP device only (got a tensor on {dev}); "
            "there is no CPU fallback"
        )
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
