"""ctypes binding of libgqa_hip.so (C ABI: include/gqa_attn.h).

The library is built in-tree by ``gqa-flash-attn-rtx3060_amd/build.py`` and
lives next to this file.  There is no fallback: if the library is missing or
does not export the expected symbols, ``load()`` raises, so a GPU run can never
silently take another path.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libgqa_hip.so"

DTYPE_BF16 = 0
DTYPE_FP16 = 1

GQA_MAX_SPLITS = 1024
GQA_MAX_BLOCK_SIZE = 65536
GQA_PAGED_CHUNK_PAGES = 2048
GQA_NOALLOC_SCRATCH_BYTES = 16 << 20
GQA_E_SCRATCH = -9
ABI_VERSION = 13

_i64x4 = ctypes.c_int64 * 4
_i64x3 = ctypes.c_int64 * 3
_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float

# (name, restype, argtypes) for every entry point of include/gqa_attn.h.
SIGNATURES = {
    "gqa_abi_version": (_i, []),
    "gqa_strerror": (ctypes.c_char_p, [_i]),
    "gqa_device_cu_count": (_i, [_i]),
    "gqa_fwd_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i64x4, _i, _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_split_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i, _i, _i]),
    "gqa_split_first_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i, _i, _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_split_reduce_launch": (_i, [_p, _i, _p, _i64x4, _i, _i, _i, _i, _i, _p]),
    "gqa_fwd_lse_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i, _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_split_reduce_lse_launch": (_i, [_p, _i, _p, _i64x4, _p, _i, _i, _i, _i, _i, _p]),
    "gqa_split_fused_lse_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _p, _p, _i,
         _i, _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_split_counters_count": (ctypes.c_size_t, [_i, _i, _i, _i]),
    "gqa_split_fused_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _p, _i,
         _i, _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_fwd_split_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i, _i]),
    "gqa_fwd_split_counters_count": (ctypes.c_size_t, [_i, _i, _i]),
    "gqa_fwd_split_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _p, _p, _i,
         _i, _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_fwd_chunks_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _p, _p, _i,
         _i, _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_paged_split_first_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i, _p, _p, _p, _i, _i, _p, _i,
         _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_split_reduce_varlen_launch": (_i, [_p, _i, _p, _i64x4, _p, _p, _p, _i, _i, _i, _i, _i, _p]),
    "gqa_paged_fwd_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i, _p, _p, _p, _i, _i, _p, _i64x4, _p,
         _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_paged_fwd_chunks_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i, _p, _p, _p, _i, _i, _p, _i64x4, _p, _p, _i,
         _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_paged_fwd_split_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i, _p, _p, _p, _i, _i, _p, _i64x4, _p, _p, _p, _i,
         _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_paged_cache_write_launch": (
        _i,
        [_p, _i64x3, _p, _i64x3, _p, _i64x4, _p, _i64x4, _p, _i, _i, _i, _i, _i, _p],
    ),
    "gqa_split_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _p, _i,
         _i, _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
    "gqa_split_noalloc_launch": (
        _i,
        [_p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i64x4, _p, _i,
         _i, _i, _i, _i, _i, _i, _f, _i, _i, _p],
    ),
}

_lock = threading.Lock()
_lib = None


class GQAError(RuntimeError):
    """A launcher in libgqa_hip.so returned a non-zero code."""


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} not found: build it with "
                "`python gqa-flash-attn-rtx3060_amd/build.py` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError if a symbol is missing
            fn.restype = res
            fn.argtypes = args
        if lib.gqa_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"libgqa_hip.so ABI {lib.gqa_abi_version()} != expected {ABI_VERSION}; rebuild"
            )
        _lib = lib
        return lib


HOST_PATH = Path(__file__).resolve().parent / "_gqa_host.so"
_host = None


def load_host():
    """Load (once) and return the torch-tensor binding of the decode call
    (``_gqa_host.so``, built beside the library by build.py); raises if it
    is missing or was built against another library ABI."""
    global _host
    if _host is not None:
        return _host
    load()  # the library it links against, checked first (takes _lock itself)
    with _lock:
        if _host is not None:
            return _host
        import importlib.util

        if not HOST_PATH.exists():
            raise RuntimeError(f"{HOST_PATH} not found: build it with `python gqa-flash-attn-rtx3060_amd/build.py`")
        spec = importlib.util.spec_from_file_location("gqa_kernels._gqa_host", str(HOST_PATH))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        if mod.ABI_VERSION != ABI_VERSION:
            raise RuntimeError(f"_gqa_host.so built against ABI {mod.ABI_VERSION} != {ABI_VERSION}; rebuild")
        _host = mod
        return mod


def check(code: int) -> None:
    """Raise GQAError with the library's message for a non-zero return code."""
    if code != 0:
        msg = load().gqa_strerror(code).decode()
        raise GQAError(f"libgqa_hip error {code}: {msg}")


# C stride arrays by stride tuple: the launchers copy the strides before they
# return, so one array can serve every call with the same layout.
_stride_arrays: dict = {}


def strides(t) -> "ctypes.Array":
    """The 4 element strides of a torch tensor as a C int64[4]."""
    st = t.stride()
    arr = _stride_arrays.get(st)
    if arr is None:
        if len(_stride_arrays) > 4096:
            _stride_arrays.clear()
        arr = _stride_arrays[st] = _i64x4(*st)
    return arr


def strides3(t) -> "ctypes.Array":
    """The 3 element strides of a 3-d torch tensor as a C int64[3]."""
    return _i64x3(*t.stride())
