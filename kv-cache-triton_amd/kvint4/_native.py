"""ctypes binding of libkvint4.so (the C ABI declared in include/kvint4.h).

The shared library is built in-tree by ``kvint4.build`` (hipcc, gfx950). There
is deliberately no fallback: if the library is missing every operator raises,
so a GPU run can never silently compute on some other path.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkvint4.so")

KVQ_BF16, KVQ_F16, KVQ_F32 = 0, 1, 2
KVQ_OK, KVQ_EINVAL, KVQ_ESPACE, KVQ_EHIP, KVQ_EUNSUP = 0, -1, -2, -3, -4

# The argument lists below are those of major version 2 (KVQ_VERSION in
# include/kvint4.h: major*10000 + minor*100 + patch); a library of another
# major version would take them in another order, so it is refused.
KVQ_MAJOR = 2

DTYPE_CODE = {torch.bfloat16: KVQ_BF16, torch.float16: KVQ_F16, torch.float32: KVQ_F32}

# Every symbol include/kvint4.h declares (checked by the CPU test suite).
EXPORTED_SYMBOLS = (
    "kvq_version",
    "kvq_last_error",
    "kvq_quantize",
    "kvq_dequantize",
    "kvq_decode_attn_num_splits",
    "kvq_decode_attn_workspace_bytes",
    "kvq_decode_attn",
    "kvq_decode_step",
    "kvq_decode_step_noalloc",
    "kvq_quantize_paged",
    "kvq_dequantize_paged",
    "kvq_decode_attn_paged",
    "kvq_decode_step_paged",
    "kvq_prefill_attn",
    "kvq_prefill_attn_workspace_bytes",
    "kvq_prefill_attn_paged",
)

_lock = threading.Lock()
_lib = None

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_vp = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)


class KVQUnsupported(Exception):
    """The fused kernel does not handle this shape (KVQ_EUNSUP)."""


def _declare(lib: ctypes.CDLL) -> None:
    lib.kvq_version.restype = _i32
    lib.kvq_version.argtypes = []
    lib.kvq_last_error.restype = ctypes.c_char_p
    lib.kvq_last_error.argtypes = []
    lib.kvq_quantize.restype = _i32
    lib.kvq_quantize.argtypes = [
        _vp, _i32, _i64p, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64p, _vp, _i32, _i64p, _vp, _i64, _i64, _vp,
    ]
    lib.kvq_dequantize.restype = _i32
    lib.kvq_dequantize.argtypes = [
        _vp, _i64p, _vp, _i32, _i64p, _i64, _i64, _i64, _i64, _i64,
        _vp, _i32, _i64p, _i64, _vp,
    ]
    lib.kvq_decode_attn_num_splits.restype = _i64
    lib.kvq_decode_attn_num_splits.argtypes = [_i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i64]
    lib.kvq_decode_attn_workspace_bytes.restype = _i64
    lib.kvq_decode_attn_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i64]
    lib.kvq_decode_attn.restype = _i32
    lib.kvq_decode_attn.argtypes = [
        _vp, _i32, _i64p,
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        _i32,
        _vp, _i64p,
        _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        _vp, _i32, ctypes.c_float,
        _i64, _vp, _i64, _vp,
    ]
    lib.kvq_decode_step.restype = _i32
    lib.kvq_decode_step.argtypes = [
        _vp, _i32, _i64p,
        _vp, _i64p, _vp, _i64p,
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        _i32,
        _vp, _i64p,
        _i64, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, ctypes.c_float,
        _i64, _vp, _i64, _vp,
    ]
    lib.kvq_decode_step_noalloc.restype = _i32
    lib.kvq_decode_step_noalloc.argtypes = [
        _vp, _i32, _i64p,
        _vp, _i64p, _vp, _i64p,
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        _i32,
        _vp, _i64p,
        _i64, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, ctypes.c_float,
        _i64, _vp,
    ]
    lib.kvq_prefill_attn_workspace_bytes.restype = _i64
    lib.kvq_prefill_attn_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64, _i64, _i64]
    lib.kvq_prefill_attn.restype = _i32
    lib.kvq_prefill_attn.argtypes = [
        _vp, _i32, _i64p,
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        _i32,
        _vp, _i64p,
        _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        _i32, ctypes.c_float, _vp, _i64, _vp,
    ]
    # paged counterparts: (block_table, table_stride, table_cols, num_blocks,
    # page_size) after the cache arguments; pool strides are (head, row)
    pg = [_vp, _i64, _i64, _i64, _i64]
    lib.kvq_prefill_attn_paged.restype = _i32
    lib.kvq_prefill_attn_paged.argtypes = [
        _vp, _i32, _i64p,
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        _i32, *pg,
        _vp, _i64p,
        _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        _i32, ctypes.c_float, _vp, _i64, _vp,
    ]
    lib.kvq_quantize_paged.restype = _i32
    lib.kvq_quantize_paged.argtypes = [
        _vp, _i32, _i64p, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64p, _vp, _i32, _i64p, *pg, _vp, _i64, _vp,
    ]
    lib.kvq_dequantize_paged.restype = _i32
    lib.kvq_dequantize_paged.argtypes = [
        _vp, _i64p, _vp, _i32, _i64p, *pg,
        _i64, _i64, _i64, _i64, _i64, _vp, _i32, _i64p, _i64, _vp,
    ]
    lib.kvq_decode_attn_paged.restype = _i32
    lib.kvq_decode_attn_paged.argtypes = [
        _vp, _i32, _i64p,
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        _i32, *pg,
        _vp, _i64p,
        _i64, _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, _i32, ctypes.c_float,
        _i64, _vp, _i64, _vp,
    ]
    lib.kvq_decode_step_paged.restype = _i32
    lib.kvq_decode_step_paged.argtypes = [
        _vp, _i32, _i64p,
        _vp, _i64p, _vp, _i64p,
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        _i32, *pg,
        _vp, _i64p,
        _i64, _i64, _i64, _i64, _i64,
        _vp, _i64, ctypes.c_float,
        _i64, _vp, _i64, _vp,
    ]


def lib() -> ctypes.CDLL:
    """Load (once) and return the native library; raise if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"kvint4: native library not found at {LIB_PATH}; build it first "
                    "(python -m kvint4.build, or __graft_entry__.build())"
                )
            handle = ctypes.CDLL(LIB_PATH)
            _declare(handle)
            version = int(handle.kvq_version())
            if version // 10000 != KVQ_MAJOR:
                raise RuntimeError(
                    f"kvint4: {LIB_PATH} is version {version}, this binding needs major version "
                    f"{KVQ_MAJOR}; rebuild it (python -m kvint4.build)"
                )
            _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().kvq_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Translate a kvq status code into the reference's exception types."""
    if rc == KVQ_OK:
        return
    msg = last_error() or what
    if rc == KVQ_EINVAL:
        raise ValueError(msg)
    if rc == KVQ_EUNSUP:
        raise KVQUnsupported(msg)
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


def i64_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (ctypes.c_int64 * len(vals))(*vals)


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class device_of:
    """Make `tensor`'s device current for the duration of a native call."""

    def __init__(self, t: torch.Tensor):
        self.idx = t.device.index
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if self.idx is not None and cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False
