"""ctypes wrapper of oracle/libkvqref.so (the C restatement in kvq_ref.c).

TEST INFRASTRUCTURE ONLY — imported by tests/ and bench.py's cpu_baseline leg.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkvqref.so")
_DT = {"bf16": 0, "f16": 1, "f32": 2}
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from . import build as _build

            _build.build()
        l = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        l.kvqref_quantize.argtypes = [vp, i64, i64, i64, i32, vp, vp]
        l.kvqref_quantize.restype = None
        l.kvqref_dequantize.argtypes = [vp, vp, i64, i64, i64, i64, i32, vp]
        l.kvqref_dequantize.restype = None
        l.kvqref_decode_attn.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i64,
                                         vp, i32, ctypes.c_float, vp, i32]
        l.kvqref_decode_attn.restype = i32
        l.kvqref_num_threads.argtypes = []
        l.kvqref_num_threads.restype = i32
        l.kvqref_check_div7.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        l.kvqref_check_div7.restype = i64
        l.kvqref_check_rint_margin.argtypes = [ctypes.c_uint64, i64, ctypes.c_int, ctypes.c_int]
        l.kvqref_check_rint_margin.restype = i64
        l.kvqref_check_rint_margin_fma8.argtypes = [ctypes.c_uint64, i64, ctypes.c_int, ctypes.c_int]
        l.kvqref_check_rint_margin_fma8.restype = i64
        _lib = l
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def quantize_int4(x: np.ndarray, group_size: int, scale_dtype: str):
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[-1]
    rows = int(np.prod(x.shape[:-1]))
    ng = -(-d // group_size)
    w = ng * ((group_size + 1) // 2)
    packed = np.empty((*x.shape[:-1], w), np.uint8)
    scales = np.empty((*x.shape[:-1], ng), np.float32)
    lib().kvqref_quantize(_ptr(x), rows, d, group_size, _DT[scale_dtype], _ptr(packed), _ptr(scales))
    return packed, scales


def dequantize_int4(packed, scales, group_size: int, d_head: int, out_dtype: str):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    rows = int(np.prod(packed.shape[:-1]))
    ng = scales.shape[-1]
    out = np.empty((*packed.shape[:-1], d_head), np.float32)
    lib().kvqref_dequantize(_ptr(packed), _ptr(scales), rows, ng, group_size, d_head,
                            _DT[out_dtype], _ptr(out))
    return out


def decode_attn(q, kp, ks, vp, vs, *, group_size: int, scale: float, is_causal: bool = False,
                seq_lens=None, threads: int = 0):
    q = np.ascontiguousarray(q, dtype=np.float32)
    kp = np.ascontiguousarray(kp, dtype=np.uint8)
    vp = np.ascontiguousarray(vp, dtype=np.uint8)
    ks = np.ascontiguousarray(ks, dtype=np.float32)
    vs = np.ascontiguousarray(vs, dtype=np.float32)
    B, Hq, Sq, D = q.shape
    Hkv, Sk = kp.shape[1], kp.shape[2]
    out = np.empty_like(q)
    sl = None
    if seq_lens is not None:
        sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    rc = lib().kvqref_decode_attn(_ptr(q), _ptr(kp), _ptr(ks), _ptr(vp), _ptr(vs), B, Hq, Hkv, Sq,
                                  Sk, D, group_size, _ptr(sl) if sl is not None else None,
                                  1 if is_causal else 0, float(scale), _ptr(out), int(threads))
    if rc != 0:
        raise RuntimeError(f"kvqref_decode_attn failed ({rc})")
    return out


def num_threads() -> int:
    return int(lib().kvqref_num_threads())
