"""CPU oracle for the INT4 KV path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker / the timed CPU
baseline. The product path (``kvint4``) never calls it.

This is a numpy restatement of the reference's CPU path
(johnchmura/kv-cache-triton), function by function:

  quantize_int4     kernels/llama3/quantize.py:126-148 (_quantize_int4_torch);
                    kernels/gpt2/quantize.py:111-133 (identical codes, fp16 scales)
  dequantize_int4   kernels/llama3/quantize.py:210-234 (_dequantize_int4_torch);
                    kernels/gpt2/quantize.py:217-235 (fp16 output)
  attention         kernels/llama3/attention_quant.py:24-152 semantics (GQA map
                    h // ratio :71, bottom-right causal offset :91-97,123) as
                    restated by the reference's fp32 loop oracle
                    tests/llama3/test_attention_fused_vs_ref_sm70.py:14-51,
                    computed here in float64; per-sequence key lengths extend it
                    to ragged batches.
  cache_append      models/llama3/kv_cache.py:76-102 (append = concat on dim 2).

Numbers are carried as float32 *values*: a bf16/fp16 tensor is represented by
the float32 array of its exact values, and narrowing to bf16/fp16 is done with
round-to-nearest-even (`round_to`).

Pinning (tests/test_oracle_*.py): every function here is checked against the
exact-rational known-answer vectors in tests/golden/ (written by
tests/golden/make_kat.py with fractions.Fraction, no floating point), against
closed forms / invariants / brute force, against the C restatement
(oracle/kvq_ref.c), and — for attention — against torch's SDPA on the CPU.
"""

from __future__ import annotations

import math

import numpy as np

SCALE_DTYPES = ("bf16", "f16", "f32")


# ---------------------------------------------------------------------------
# float formats


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to bf16 / fp16 / fp32 (nearest, ties to even);
    returns float32 values."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
        r = np.where(nan, np.uint32(0x7FC00000), r)
        return r.view(np.float32)
    raise ValueError(f"unknown dtype {dtype}")


def bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """Bit patterns of values already representable in `dtype`."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x.view(np.uint32).copy()
    if dtype == "f16":
        return x.astype(np.float16).view(np.uint16).copy()
    if dtype == "bf16":
        return (x.view(np.uint32) >> 16).astype(np.uint16)
    raise ValueError(dtype)


def from_bits(b: np.ndarray, dtype: str) -> np.ndarray:
    b = np.asarray(b)
    if dtype == "f32":
        return b.astype(np.uint32).view(np.float32)
    if dtype == "f16":
        return b.astype(np.uint16).view(np.float16).astype(np.float32)
    if dtype == "bf16":
        return (b.astype(np.uint32) << 16).view(np.float32)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# quantize / dequantize


def quantize_int4(x: np.ndarray, group_size: int, scale_dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """Restates kernels/llama3/quantize.py:126-148.

    x: float32 values [..., d]. Returns (packed uint8 [..., ceil(d/G)*ceil(G/2)],
    scales float32 values rounded to `scale_dtype` [..., ceil(d/G)]).
    """
    if group_size <= 0:
        raise ValueError("group_size must be > 0")
    x = np.asarray(x, dtype=np.float32)
    lead = x.shape[:-1]
    d = x.shape[-1]
    ng = math.ceil(d / group_size)
    pad = ng * group_size - d
    work = x
    if pad > 0:
        work = np.pad(work, [(0, 0)] * (x.ndim - 1) + [(0, pad)])
    grouped = work.reshape(*lead, ng, group_size)
    if ng == 0:
        return (np.zeros((*lead, 0), np.uint8), np.zeros((*lead, 0), np.float32))
    max_abs = np.abs(grouped).max(axis=-1, keepdims=True)
    scales = np.where(max_abs > 0, max_abs / np.float32(7.0), np.float32(1.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint(grouped / scales)  # IEEE fp32 division, round half to even
    q = (np.clip(q, -8, 7).astype(np.int16) + 8).astype(np.uint8)
    if group_size % 2 != 0:
        q = np.pad(q, [(0, 0)] * (q.ndim - 1) + [(0, 1)])
    lo = q[..., 0::2]
    hi = q[..., 1::2] << 4
    packed = (lo | hi).reshape(*lead, -1)
    return packed, round_to(scales[..., 0], scale_dtype)


def dequantize_int4(
    packed: np.ndarray, scales: np.ndarray, group_size: int, d_head: int, out_dtype: str
) -> np.ndarray:
    """Restates kernels/llama3/quantize.py:210-234: (nibble - 8) * fp32(scale),
    first d_head columns, rounded once to out_dtype."""
    packed = np.asarray(packed, dtype=np.uint8)
    scales = np.asarray(scales, dtype=np.float32)
    ng = scales.shape[-1]
    lead = packed.shape[:-1]
    unpacked = np.empty((*lead, packed.shape[-1] * 2), dtype=np.float32)
    unpacked[..., 0::2] = (packed & 0x0F).astype(np.float32) - 8.0
    unpacked[..., 1::2] = ((packed >> 4) & 0x0F).astype(np.float32) - 8.0
    grouped = unpacked.reshape(*lead, ng, -1)
    if grouped.shape[-1] < group_size:
        raise ValueError("packed has insufficient width for the provided group_size")
    grouped = grouped[..., :group_size]
    out = (grouped * scales[..., None]).astype(np.float32)
    out = out.reshape(*lead, -1)[..., :d_head]
    return round_to(out, out_dtype)


def cache_append(cache: tuple | None, k: np.ndarray, v: np.ndarray, group_size: int, scale_dtype: str):
    """Restates models/llama3/kv_cache.py:76-102: quantize the new rows, then
    concatenate along the sequence axis (dim 2)."""
    kp, ks = quantize_int4(k, group_size, scale_dtype)
    vp, vs = quantize_int4(v, group_size, scale_dtype)
    if cache is None:
        return kp, ks, vp, vs
    return tuple(np.concatenate([a, b], axis=2) for a, b in zip(cache, (kp, ks, vp, vs)))


# ---------------------------------------------------------------------------
# attention


def attention(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    *,
    scale: float,
    is_causal: bool = False,
    seq_lens=None,
) -> np.ndarray:
    """softmax(q k^T * scale) v in float64 with the GQA map h -> h // (Hq/Hkv).

    q [B, Hq, Sq, D]; k, v [B, Hkv, Sk, D] (dequantized values). Sequence b
    attends its first L_b = min(seq_lens[b], Sk) keys; with is_causal, query i
    sees keys j <= L_b - Sq + i. A query row with no admissible key is zero.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    ratio = Hq // Hkv
    out = np.zeros((B, Hq, Sq, v.shape[-1]), dtype=np.float64)
    for b in range(B):
        L = Sk if seq_lens is None else max(0, min(int(seq_lens[b]), Sk))
        if L == 0:
            continue
        jj = np.arange(L)[None, :]
        ii = np.arange(Sq)[:, None]
        allowed = np.ones((Sq, L), dtype=bool)
        if is_causal:
            allowed = jj <= (L - Sq + ii)
        for h in range(Hkv):
            qg = q[b, h * ratio:(h + 1) * ratio]               # [r, Sq, D]
            s = np.einsum("rqd,kd->rqk", qg, k[b, h, :L]) * scale
            s = np.where(allowed[None], s, -np.inf)
            m = s.max(axis=-1, keepdims=True)
            ok = np.isfinite(m)
            e = np.where(allowed[None], np.exp(s - np.where(ok, m, 0.0)), 0.0)
            den = e.sum(axis=-1, keepdims=True)
            p = np.divide(e, den, out=np.zeros_like(e), where=den > 0)
            out[b, h * ratio:(h + 1) * ratio] = np.einsum("rqk,kd->rqd", p, v[b, h, :L])
    return out


def attention_over_quantized(
    q: np.ndarray,
    k_packed: np.ndarray,
    k_scales: np.ndarray,
    v_packed: np.ndarray,
    v_scales: np.ndarray,
    *,
    group_size: int,
    scale: float | None = None,
    is_causal: bool = False,
    seq_lens=None,
) -> np.ndarray:
    """Exact-dequant (fp32) attention over INT4 K/V, float64 math."""
    d = q.shape[-1]
    k = dequantize_int4(k_packed, k_scales, group_size, d, "f32")
    v = dequantize_int4(v_packed, v_scales, group_size, d, "f32")
    return attention(q, k, v, scale=d ** -0.5 if scale is None else scale,
                     is_causal=is_causal, seq_lens=seq_lens)
