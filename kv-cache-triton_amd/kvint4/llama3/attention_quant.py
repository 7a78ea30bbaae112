"""Fused GQA attention over INT4-packed K/V for Llama-3 (HIP, gfx950).

Mirrors ``attention_forward_quant_gqa`` of ``kernels/llama3/attention_quant.py``
(:159-286): same signature, validation order and ``ValueError`` messages.

    q:        [B, n_q,  sq, d]               bf16 / fp16 / fp32 (GPU)
    k_packed: [B, n_kv, sk, packed_width]    uint8
    k_scales: [B, n_kv, sk, n_groups]        bf16 / fp16 / fp32
    v_packed, v_scales: same as k
    returns   [B, n_q,  sq, d]               dtype of q

Query head h reads KV head h // (n_q // n_kv). Decode (and short query blocks)
run in the fused split-K kernel; prompts and long query blocks run in the
matrix-core prefill kernel, which dequantizes each K/V tile into LDS, so a
prefill also attends over the quantized K/V as the reference's prefill does.
What neither kernel takes (rows beyond the fused kernel's range that the
prefill kernel does not cover) dequantizes the cache in HIP and runs SDPA.

Additions over the reference signature (keyword-only, default to the
reference's behaviour): ``scale`` (default d**-0.5, :231) and ``seq_lens``
(device int32 [B] of per-sequence key lengths for ragged batches; the rows
past a sequence's length are ignored).
"""

from __future__ import annotations

import math

import torch

from .. import ops

_Q_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
_SCALE_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def attention_forward_quant_gqa(
    q: torch.Tensor,
    k_packed: torch.Tensor,
    k_scales: torch.Tensor,
    v_packed: torch.Tensor,
    v_scales: torch.Tensor,
    *,
    n_q_heads: int,
    n_kv_heads: int,
    group_size: int = 32,
    is_causal: bool = False,
    scale: float | None = None,
    seq_lens: torch.Tensor | None = None,
) -> torch.Tensor:
    """Fused GQA scaled-dot-product attention reading packed INT4 K/V."""
    if group_size <= 0:
        raise ValueError("group_size must be > 0")
    if n_q_heads <= 0 or n_kv_heads <= 0:
        raise ValueError("n_q_heads and n_kv_heads must be > 0")
    if n_q_heads % n_kv_heads != 0:
        raise ValueError("n_q_heads must be divisible by n_kv_heads")

    if not q.is_cuda:
        raise ValueError("attention_forward_quant_gqa expects CUDA tensors")
    if not all(t.is_cuda for t in (k_packed, k_scales, v_packed, v_scales)):
        raise ValueError("attention_forward_quant_gqa expects CUDA tensors")

    if q.dtype not in _Q_DTYPES:
        raise ValueError("q must be bf16/fp16/fp32")
    if k_packed.dtype != torch.uint8 or v_packed.dtype != torch.uint8:
        raise ValueError("k_packed and v_packed must be uint8")
    if k_scales.dtype not in _SCALE_DTYPES or v_scales.dtype not in _SCALE_DTYPES:
        raise ValueError("scales must be bf16/fp16/fp32")

    if k_packed.shape != v_packed.shape:
        raise ValueError("k_packed and v_packed must have the same shape")
    if k_scales.shape != v_scales.shape:
        raise ValueError("k_scales and v_scales must have the same shape")
    if k_packed.shape[:-1] != k_scales.shape[:-1]:
        raise ValueError("packed/scales leading dimensions must match")

    if q.dim() != 4:
        raise ValueError("q must be 4D: [B, n_q_heads, sq, d_head]")
    b, hq, sq, d = q.shape
    if hq != n_q_heads:
        raise ValueError(f"q head dim {hq} != n_q_heads {n_q_heads}")
    if k_packed.shape[0] != b or k_packed.shape[1] != n_kv_heads:
        raise ValueError("k/v leading dims must be [B, n_kv_heads, ...]")

    if k_packed.shape[-1] < math.ceil(d / 2):
        raise ValueError("packed last dimension is too small for q d_head")
    if k_scales.shape[-1] < math.ceil(d / group_size):
        raise ValueError("scales last dimension is too small for q d_head/group_size")

    sm_scale = d ** -0.5 if scale is None else float(scale)
    return ops.attention_over_quantized(
        q, k_packed, k_scales, v_packed, v_scales,
        n_kv_heads=n_kv_heads, group_size=group_size, is_causal=is_causal,
        sm_scale=sm_scale, seq_lens=seq_lens,
    )
