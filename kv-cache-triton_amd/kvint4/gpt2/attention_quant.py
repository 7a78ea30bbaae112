"""Fused attention over INT4-packed K/V cache for GPT-2 (MHA, HIP, gfx950).

Mirrors ``attention_forward_quant`` of ``kernels/gpt2/attention_quant.py``
(:140-248): same validation and messages; q must be fp16 or fp32. Runs the same
fused kernel as the Llama path with n_kv == n_q (GQA ratio 1). Keyword-only
additions: ``scale`` (default d**-0.5) and ``seq_lens`` (ragged batches).
"""

from __future__ import annotations

import math

import torch

from .. import ops


def attention_forward_quant(
    q: torch.Tensor,
    k_packed: torch.Tensor,
    k_scales: torch.Tensor,
    v_packed: torch.Tensor,
    v_scales: torch.Tensor,
    *,
    group_size: int = 32,
    is_causal: bool = False,
    scale: float | None = None,
    seq_lens: torch.Tensor | None = None,
) -> torch.Tensor:
    """Scaled dot-product attention using packed INT4 K/V cache."""
    if group_size <= 0:
        raise ValueError("group_size must be > 0")
    if not q.is_cuda:
        raise ValueError("attention_forward_quant expects CUDA tensors")
    if q.dtype not in (torch.float16, torch.float32):
        raise ValueError("q must be float16 or float32")
    if k_packed.dtype != torch.uint8 or v_packed.dtype != torch.uint8:
        raise ValueError("k_packed and v_packed must be uint8")
    if k_scales.dtype not in (torch.float16, torch.float32, torch.bfloat16):
        raise ValueError("k_scales must be floating point")
    if v_scales.dtype not in (torch.float16, torch.float32, torch.bfloat16):
        raise ValueError("v_scales must be floating point")
    if not all(t.is_cuda for t in (k_packed, k_scales, v_packed, v_scales)):
        raise ValueError("attention_forward_quant expects CUDA tensors")
    if k_packed.shape != v_packed.shape:
        raise ValueError("k_packed and v_packed must have the same shape")
    if k_scales.shape != v_scales.shape:
        raise ValueError("k_scales and v_scales must have the same shape")
    if k_packed.shape[:-1] != k_scales.shape[:-1]:
        raise ValueError("packed/scales leading dimensions must match")
    if q.dim() != 4:
        raise ValueError("q must be 4D: [B, H, sq, d_head]")
    b, h, sq, d = q.shape
    if tuple(k_packed.shape[:2]) != (b, h):
        raise ValueError("batch/head dimensions must match q")
    if tuple(k_scales.shape[:2]) != (b, h):
        raise ValueError("batch/head dimensions must match q")
    if k_packed.shape[-1] < math.ceil(d / 2):
        raise ValueError("packed last dimension is too small for q d_head")
    if k_scales.shape[-1] < math.ceil(d / group_size):
        raise ValueError("scales last dimension is too small for q d_head/group_size")
    sm_scale = d ** -0.5 if scale is None else float(scale)
    return ops.attention_over_quantized(
        q, k_packed, k_scales, v_packed, v_scales,
        n_kv_heads=h, group_size=group_size, is_causal=is_causal,
        sm_scale=sm_scale, seq_lens=seq_lens,
    )
