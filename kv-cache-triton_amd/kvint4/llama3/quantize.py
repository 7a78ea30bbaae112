"""INT4 groupwise quantize/dequantize for the Llama-3 KV cache (HIP, gfx950).

Mirrors ``kernels/llama3/quantize.py`` of the reference: same names, signatures,
``ValueError`` contracts and bit-exact results of its CPU path
``_quantize_int4_torch`` (:126-148) / ``_dequantize_int4_torch`` (:210-234).

Shapes:
    x:      [..., d]                          bf16 / fp16 / fp32 (GPU)
    packed: [..., ceil(d/G) * ceil(G/2)]      uint8
    scales: [..., ceil(d/G)]                  same dtype as x

Symmetric INT4: scale = max|x_g| / 7 (1 for an all-zero group), code =
round_half_even(x / scale) clamped to [-8, 7] and stored with a +8 bias.
"""

from __future__ import annotations

import torch

from .. import ops

_SUPPORTED_FLOATS = (torch.bfloat16, torch.float16, torch.float32)


def _validate_group_size(group_size: int) -> None:
    if group_size <= 0:
        raise ValueError("group_size must be > 0")


def quantize_int4(x: torch.Tensor, group_size: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize the last dim to symmetric INT4 with per-group scales.

    Returns ``(packed_uint8, scales)``; ``scales`` keeps the dtype of ``x``.
    Reference: kernels/llama3/quantize.py:189-207.
    """
    _validate_group_size(group_size)
    if x.dtype not in _SUPPORTED_FLOATS:
        raise ValueError("quantize_int4 expects bf16/fp16/fp32 input")
    if x.dim() < 1:
        raise ValueError("quantize_int4 expects at least 1D input")
    return ops.quantize(x, group_size, scale_dtype=x.dtype)


def dequantize_int4(
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int = 32,
    d_head: int | None = None,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Dequantize a packed INT4 tensor back to ``out_dtype`` (default: scales dtype).

    Reference: kernels/llama3/quantize.py:274-308.
    """
    _validate_group_size(group_size)
    if packed.dtype != torch.uint8:
        raise ValueError("packed must be uint8")
    if scales.dtype not in _SUPPORTED_FLOATS:
        raise ValueError("scales must be bf16/fp16/fp32")
    if packed.shape[:-1] != scales.shape[:-1]:
        raise ValueError("packed/scales leading dimensions must match")
    if packed.device != scales.device:
        raise ValueError("packed and scales must be on the same device")
    if out_dtype is None:
        out_dtype = scales.dtype
    if out_dtype not in _SUPPORTED_FLOATS:
        raise ValueError("out_dtype must be bf16/fp16/fp32")
    n_groups = scales.shape[-1]
    target_d = n_groups * group_size if d_head is None else int(d_head)
    if target_d <= 0:
        raise ValueError("d_head must be > 0 when provided")
    return ops.dequantize(packed, scales, group_size, target_d, out_dtype)
