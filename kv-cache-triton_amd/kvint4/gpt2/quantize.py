"""INT4 KV quantization helpers for GPT-2 (HIP, gfx950).

Mirrors ``kernels/gpt2/quantize.py`` of the reference: identical codes to the
Llama quantizer, but scales are always stored as fp16 (:61, :133) and
``dequantize_int4`` always returns fp16 (:235, :271). Bit-exact to the
reference's CPU path ``_quantize_int4_torch`` (:111-133) /
``_dequantize_int4_torch`` (:217-235).
"""

from __future__ import annotations

import torch

from .. import ops

_SUPPORTED_FLOATS = (torch.float16, torch.float32, torch.bfloat16)


def _validate_group_size(group_size: int) -> None:
    if group_size <= 0:
        raise ValueError("group_size must be > 0")


def quantize_int4(x: torch.Tensor, group_size: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize last dimension to symmetric INT4 with per-group fp16 scales."""
    _validate_group_size(group_size)
    if x.dtype not in _SUPPORTED_FLOATS:
        raise ValueError("quantize_int4 expects float16/float32/bfloat16 input")
    if x.dim() < 1:
        raise ValueError("quantize_int4 expects at least 1D input")
    return ops.quantize(x, group_size, scale_dtype=torch.float16)


def dequantize_int4(
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int = 32,
    d_head: int | None = None,
) -> torch.Tensor:
    """Dequantize uint8-packed INT4 tensor back to float16."""
    _validate_group_size(group_size)
    if packed.dtype != torch.uint8:
        raise ValueError("packed must be uint8")
    if scales.dtype not in _SUPPORTED_FLOATS:
        raise ValueError("scales must be float16/float32/bfloat16")
    if packed.shape[:-1] != scales.shape[:-1]:
        raise ValueError("packed/scales leading dimensions must match")
    if packed.device != scales.device:
        raise ValueError("packed and scales must be on the same device")
    n_groups = scales.shape[-1]
    target_d = n_groups * group_size if d_head is None else int(d_head)
    if target_d <= 0:
        raise ValueError("d_head must be > 0 when provided")
    return ops.dequantize(packed, scales, group_size, target_d, torch.float16)
