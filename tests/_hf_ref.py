"""Stock-HF reference attentions for model-level comparisons on the GPU.

Registered with transformers' AttentionInterface:
  * "kvq_fp32_ref": the unquantized K/V of a DynamicCache, GQA-expanded,
    attended in float32 (dense SDPA, math backend) and cast back;
  * "kvq_ref_fused_prefill": the same for decode tokens; prompts go through
    the fused flash / memory-efficient SDPA kernels in the model's dtype;
  * "kvq_ref_int4_dense": as the previous, over K/V passed through INT4
    quantize -> dequantize (the reference's INT4 semantics in dense form).
Running the stock model with them keeps half-precision batched GEMMs off the
GPU while every other kernel of the model is the same as in the quantized
run, so a comparison isolates the INT4 KV (or, against the INT4 dense
reference, the INT4 path's implementation).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel
from transformers import AttentionInterface

NAME = "kvq_fp32_ref"


def _fp32_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    rep = query.shape[1] // key.shape[1]
    q = query.float()
    k = key.float().repeat_interleave(rep, dim=1)
    v = value.float().repeat_interleave(rep, dim=1)
    Sq, Sk = q.shape[2], k.shape[2]
    mask = None
    if attention_mask is not None:
        mask = attention_mask if attention_mask.dtype == torch.bool else attention_mask.float()
    elif Sq > 1:
        i = torch.arange(Sq, device=q.device)[:, None]
        j = torch.arange(Sk, device=q.device)[None, :]
        mask = j <= (Sk - Sq + i)
    with sdpa_kernel([SDPBackend.MATH]):
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scaling)
    return out.transpose(1, 2).contiguous().to(query.dtype), None


AttentionInterface.register(NAME, _fp32_attention)

FLASH_PREFILL_NAME = "kvq_ref_fused_prefill"  # (transformers treats names containing "flash" as flash-attn kernels)


def _flash_prefill_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """Long prompts: the fused flash / memory-efficient SDPA kernels in the
    model's dtype over the dense K/V (a float32 math-path prefill would
    materialise Sq x Sk scores). Single-token decode: as _fp32_attention."""
    Sq, Sk = query.shape[2], key.shape[2]
    if Sq == 1 or query.dtype == torch.float32 or (attention_mask is None and Sq != Sk):
        return _fp32_attention(module, query, key, value, attention_mask, scaling=scaling)
    rep = query.shape[1] // key.shape[1]
    k = key.repeat_interleave(rep, dim=1)
    v = value.repeat_interleave(rep, dim=1)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        if attention_mask is None:
            out = F.scaled_dot_product_attention(query, k, v, is_causal=Sq == Sk, scale=scaling)
        else:
            out = F.scaled_dot_product_attention(query, k, v, attn_mask=attention_mask, scale=scaling)
    return out.transpose(1, 2).contiguous(), None


AttentionInterface.register(FLASH_PREFILL_NAME, _flash_prefill_attention)


INT4_DENSE_NAME = "kvq_ref_int4_dense"


def _int4_dense_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """The reference's INT4 semantics in dense form: the DynamicCache's K/V
    passed through INT4 quantize -> dequantize (group 32, scales in the K/V
    dtype; codes bit-exact with the oracle), then _flash_prefill_attention.
    Requantizing dequantized values reproduces the same codes, so the whole
    cache can be passed through on every call."""
    from kvint4 import ops

    def qdq(t):
        p, s = ops.quantize(t.contiguous(), 32, t.dtype)
        return ops.dequantize(p, s, 32, t.shape[-1], t.dtype)

    return _flash_prefill_attention(module, query, qdq(key), qdq(value), attention_mask, scaling=scaling)


AttentionInterface.register(INT4_DENSE_NAME, _int4_dense_attention)


def use_fp32_reference_attention(model) -> None:
    model.set_attn_implementation(NAME)


def use_flash_prefill_reference_attention(model) -> None:
    model.set_attn_implementation(FLASH_PREFILL_NAME)


def use_int4_dense_reference_attention(model) -> None:
    model.set_attn_implementation(INT4_DENSE_NAME)
