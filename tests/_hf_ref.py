"""A stock-HF reference attention for model-level comparisons on the GPU.

Registered with transformers' AttentionInterface as "kvq_fp32_ref": the
unquantized K/V of a DynamicCache, GQA-expanded, attended in float32
(dense SDPA, math backend) and cast back. Running the stock model with it keeps
half-precision batched GEMMs off the GPU while every other kernel of the model
is the same as in the quantized run, so the comparison isolates the INT4 KV.
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


def use_fp32_reference_attention(model) -> None:
    model.set_attn_implementation(NAME)
