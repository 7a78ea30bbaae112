"""GPT-2 attention with the INT4 KV cache and the fused HIP decode kernel.

Drop-in for ``models/gpt2/gpt2_quant.py`` (:16-157), written against
transformers 5.x ``GPT2Attention.forward``. Self-attention with a kvint4
``QuantizedKVCache`` appends through the HIP quantizer and attends over the
packed cache:
  * decode token, no mask, 16-bit activations -> ``append_and_attend``: one
    HIP launch quantizes the new K/V into the cache and attends over it;
  * no mask -> ``attention_forward_quant`` over the packed cache (short query
    blocks: fused split-K kernel; prompts: matrix-core prefill kernel), scaled
    by the module's ``scaling``;
  * mask present -> dequantized cache through the HF attention interface.
The reference takes the fused path at q_len == 1 even when a padding mask is
present (:93-99), which ignores the padding; here a mask always takes the
masked path. Cross-attention and other caches use the stock logic.
"""

from __future__ import annotations

from typing import Callable, Optional

import torch
from transformers.cache_utils import EncoderDecoderCache
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
from transformers.models.gpt2.modeling_gpt2 import GPT2Attention, eager_attention_forward

from .attention_quant import attention_forward_quant
from ..module_swap import swap_attention_modules
from ..paged_cache import PagedQuantizedKVCache
from .kv_cache import QuantizedKVCache


class GPT2AttentionQuantized(GPT2Attention):
    """GPT2Attention with quantized KV cache support."""

    def __init__(self, config, is_cross_attention: bool = False, layer_idx: int | None = None, group_size: int = 32):
        super().__init__(config, is_cross_attention=is_cross_attention, layer_idx=layer_idx)
        self.quant_group_size = int(group_size)

    def forward(
        self,
        hidden_states: Optional[torch.Tensor],
        past_key_values=None,
        attention_mask: Optional[torch.Tensor] = None,
        encoder_hidden_states: Optional[torch.Tensor] = None,
        encoder_attention_mask: Optional[torch.Tensor] = None,
        output_attentions: Optional[bool] = False,
        cache_position: Optional[torch.LongTensor] = None,
        **kwargs,
    ):
        is_cross_attention = encoder_hidden_states is not None
        quant_types = (QuantizedKVCache, PagedQuantizedKVCache)
        quant_cache = past_key_values if isinstance(past_key_values, quant_types) else None
        if quant_cache is None or is_cross_attention:
            return super().forward(
                hidden_states,
                past_key_values=None if isinstance(past_key_values, quant_types) else past_key_values,
                attention_mask=attention_mask,
                encoder_hidden_states=encoder_hidden_states,
                encoder_attention_mask=encoder_attention_mask,
                output_attentions=output_attentions,
                **kwargs,
            )

        query_states, key_states, value_states = self.c_attn(hidden_states).split(self.split_size, dim=2)
        shape_kv = (*key_states.shape[:-1], -1, self.head_dim)
        key_states = key_states.view(shape_kv).transpose(1, 2)
        value_states = value_states.view(shape_kv).transpose(1, 2)
        shape_q = (*query_states.shape[:-1], -1, self.head_dim)
        query_states = query_states.view(shape_q).transpose(1, 2)

        using_eager = self.config._attn_implementation == "eager"
        fused_out = None
        if attention_mask is None and query_states.shape[-2] == 1 and not (using_eager and self.reorder_and_upcast_attn):
            # decode token: append + attention in one launch (16-bit models)
            fused_out = quant_cache.append_and_attend(
                query_states, key_states, value_states, self.layer_idx,
                n_kv_heads=query_states.shape[1], scale=self.scaling,
            )
        if fused_out is None:
            quant_cache.append(key_states, value_states, self.layer_idx)

        if fused_out is not None:
            attn_output = fused_out.transpose(1, 2)
            attn_weights = None
        elif using_eager and self.reorder_and_upcast_attn:
            k_full, v_full = quant_cache.get_dequantized(self.layer_idx)
            attn_output, attn_weights = self._upcast_and_reordered_attn(
                query_states, k_full.to(query_states.dtype), v_full.to(query_states.dtype), attention_mask
            )
        elif attention_mask is None and isinstance(quant_cache, PagedQuantizedKVCache):
            attn_output = quant_cache.attend(
                query_states, self.layer_idx, n_kv_heads=query_states.shape[1], scale=self.scaling,
                is_causal=query_states.shape[-2] > 1,
            ).transpose(1, 2)
            attn_weights = None
        elif attention_mask is None:
            k_packed, k_scales, v_packed, v_scales = quant_cache.get_quantized(self.layer_idx)
            q_in = query_states if query_states.dtype in (torch.float16, torch.float32) else query_states.float()
            attn_output = attention_forward_quant(
                q_in,
                k_packed,
                k_scales,
                v_packed,
                v_scales,
                group_size=self.quant_group_size,
                is_causal=query_states.shape[-2] > 1,
                scale=self.scaling,
                seq_lens=quant_cache.get_seq_lens(self.layer_idx),
            ).to(query_states.dtype)
            attn_output = attn_output.transpose(1, 2)
            attn_weights = None
        else:
            k_full, v_full = quant_cache.get_dequantized(self.layer_idx)
            attention_interface: Callable = ALL_ATTENTION_FUNCTIONS.get_interface(
                self.config._attn_implementation, eager_attention_forward
            )
            attn_output, attn_weights = attention_interface(
                self,
                query_states,
                k_full.to(query_states.dtype),
                v_full.to(query_states.dtype),
                attention_mask,
                dropout=self.attn_dropout.p if self.training else 0.0,
                scaling=self.scaling,
                **kwargs,
            )

        attn_output = attn_output.reshape(*attn_output.shape[:-2], -1).contiguous()
        attn_output = self.c_proj(attn_output)
        attn_output = self.resid_dropout(attn_output)
        return attn_output, attn_weights


def replace_gpt2_attention_with_quantized(model: torch.nn.Module, group_size: int = 32) -> None:
    """In place: swap each GPT2Block self-attention for the quantized variant,
    reusing its Parameters (the reference copies a state dict instead,
    models/gpt2/gpt2_quant.py:141-157). Calling it again only updates the group
    size."""
    blocks = getattr(getattr(model, "transformer", None), "h", None)
    if blocks is None:
        raise ValueError("expected a GPT2 model with .transformer.h blocks")
    swap_attention_modules(
        blocks, "attn", GPT2AttentionQuantized,
        lambda old: GPT2AttentionQuantized(old.config, is_cross_attention=old.is_cross_attention,
                                           layer_idx=old.layer_idx, group_size=group_size),
        group_size,
    )
