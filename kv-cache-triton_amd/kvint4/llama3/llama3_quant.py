"""Llama-3 attention with the INT4 KV cache and the fused HIP decode kernel.

Drop-in for ``models/llama3/llama3_quant.py`` (:36-204):

    hidden_states -> q_proj / k_proj / v_proj -> [B, n, S, d] -> RoPE(q, k)
    if past_key_values is a kvint4 QuantizedKVCache:
        decode token, no mask -> cache.append_and_attend: one HIP launch
                    quantizes the new K/V into the cache and attends over it
        otherwise: cache.append(k, v)  (HIP quantize, written in place)
        no mask  -> attention over the packed cache (attention_forward_quant_gqa
                    or, for a paged cache, its attend): query blocks of up to a few
                    rows per KV head take the fused split-K kernel, prompts and
                    long chunks the matrix-core prefill kernel
        mask     -> dequantize the cache, HF attention interface with the mask
    else: the stock path (cache.update + HF attention interface)
    -> o_proj

Written against transformers 5.x ``LlamaAttention.forward(hidden_states,
position_embeddings, attention_mask, past_key_values, **kwargs)``; the
reference's extra ``cache_position`` argument is accepted and ignored.
Differences: the fused path passes the module's own ``scaling`` and, for
ragged caches, the per-sequence lengths; CPU tensors are not supported by the
quantized path (there is no CPU implementation).
"""

from __future__ import annotations

from typing import Callable, Optional

import torch
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
from transformers.models.llama.modeling_llama import (
    LlamaAttention,
    apply_rotary_pos_emb,
    eager_attention_forward,
)

from .attention_quant import attention_forward_quant_gqa
from ..module_swap import swap_attention_modules
from ..paged_cache import PagedQuantizedKVCache
from .kv_cache import QuantizedKVCache


class LlamaAttentionQuantized(LlamaAttention):
    """LlamaAttention subclass that routes to the fused INT4 kernel when a
    ``QuantizedKVCache`` is in use."""

    def __init__(self, config, layer_idx: int, group_size: int = 32):
        super().__init__(config=config, layer_idx=layer_idx)
        self.quant_group_size = int(group_size)

    def forward(
        self,
        hidden_states: torch.Tensor,
        position_embeddings: Optional[tuple[torch.Tensor, torch.Tensor]] = None,
        attention_mask: Optional[torch.Tensor] = None,
        past_key_values=None,
        cache_position: Optional[torch.LongTensor] = None,
        **kwargs,
    ) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)

        query_states = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        key_states = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)

        cos, sin = position_embeddings
        query_states, key_states = apply_rotary_pos_emb(query_states, key_states, cos, sin)

        if isinstance(past_key_values, (QuantizedKVCache, PagedQuantizedKVCache)):
            cache = past_key_values
            if attention_mask is None and query_states.shape[-2] == 1:
                # decode: append + attention in one launch
                attn_output = cache.append_and_attend(
                    query_states, key_states, value_states, self.layer_idx,
                    n_kv_heads=self.config.num_key_value_heads, scale=self.scaling,
                )
                if attn_output is not None:
                    attn_output = attn_output.transpose(1, 2).reshape(*input_shape, -1).contiguous()
                    return self.o_proj(attn_output), None
            cache.append(key_states, value_states, self.layer_idx)
            if attention_mask is None and isinstance(cache, PagedQuantizedKVCache):
                attn_output = cache.attend(
                    query_states, self.layer_idx, n_kv_heads=self.config.num_key_value_heads,
                    scale=self.scaling, is_causal=query_states.shape[-2] > 1,
                )
                attn_output = attn_output.transpose(1, 2).reshape(*input_shape, -1).contiguous()
                return self.o_proj(attn_output), None
            if attention_mask is None:
                k_packed, k_scales, v_packed, v_scales = cache.get_quantized(self.layer_idx)
                attn_output = attention_forward_quant_gqa(
                    query_states,
                    k_packed,
                    k_scales,
                    v_packed,
                    v_scales,
                    n_q_heads=self.config.num_attention_heads,
                    n_kv_heads=self.config.num_key_value_heads,
                    group_size=self.quant_group_size,
                    is_causal=query_states.shape[-2] > 1,
                    scale=self.scaling,
                    seq_lens=cache.get_seq_lens(self.layer_idx),
                )
                attn_output = attn_output.transpose(1, 2).reshape(*input_shape, -1).contiguous()
                return self.o_proj(attn_output), None
            k_full, v_full = cache.get_dequantized(self.layer_idx, out_dtype=query_states.dtype)
            return self._fallback_attention(
                query_states, k_full, v_full, attention_mask=attention_mask,
                input_shape=input_shape, **kwargs,
            )

        if past_key_values is not None:
            key_states, value_states = past_key_values.update(key_states, value_states, self.layer_idx)
        return self._fallback_attention(
            query_states, key_states, value_states, attention_mask=attention_mask,
            input_shape=input_shape, **kwargs,
        )

    def _fallback_attention(
        self,
        query_states: torch.Tensor,
        key_states: torch.Tensor,
        value_states: torch.Tensor,
        *,
        attention_mask: Optional[torch.Tensor],
        input_shape: tuple[int, ...],
        **kwargs,
    ) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
        attention_interface: Callable = ALL_ATTENTION_FUNCTIONS.get_interface(
            self.config._attn_implementation, eager_attention_forward
        )
        attn_output, attn_weights = attention_interface(
            self,
            query_states,
            key_states,
            value_states,
            attention_mask,
            dropout=0.0 if not self.training else self.attention_dropout,
            scaling=self.scaling,
            **kwargs,
        )
        attn_output = attn_output.reshape(*input_shape, -1).contiguous()
        return self.o_proj(attn_output), attn_weights


def replace_llama_attention_with_quantized(model: torch.nn.Module, group_size: int = 32) -> None:
    """In place: swap each Llama decoder layer's self-attention for the
    quantized variant, reusing the projection Parameters (no copies) and moving
    any accelerate hooks. Calling it again only updates the group size
    (reference: models/llama3/llama3_quant.py:171-204)."""
    layers = getattr(getattr(model, "model", None), "layers", None)
    if layers is None:
        raise ValueError("expected a Llama CausalLM model with .model.layers")
    swap_attention_modules(
        layers, "self_attn", LlamaAttentionQuantized,
        lambda old: LlamaAttentionQuantized(old.config, layer_idx=old.layer_idx, group_size=group_size),
        group_size,
    )
