"""Quantized KV cache for Llama-3 decode with packed INT4 storage (HIP, gfx950).

Drop-in for ``models/llama3/kv_cache.py`` (:30-166): same class name,
constructor, methods and return values; scales are stored in the K/V dtype
(bf16 for a bf16 model). Implements the cache protocol transformers 5.x asks
of a ``past_key_values`` object (``get_seq_length``, ``get_query_offset``,
``get_mask_sizes``, ``is_sliding``, ``is_compileable``, ``update`` ...).

Differences from the reference, by design:
  * appends are in place into preallocated capacity (no per-step torch.cat);
  * ``get_quantized`` returns views ``[:, :, :seq_len]`` of that storage;
  * optional ragged batches (``load_ragged`` / ``get_seq_lens``).
"""

from __future__ import annotations

import torch

from ..cache_base import QuantizedKVCacheBase, _LayerQuantizedKV  # noqa: F401  (re-export)


class QuantizedKVCache(QuantizedKVCacheBase):
    """Per-layer INT4-packed KV cache. Compatible with HF Llama attention."""

    def _scale_dtype_for(self, x: torch.Tensor) -> torch.dtype:
        return x.dtype

    def get_mask_sizes(self, cache_position, layer_idx: int) -> tuple[int, int]:
        """(kv_length, kv_offset) for mask creation; accepts the query length
        as an int (transformers 5.x) or a cache_position tensor (4.x)."""
        past_len = self.get_seq_length(layer_idx)
        if isinstance(cache_position, torch.Tensor):
            query_length = int(cache_position.item()) if cache_position.dim() == 0 else int(cache_position.shape[0])
        else:
            query_length = int(cache_position)
        return past_len + query_length, 0

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return -1

    def update(
        self,
        key_states: torch.Tensor,
        value_states: torch.Tensor,
        layer_idx: int,
        cache_kwargs: dict | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Quantize and append K/V, then return the full dequantized cache.

        Used only by stock (unswapped) attention modules; the swapped module
        reads the packed tensors through ``get_quantized``.
        """
        del cache_kwargs
        self._append_quantized(key_states, value_states, layer_idx)
        return self.get_dequantized(layer_idx, out_dtype=key_states.dtype)

    def get_dequantized(
        self,
        layer_idx: int,
        out_dtype: torch.dtype = torch.bfloat16,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        return self._dequantized(layer_idx, out_dtype)
