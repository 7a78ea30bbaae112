"""Quantized KV cache for GPT-2 decode with packed INT4 storage (HIP, gfx950).

Drop-in for ``models/gpt2/kv_cache.py`` (:21-112): scales always fp16 and
``get_dequantized`` always returns fp16, as in the reference. Storage, in-place
appends, ragged support and the transformers 5.x protocol come from
``kvint4.cache_base``.
"""

from __future__ import annotations

import torch

from ..cache_base import QuantizedKVCacheBase, _LayerQuantizedKV  # noqa: F401  (re-export)


class QuantizedKVCache(QuantizedKVCacheBase):
    """Minimal cache object compatible with GPT-2 cache usage."""

    def _scale_dtype_for(self, x: torch.Tensor) -> torch.dtype:
        return torch.float16

    def get_mask_sizes(self, cache_position, layer_idx: int = 0) -> tuple[int, int]:
        """(kv_length, kv_offset). The reference reads ``cache_position.shape[0]``
        (models/gpt2/kv_cache.py:34-37); transformers 5.x passes the query
        length as an int, which is accepted too."""
        past_len = self.get_seq_length(layer_idx)
        if isinstance(cache_position, torch.Tensor):
            query_length = int(cache_position.item()) if cache_position.dim() == 0 else int(cache_position.shape[0])
        else:
            query_length = int(cache_position)
        return past_len + query_length, 0

    def get_max_cache_shape(self, layer_idx: int = 0) -> int | None:
        return None

    def update(
        self,
        key_states: torch.Tensor,
        value_states: torch.Tensor,
        layer_idx: int,
        cache_kwargs: dict | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Quantize and append K/V, then return the dequantized full cache (fp16)."""
        del cache_kwargs
        self._append_quantized(key_states, value_states, layer_idx)
        return self.get_dequantized(layer_idx)

    def get_dequantized(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self._dequantized(layer_idx, torch.float16)
