"""Storage engine shared by the Llama-3 and GPT-2 ``QuantizedKVCache`` classes.

The reference appends by ``torch.cat`` of the whole layer cache on every step
(``models/llama3/kv_cache.py:96-101``), moving O(S) bytes per token. Here each
layer owns preallocated capacity buffers

    k_packed, v_packed : [B, H_kv, capacity, packed_width]   uint8
    k_scales, v_scales : [B, H_kv, capacity, n_groups]       scale dtype

and new tokens are quantized by the HIP kernel straight into rows
[seq_len, seq_len + S). Capacity grows geometrically (one copy per doubling).
``get_quantized`` returns ``[:, :, :seq_len]`` views: same shapes and values as
the reference's tensors, no copy.

Ragged batches (per-sequence lengths, not in the reference) are supported by
``load_ragged`` + ``append``: sequence b's new rows go to positions
seq_lens[b] + s (a device int32 tensor updated in place), and the attention
kernel masks keys past each sequence's length.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _native, ops

_ROUND = 256  # capacity granularity (tokens)


@dataclass
class _LayerQuantizedKV:
    """Per-layer state. Field names follow the reference
    (models/llama3/kv_cache.py:21-27); the tensors may hold more rows than
    ``seq_len`` (capacity). ``seq_lens`` (device lengths) is set for ragged
    layers and after ``make_static``."""

    k_packed: torch.Tensor
    k_scales: torch.Tensor
    v_packed: torch.Tensor
    v_scales: torch.Tensor
    seq_len: int
    seq_lens: Optional[torch.Tensor] = None

    @property
    def capacity(self) -> int:
        return int(self.k_packed.shape[2])


def _round_up(n: int, m: int) -> int:
    return (n + m - 1) // m * m


class QuantizedKVCacheBase:
    """Family-independent part of the INT4 cache. Subclasses set
    ``_scale_dtype_for(x)`` and ``_deq_dtype_default``."""

    def __init__(self, group_size: int = 32, reserve_tokens: int = 0):
        if group_size <= 0:
            raise ValueError("group_size must be > 0")
        self.group_size = int(group_size)
        self.reserve_tokens = int(reserve_tokens)
        self._layers: dict[int, _LayerQuantizedKV] = {}
        self.fused_steps = 0  # append_and_attend calls served by the one-launch decode step

    # -- family policy -------------------------------------------------------
    def _scale_dtype_for(self, x: torch.Tensor) -> torch.dtype:  # pragma: no cover
        raise NotImplementedError

    # -- HF cache protocol ---------------------------------------------------
    def get_seq_length(self, layer_idx: int = 0) -> int:
        layer = self._layers.get(layer_idx)
        return 0 if layer is None else int(layer.seq_len)

    def get_query_offset(self, layer_idx: int = 0) -> int:
        """transformers>=5 masking: first position of the incoming queries."""
        return self.get_seq_length(layer_idx)

    @property
    def is_initialized(self) -> bool:
        return len(self._layers) > 0

    @property
    def is_sliding(self) -> list[bool]:
        return [False for _ in self._layers]

    is_compileable = False

    def __len__(self) -> int:
        return len(self._layers)

    def reset(self) -> None:
        self._layers.clear()

    def has_layer(self, layer_idx: int) -> bool:
        return layer_idx in self._layers

    # -- storage -------------------------------------------------------------
    def _alloc(self, like: torch.Tensor, B: int, H: int, cap: int, D: int, scale_dtype: torch.dtype):
        w = ops.packed_width(D, self.group_size)
        ng = ops.num_groups(D, self.group_size)
        dev = like.device
        return (
            torch.empty((B, H, cap, w), dtype=torch.uint8, device=dev),
            torch.empty((B, H, cap, ng), dtype=scale_dtype, device=dev),
            torch.empty((B, H, cap, w), dtype=torch.uint8, device=dev),
            torch.empty((B, H, cap, ng), dtype=scale_dtype, device=dev),
        )

    def _ensure_layer(self, key_states: torch.Tensor, layer_idx: int, needed: int) -> _LayerQuantizedKV:
        B, H, _, D = key_states.shape
        scale_dtype = self._scale_dtype_for(key_states)
        layer = self._layers.get(layer_idx)
        if layer is None:
            cap = _round_up(max(needed + max(_ROUND, needed // 8), self.reserve_tokens), _ROUND)
            kp, ks, vp, vs = self._alloc(key_states, B, H, cap, D, scale_dtype)
            layer = _LayerQuantizedKV(kp, ks, vp, vs, 0)
            self._layers[layer_idx] = layer
            return layer
        if layer.k_packed.shape[:2] != (B, H) or layer.k_packed.shape[-1] != ops.packed_width(D, self.group_size):
            raise ValueError(
                f"layer {layer_idx}: new K/V shape {tuple(key_states.shape)} does not match the cache "
                f"(B={layer.k_packed.shape[0]}, H={layer.k_packed.shape[1]})"
            )
        if layer.k_scales.dtype != scale_dtype:
            raise ValueError(f"layer {layer_idx}: scale dtype {scale_dtype} differs from the cache's")
        if needed > layer.capacity:
            self._grow(layer, _round_up(max(needed, 2 * layer.capacity), _ROUND))
        return layer

    @staticmethod
    def _grow(layer: _LayerQuantizedKV, cap: int) -> None:
        """Move a layer's rows into buffers of `cap` rows (one copy)."""
        n = layer.seq_len
        new = [torch.empty((*t.shape[:2], cap, t.shape[3]), dtype=t.dtype, device=t.device)
               for t in (layer.k_packed, layer.k_scales, layer.v_packed, layer.v_scales)]
        for dst, src in zip(new, (layer.k_packed, layer.k_scales, layer.v_packed, layer.v_scales)):
            dst[:, :, :n].copy_(src[:, :, :n])
        layer.k_packed, layer.k_scales, layer.v_packed, layer.v_scales = new

    def make_static(self, extra_tokens: int) -> None:
        """Prepare every layer for decode steps captured in a HIP graph.

        A replay cannot allocate, and it must not bake a Python write position
        into its launches. So room for `extra_tokens` more tokens per sequence
        is reserved now, and each layer's lengths move to a device int32 [B]
        tensor (if not there already, as for ragged layers). ``append`` and
        ``append_and_attend`` then read the write position from that tensor and
        advance it in place, which a captured step replays.

        The Python-side lengths (``get_seq_length``) are not touched by a replay.
        Whoever replays advances them with ``advance_host_lengths``."""
        extra_tokens = int(extra_tokens)
        if extra_tokens < 0:
            raise ValueError("extra_tokens must be >= 0")
        if not self._layers:
            raise ValueError("make_static needs a prefilled cache (no layer holds tokens)")
        for layer in self._layers.values():
            need = layer.seq_len + extra_tokens
            if need > layer.capacity:
                self._grow(layer, _round_up(need, _ROUND))
            if layer.seq_lens is None:
                B = int(layer.k_packed.shape[0])
                layer.seq_lens = torch.full((B,), layer.seq_len, dtype=torch.int32, device=layer.k_packed.device)

    def buffer_signature(self) -> tuple:
        """Device addresses of every layer's buffers and device lengths. A HIP
        graph captured over this cache holds these addresses; an edit that
        replaces a buffer (growth, reorder, batch select, load) changes the
        signature."""
        return tuple(
            (i, l.k_packed.data_ptr(), l.k_scales.data_ptr(), l.v_packed.data_ptr(), l.v_scales.data_ptr(),
             None if l.seq_lens is None else l.seq_lens.data_ptr())
            for i, l in sorted(self._layers.items())
        )

    def room(self) -> int:
        """Tokens every layer can still take without growing its buffers."""
        return min((l.capacity - l.seq_len for l in self._layers.values()), default=0)

    def host_lengths(self) -> dict[int, int]:
        """Python-side length of every layer (what ``get_seq_length`` reports)."""
        return {i: int(l.seq_len) for i, l in self._layers.items()}

    def advance_host_lengths(self, base: dict[int, int], n: int) -> None:
        """Set each layer's Python-side length to base[layer] + n: the
        bookkeeping of n decode steps that ran as graph replays (the device
        lengths were advanced by the replays themselves)."""
        for i, l in self._layers.items():
            l.seq_len = int(base[i]) + int(n)

    def _append_quantized(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int) -> None:
        if key_states.shape != value_states.shape:
            raise ValueError("key_states and value_states must have the same shape")
        if key_states.dim() != 4:
            raise ValueError("key/value states must be [B, H_kv, S, d_head]")
        S = int(key_states.shape[2])
        prev = self._layers.get(layer_idx)
        start = 0 if prev is None else prev.seq_len
        layer = self._ensure_layer(key_states, layer_idx, start + S)
        pos = layer.seq_lens if layer.seq_lens is not None else start
        ops.quantize_into(key_states, layer.k_packed, layer.k_scales, self.group_size, pos)
        ops.quantize_into(value_states, layer.v_packed, layer.v_scales, self.group_size, pos)
        if layer.seq_lens is not None:
            layer.seq_lens.add_(S)
        layer.seq_len = start + S

    def append(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int) -> None:
        """Quantize [B, H_kv, S, d] K/V and append them to layer `layer_idx`."""
        self._append_quantized(key_states, value_states, layer_idx)

    def append_and_attend(
        self,
        query_states: torch.Tensor,
        key_states: torch.Tensor,
        value_states: torch.Tensor,
        layer_idx: int,
        *,
        n_kv_heads: int,
        scale: float,
    ) -> Optional[torch.Tensor]:
        """Decode fast path: one kernel launch quantizes the new token's K/V
        [B, H_kv, 1, d] into the layer's buffers (in place) and attends
        query_states [B, H_q, 1, d] over the cache including it; the same
        result as ``append`` followed by fused attention over
        ``get_quantized``. Returns None, with the cache untouched, when the
        fused step does not apply (not one decode token, an empty layer, or a
        dtype / group size it does not handle); the caller then appends and
        attends separately."""
        if query_states.shape[2] != 1 or key_states.shape[2] != 1 or not query_states.is_cuda:
            return None
        if key_states.shape != value_states.shape or key_states.dim() != 4:
            return None
        prev = self._layers.get(layer_idx)
        if prev is None or prev.seq_len == 0:
            return None
        start = prev.seq_len
        layer = self._ensure_layer(key_states, layer_idx, start + 1)
        pos = layer.seq_lens if layer.seq_lens is not None else start
        try:
            out = ops.decode_step(
                query_states, key_states, value_states,
                layer.k_packed, layer.k_scales, layer.v_packed, layer.v_scales, pos,
                n_kv_heads=n_kv_heads, group_size=self.group_size, sm_scale=scale,
            )
        except _native.KVQUnsupported:
            return None
        if layer.seq_lens is not None:
            layer.seq_lens.add_(1)
        layer.seq_len = start + 1
        self.fused_steps += 1
        return out

    def load_ragged(
        self,
        key_states: torch.Tensor,
        value_states: torch.Tensor,
        layer_idx: int,
        lengths: torch.Tensor,
    ) -> None:
        """Start a ragged layer from padded K/V [B, H_kv, S_max, d] whose
        sequence b holds `lengths[b]` valid rows. Later `append` calls write
        each sequence's new rows right after its own last row."""
        if layer_idx in self._layers:
            raise ValueError(f"layer {layer_idx} already holds state")
        if lengths.numel() != key_states.shape[0]:
            raise ValueError("lengths must have one entry per batch row")
        self._append_quantized(key_states, value_states, layer_idx)
        layer = self._layers[layer_idx]
        layer.seq_lens = lengths.to(device=key_states.device, dtype=torch.int32).clone()

    def get_seq_lens(self, layer_idx: int) -> Optional[torch.Tensor]:
        """Per-sequence lengths of a ragged layer (device int32 [B]) or None."""
        layer = self._layers.get(layer_idx)
        return None if layer is None else layer.seq_lens

    def get_quantized(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        layer = self._layers.get(layer_idx)
        if layer is None:
            raise KeyError(f"no cache state for layer {layer_idx}")
        n = layer.seq_len
        return (layer.k_packed[:, :, :n], layer.k_scales[:, :, :n],
                layer.v_packed[:, :, :n], layer.v_scales[:, :, :n])

    def _dequantized(self, layer_idx: int, out_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        kp, ks, vp, vs = self.get_quantized(layer_idx)
        d_head = ks.shape[-1] * self.group_size
        k = ops.dequantize(kp, ks, self.group_size, d_head, out_dtype)
        v = ops.dequantize(vp, vs, self.group_size, d_head, out_dtype)
        return k, v

    # -- batch and length edits (generate(): beam search, assisted decoding) --
    def _gather_batch(self, index: torch.Tensor) -> None:
        """Every layer keeps the batch rows `index` (int64), in that order:
        new sequence b is old sequence index[b]. Each layer's stored rows are
        copied into fresh capacity buffers."""
        for layer in self._layers.values():
            n = layer.seq_len
            idx = index.to(layer.k_packed.device)
            bufs = []
            for t in (layer.k_packed, layer.k_scales, layer.v_packed, layer.v_scales):
                new = torch.empty((idx.numel(),) + tuple(t.shape[1:]), dtype=t.dtype, device=t.device)
                new[:, :, :n] = t[idx, :, :n]
                bufs.append(new)
            layer.k_packed, layer.k_scales, layer.v_packed, layer.v_scales = bufs
            if layer.seq_lens is not None:
                layer.seq_lens = layer.seq_lens[idx].contiguous()

    def _batch_size(self) -> int:
        return int(next(iter(self._layers.values())).k_packed.shape[0]) if self._layers else 0

    def reorder_cache(self, beam_idx: torch.Tensor) -> None:
        """Beam search (HF ``Cache.reorder_cache``): sequence b becomes the old
        sequence beam_idx[b]."""
        self._gather_batch(beam_idx.long())

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        """Keep only the batch rows `indices` (int indices or a bool mask)."""
        idx = indices.nonzero().flatten() if indices.dtype == torch.bool else indices.long()
        self._gather_batch(idx)

    def batch_repeat_interleave(self, repeats: int) -> None:
        """Repeat every sequence `repeats` times along the batch."""
        self._gather_batch(torch.arange(self._batch_size()).repeat_interleave(int(repeats)))

    def activate_past_recording(self) -> None:
        """HF assisted decoding calls this before drafting. Every stored token
        is kept until ``crop``, so there is nothing to switch on."""

    def get_max_length(self, layer_idx: int = 0) -> int:
        """transformers 5.15 name of ``get_max_cache_shape``: -1, no maximum."""
        return -1

    def crop(self, max_length: int) -> None:
        """Drop tokens from the end of every layer (HF ``Cache.crop``):
        max_length < 0 removes -max_length tokens; max_length > 0 keeps the
        first max_length (nothing if that is not shorter); 0 does nothing. A
        ragged layer cuts every sequence by the same rule."""
        max_length = int(max_length)
        if max_length == 0:
            return
        for layer in self._layers.values():
            n = layer.seq_len
            keep = max(n + max_length, 0) if max_length < 0 else min(max_length, n)
            if keep == n:
                continue
            if layer.seq_lens is not None:
                if max_length < 0:
                    layer.seq_lens.add_(max_length).clamp_(min=0)
                else:
                    layer.seq_lens.clamp_(max=keep)
            layer.seq_len = keep

    def nbytes(self) -> int:
        """Bytes of packed codes + scales for the stored tokens of all layers
        (same accounting as the reference, models/llama3/kv_cache.py:158-166)."""
        total = 0
        for idx in self._layers:
            for t in self.get_quantized(idx):
                total += t.element_size() * t.numel()
        return total

    def capacity_nbytes(self) -> int:
        """Bytes actually reserved on the device (capacity buffers)."""
        total = 0
        for layer in self._layers.values():
            for t in (layer.k_packed, layer.k_scales, layer.v_packed, layer.v_scales):
                total += t.element_size() * t.numel()
        return total
