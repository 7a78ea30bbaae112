"""Paged INT4 KV cache: a block pool per layer, one block table for the batch.

The reference keeps each layer's packed K/V as one contiguous tensor grown by
``torch.cat`` (``models/llama3/kv_cache.py:76-105``) and has no paged layout.
Here a layer's rows live in pools

    k_pool, v_pool        [H_kv, num_blocks * page_size, packed_width]   uint8
    k_scales, v_scales    [H_kv, num_blocks * page_size, n_groups]       scale dtype

and sequence b's token t is pool row ``table[b, t // page_size] * page_size +
t % page_size``. The block table (device int32 ``[B, cols]``, -1 = no block)
is shared by all layers: every layer appends the same tokens, so a block id
names the same positions in each layer's pool. Blocks are taken from a free
list as sequences grow; the pools grow by doubling (block ids stay valid), and
``free_sequence`` returns a finished sequence's blocks for reuse by another.

Blocks are reference-counted so that sequences can share them: beam search's
``reorder_cache`` (and ``batch_select_indices`` / ``batch_repeat_interleave``)
hands a parent's blocks to each of its children without copying, and the
first write into a shared block copies that one block (every layer's rows)
to a fresh one (copy on write). ``crop`` shortens sequences for assisted
decoding and releases blocks past the new ends.

Every sequence has its own length (ragged batches are the normal case). The
HIP kernels read and write through the table: ``quantize_into_paged`` for
appends, ``decode_step_paged`` for a decode token (append + attention in one
launch), ``fused_decode_attention_paged`` for short query blocks and
``dequantize_paged`` (+ dense SDPA) for long ones.

The class keeps the HF cache protocol of ``QuantizedKVCache`` (transformers
5.x) so it can be passed as ``past_key_values`` to a model whose attention was
swapped by ``replace_llama_attention_with_quantized``.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _native, ops


class PagedQuantizedKVCache:
    """INT4 KV cache in fixed-size pages.

    group_size: quantization group along d_head (as QuantizedKVCache).
    page_size:  rows per page, a power of two (>= 64 for the attention kernels).
    num_blocks: initial pool size in blocks per layer (grown on demand).
    scale_dtype: scale storage dtype; None = the K/V dtype (Llama policy).
    """

    def __init__(self, group_size: int = 32, page_size: int = 64, num_blocks: int = 0,
                 scale_dtype: Optional[torch.dtype] = None):
        if group_size <= 0:
            raise ValueError("group_size must be > 0")
        if page_size < 1 or page_size & (page_size - 1):
            raise ValueError("page_size must be a power of two")
        self.group_size = int(group_size)
        self.page_size = int(page_size)
        self._init_blocks = max(int(num_blocks), 0)
        self._scale_dtype = scale_dtype
        self.reset()

    # -- storage -------------------------------------------------------------
    def reset(self) -> None:
        self._pools: dict[int, list[torch.Tensor]] = {}
        self._lens: dict[int, list[int]] = {}           # host copy of each layer's lengths
        self._seq_lens: dict[int, torch.Tensor] = {}    # device int32 [B] per layer
        self._pages: list[list[int]] = []               # block ids of each sequence
        self._free: list[int] = []
        self._ref: list[int] = []                       # sequences holding each block
        self._num_blocks = 0
        self._table: Optional[torch.Tensor] = None
        self._table_dirty = False
        self._shape: Optional[tuple] = None             # (B, H, D, x dtype, scale dtype, device)
        self.fused_steps = 0  # append_and_attend calls served by the one-launch decode step

    def _setup(self, x: torch.Tensor) -> None:
        B, H, _, D = x.shape
        sd = self._scale_dtype or x.dtype
        if self._shape is None:
            self._shape = (B, H, D, x.dtype, sd, x.device)
            self._pages = [[] for _ in range(B)]
            self._grow_pool(self._init_blocks)
            return
        if self._shape[:3] != (B, H, D) or self._shape[5] != x.device:
            raise ValueError(f"K/V shape {tuple(x.shape)} does not match the cache (B={self._shape[0]}, "
                             f"H={self._shape[1]}, D={self._shape[2]})")

    def _alloc_pool(self, rows: int) -> list[torch.Tensor]:
        _, H, D, _, sd, dev = self._shape
        w, ng = ops.packed_width(D, self.group_size), ops.num_groups(D, self.group_size)
        return [torch.empty((H, rows, w), dtype=torch.uint8, device=dev),
                torch.empty((H, rows, ng), dtype=sd, device=dev),
                torch.empty((H, rows, w), dtype=torch.uint8, device=dev),
                torch.empty((H, rows, ng), dtype=sd, device=dev)]

    def _grow_pool(self, n_blocks: int) -> None:
        if n_blocks <= self._num_blocks:
            return
        old_rows = self._num_blocks * self.page_size
        for idx, pools in self._pools.items():
            new = self._alloc_pool(n_blocks * self.page_size)
            for dst, src in zip(new, pools):
                dst[:, :old_rows].copy_(src[:, :old_rows])
            self._pools[idx] = new
        self._free.extend(range(n_blocks - 1, self._num_blocks - 1, -1))
        self._ref.extend([0] * (n_blocks - self._num_blocks))
        self._num_blocks = n_blocks

    def _take_block(self) -> int:
        if not self._free:
            self._grow_pool(max(2 * self._num_blocks, 8))
        blk = self._free.pop()
        self._ref[blk] = 1
        return blk

    def _release(self, blk: int) -> None:
        self._ref[blk] -= 1
        if self._ref[blk] == 0:
            self._free.append(blk)

    def _make_writable(self, starts: list[int], n_new: int | list[int]) -> None:
        """Before sequence b writes positions [starts[b], starts[b] + n), give
        it its own copy of every shared block those positions fall in."""
        P = self.page_size
        for b, lo in enumerate(starts):
            n = n_new[b] if isinstance(n_new, list) else n_new
            if n <= 0:
                continue
            pages = self._pages[b]
            for i in range(lo // P, min((lo + n - 1) // P + 1, len(pages))):
                old = pages[i]
                if self._ref[old] <= 1:
                    continue
                new = self._take_block()
                src, dst = slice(old * P, (old + 1) * P), slice(new * P, (new + 1) * P)
                for pools in self._pools.values():
                    for t in pools:
                        t[:, dst] = t[:, src]
                self._release(old)
                pages[i] = new
                self._table_dirty = True

    def _ensure_pages(self, lengths: list[int]) -> None:
        """Give every sequence blocks for its first lengths[b] positions."""
        need = [-(-n // self.page_size) - len(p) for n, p in zip(lengths, self._pages)]
        short = sum(max(n, 0) for n in need) - len(self._free)
        if short > 0:
            self._grow_pool(max(2 * self._num_blocks, self._num_blocks + short, 8))
        for b, n in enumerate(need):
            for _ in range(n):
                self._pages[b].append(self._take_block())
                self._table_dirty = True
        cols = max((len(p) for p in self._pages), default=0)
        if self._table is None or self._table.shape[1] < cols:
            self._table_dirty = True

    def _page_table(self) -> ops.PageTable:
        if self._table_dirty or self._table is None:
            B = self._shape[0]
            cols = max(max((len(p) for p in self._pages), default=0), 1)
            if self._table is not None and self._table.shape[1] >= cols:
                cols = self._table.shape[1]
            else:
                cols = max(cols, 2 * (self._table.shape[1] if self._table is not None else 0))
            host = torch.full((B, cols), -1, dtype=torch.int32)
            for b, p in enumerate(self._pages):
                if p:
                    host[b, :len(p)] = torch.tensor(p, dtype=torch.int32)
            self._table = host.to(self._shape[5])
            self._table_dirty = False
        return ops.PageTable(self._table, self.page_size, self._num_blocks)

    def _layer(self, layer_idx: int) -> list[torch.Tensor]:
        pools = self._pools.get(layer_idx)
        if pools is None:
            pools = self._alloc_pool(self._num_blocks * self.page_size)
            self._pools[layer_idx] = pools
            B = self._shape[0]
            self._lens[layer_idx] = [0] * B
            self._seq_lens[layer_idx] = torch.zeros(B, dtype=torch.int32, device=self._shape[5])
        return pools

    def free_sequence(self, b: int) -> None:
        """Return sequence b's blocks to the free list and zero its length in
        every layer (the slot can then take a new sequence)."""
        for blk in reversed(self._pages[b]):
            self._release(blk)
        self._pages[b] = []
        self._table_dirty = True
        for idx in self._lens:
            self._lens[idx][b] = 0
            self._seq_lens[idx][b] = 0

    def _load_layer(self, layer_idx: int, parts: list[torch.Tensor], lens: list[int], d_head: int) -> None:
        """Install already-quantized rows ([B, H_kv, S, .] codes and scales of
        every sequence, its first lens[b] rows valid) as layer `layer_idx`."""
        kp, ks = parts[0], parts[1]
        B, H, S, _ = kp.shape
        if self._shape is None:
            self._shape = (B, H, d_head, ks.dtype, self._scale_dtype or ks.dtype, kp.device)
            self._pages = [[] for _ in range(B)]
            self._grow_pool(self._init_blocks)
        if self._shape[:3] != (B, H, d_head) or self._shape[4] != ks.dtype:
            raise ValueError("stored layer does not match the cache's shape or scale dtype")
        if layer_idx in self._pools and any(self._lens[layer_idx]):
            raise ValueError(f"layer {layer_idx} already holds state")
        self._layer(layer_idx)
        self._ensure_pages(lens)
        self._make_writable([0] * B, list(lens))
        pools = self._pools[layer_idx]
        pt = self._page_table()
        t = torch.arange(S, device=kp.device)
        page = pt.table[:, (t // self.page_size).clamp(max=pt.table.shape[1] - 1)].to(torch.int64)
        rows = page.clamp(min=0) * self.page_size + (t % self.page_size)[None, :]      # [B, S]
        valid = t[None, :] < torch.tensor(lens, device=kp.device)[:, None]            # [B, S]
        for pool, src in zip(pools, parts):
            pool[:, rows[valid]] = src.permute(1, 0, 2, 3)[:, valid]
        self._lens[layer_idx] = list(lens)
        self._seq_lens[layer_idx].copy_(torch.tensor(lens, dtype=torch.int32))

    # -- appends -------------------------------------------------------------
    def append(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int) -> None:
        """Quantize [B, H_kv, S, d] K/V and append them after each sequence's
        last position in layer `layer_idx`."""
        if key_states.shape != value_states.shape or key_states.dim() != 4:
            raise ValueError("key/value states must be [B, H_kv, S, d_head] of one shape")
        self._setup(key_states)
        pools = self._layer(layer_idx)
        S = int(key_states.shape[2])
        lens = self._lens[layer_idx]
        self._ensure_pages([n + S for n in lens])
        self._make_writable(lens, S)
        pools = self._pools[layer_idx]
        pt = self._page_table()
        pos = self._seq_lens[layer_idx]
        ops.quantize_into_paged(key_states, pools[0], pools[1], pt, self.group_size, pos)
        ops.quantize_into_paged(value_states, pools[2], pools[3], pt, self.group_size, pos)
        pos.add_(S)
        self._lens[layer_idx] = [n + S for n in lens]

    def load_ragged(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
                    lengths: torch.Tensor) -> None:
        """Start layer `layer_idx` from padded K/V [B, H_kv, S_max, d] whose
        sequence b holds lengths[b] valid rows; only those rows get blocks."""
        if layer_idx in self._pools and any(self._lens[layer_idx]):
            raise ValueError(f"layer {layer_idx} already holds state")
        if lengths.numel() != key_states.shape[0]:
            raise ValueError("lengths must have one entry per batch row")
        self._setup(key_states)
        self._layer(layer_idx)
        lens = [int(n) for n in lengths.tolist()]
        if any(n < 0 or n > key_states.shape[2] for n in lens):
            raise ValueError("lengths must lie in [0, S_max]")
        self._ensure_pages(lens)
        self._make_writable([0] * len(lens), int(key_states.shape[2]))
        pools = self._pools[layer_idx]
        pt = self._page_table()
        # rows past a sequence's length land in its last page's slack or, past
        # its pages, are dropped by the kernel; either way they are never read
        ops.quantize_into_paged(key_states, pools[0], pools[1], pt, self.group_size, 0)
        ops.quantize_into_paged(value_states, pools[2], pools[3], pt, self.group_size, 0)
        self._lens[layer_idx] = lens
        self._seq_lens[layer_idx].copy_(torch.tensor(lens, dtype=torch.int32))

    def append_and_attend(self, query_states: torch.Tensor, key_states: torch.Tensor,
                          value_states: torch.Tensor, layer_idx: int, *, n_kv_heads: int,
                          scale: float) -> Optional[torch.Tensor]:
        """One decode token per sequence: quantize-append and attend in one
        launch (``decode_step_paged``). Returns None, cache untouched, where
        the fused step does not apply (the caller appends and attends)."""
        if query_states.shape[2] != 1 or key_states.shape[2] != 1 or not query_states.is_cuda:
            return None
        if key_states.shape != value_states.shape or key_states.dim() != 4:
            return None
        if layer_idx not in self._pools or self.page_size < 64:
            return None
        self._setup(key_states)
        lens = self._lens[layer_idx]
        self._ensure_pages([n + 1 for n in lens])
        self._make_writable(lens, 1)
        pools = self._pools[layer_idx]
        pt = self._page_table()
        pos = self._seq_lens[layer_idx]
        try:
            out = ops.decode_step_paged(query_states, key_states, value_states, *pools, pt, pos,
                                        n_kv_heads=n_kv_heads, group_size=self.group_size, sm_scale=scale)
        except _native.KVQUnsupported:
            return None
        pos.add_(1)
        self._lens[layer_idx] = [n + 1 for n in lens]
        self.fused_steps += 1
        return out

    # -- decode steps captured in a HIP graph --------------------------------
    def make_static(self, extra_tokens: int) -> None:
        """Prepare every layer for decode steps captured in a HIP graph.

        A replay cannot allocate, copy blocks or upload a table, and it keeps
        the pools and the table it was captured with. So every sequence gets
        its blocks for `extra_tokens` more positions now (the pools grow now
        if they must), every block in those positions that sequences share
        (after a beam reorder or a batch repeat) is copied to its own block
        now, and the table is uploaded once. A captured decode step then finds
        nothing to allocate, copy or upload; its write positions are the
        layers' device lengths, which it advances in place.

        The Python-side lengths (``get_seq_length``) are not touched by a replay.
        Whoever replays advances them with ``advance_host_lengths``."""
        extra_tokens = int(extra_tokens)
        if extra_tokens < 0:
            raise ValueError("extra_tokens must be >= 0")
        if not self._pools or self._shape is None:
            raise ValueError("make_static needs a prefilled cache (no layer holds tokens)")
        B = self._shape[0]
        lo = [min(lens[b] for lens in self._lens.values()) for b in range(B)]
        hi = [max(lens[b] for lens in self._lens.values()) + extra_tokens for b in range(B)]
        self._ensure_pages(hi)
        self._make_writable(lo, [h - l for h, l in zip(hi, lo)])
        self._page_table()

    def buffer_signature(self) -> tuple:
        """Device addresses a HIP graph captured over this cache holds: the
        block table and every layer's pools and device lengths. An edit that
        replaces one (pool growth, a table re-upload after new or copied
        blocks) changes the signature."""
        table = None if self._table is None else (self._table.data_ptr(), tuple(self._table.shape))
        return (table, self._num_blocks) + tuple(
            (i, *(t.data_ptr() for t in pools), self._seq_lens[i].data_ptr())
            for i, pools in sorted(self._pools.items())
        )

    def host_lengths(self) -> dict[int, int]:
        """Python-side length of every layer, for a batch whose sequences all
        have one length (the graph decoder's case); raises otherwise."""
        out = {}
        for i, lens in self._lens.items():
            if len(set(lens)) > 1:
                raise ValueError(f"layer {i}: the sequences' lengths differ ({sorted(set(lens))})")
            out[i] = int(lens[0]) if lens else 0
        return out

    def advance_host_lengths(self, base: dict[int, int], n: int) -> None:
        """Set each layer's Python-side length of every sequence to base[layer]
        + n: the bookkeeping of n decode steps that ran as graph replays (the
        device lengths were advanced by the replays themselves)."""
        for i in self._lens:
            self._lens[i] = [int(base[i]) + int(n)] * len(self._lens[i])

    # -- attention -----------------------------------------------------------
    def attend(self, query_states: torch.Tensor, layer_idx: int, *, n_kv_heads: int, scale: float,
               is_causal: bool) -> torch.Tensor:
        """Attention of query_states [B, H_q, S_q, d] over each sequence's
        cached tokens (causal: bottom-right aligned to each length). Short
        query blocks run the paged fused decode kernel; long ones with one
        length for the batch the paged prefill kernel; what neither takes
        dequantizes the pages and runs dense SDPA."""
        pools = self._pools[layer_idx]
        pt = self._page_table()
        seq_lens = self._seq_lens[layer_idx]
        B, Hq, Sq, D = query_states.shape
        lens = self._lens[layer_idx]
        rows = (Hq // n_kv_heads) * Sq
        S = max(lens, default=0)
        uniform = all(n == S for n in lens)
        dense_fast = ops.dense_fast_path(query_states, None if uniform else seq_lens)
        if self.page_size >= 64 and uniform and ops.use_prefill_kernel(rows, S):
            try:
                return ops.prefill_attention_paged(
                    query_states, *pools, pt, S, n_kv_heads=n_kv_heads, group_size=self.group_size,
                    is_causal=is_causal, sm_scale=scale)
            except _native.KVQUnsupported:
                pass
        if self.page_size >= 64 and (rows <= ops.MAX_FUSED_ROWS or not dense_fast):
            try:
                return ops.fused_decode_attention_paged(
                    query_states, *pools, pt, n_kv_heads=n_kv_heads, group_size=self.group_size,
                    is_causal=is_causal, sm_scale=scale, seq_lens=seq_lens)
            except _native.KVQUnsupported:
                pass
        k = ops.dequantize_paged(pools[0], pools[1], pt, B, S, self.group_size, D, query_states.dtype)
        v = ops.dequantize_paged(pools[2], pools[3], pt, B, S, self.group_size, D, query_states.dtype)
        return ops.dense_attention(query_states, k, v, n_kv_heads=n_kv_heads, is_causal=is_causal,
                                   sm_scale=scale, seq_lens=None if uniform else seq_lens)

    # -- batch and length edits (generate(): beam search, assisted decoding) --
    def _remap(self, src: list[int]) -> None:
        """New sequence b continues old sequence src[b] (sharing its blocks)."""
        if self._shape is None:
            return
        B = self._shape[0]
        if any(s < 0 or s >= B for s in src):
            raise IndexError(f"batch index out of range for a batch of {B}")
        new_pages = [list(self._pages[s]) for s in src]
        for pages in new_pages:
            for blk in pages:
                self._ref[blk] += 1
        for pages in self._pages:
            for blk in pages:
                self._release(blk)
        self._pages = new_pages
        self._shape = (len(src),) + self._shape[1:]
        index = torch.tensor(src, dtype=torch.int64, device=self._shape[5])
        for idx in self._lens:
            self._lens[idx] = [self._lens[idx][s] for s in src]
            self._seq_lens[idx] = self._seq_lens[idx][index].contiguous()
        self._table = None
        self._table_dirty = True

    def reorder_cache(self, beam_idx: torch.Tensor) -> None:
        """Beam search (HF ``Cache.reorder_cache``): sequence b becomes the old
        sequence beam_idx[b]."""
        self._remap([int(i) for i in beam_idx.tolist()])

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        """Keep only the batch rows `indices` (int indices or a bool mask)."""
        idx = indices.nonzero().flatten() if indices.dtype == torch.bool else indices
        self._remap([int(i) for i in idx.tolist()])

    def batch_repeat_interleave(self, repeats: int) -> None:
        """Repeat every sequence `repeats` times along the batch."""
        if self._shape is not None:
            self._remap([b for b in range(self._shape[0]) for _ in range(int(repeats))])

    def activate_past_recording(self) -> None:
        """HF assisted decoding calls this before drafting. Every stored token
        is kept until ``crop``, so there is nothing to switch on."""

    def get_max_length(self, layer_idx: int = 0) -> int:
        """transformers 5.15 name of ``get_max_cache_shape``: -1, no maximum."""
        return -1

    def crop(self, max_length: int) -> None:
        """Drop tokens from the end of every sequence of every layer (HF
        ``Cache.crop``): max_length < 0 removes -max_length tokens;
        max_length > 0 keeps at most the first max_length; 0 does nothing.
        Blocks past every layer's new end are released."""
        max_length = int(max_length)
        if max_length == 0 or self._shape is None:
            return
        for idx, lens in self._lens.items():
            new = [max(n + max_length, 0) if max_length < 0 else min(n, max_length) for n in lens]
            self._lens[idx] = new
            self._seq_lens[idx].copy_(torch.tensor(new, dtype=torch.int32))
        P = self.page_size
        for b, pages in enumerate(self._pages):
            keep = -(-max((lens[b] for lens in self._lens.values()), default=0) // P)
            while len(pages) > keep:
                self._release(pages.pop())
                self._table_dirty = True

    # -- views ---------------------------------------------------------------
    def block_table(self) -> torch.Tensor:
        return self._page_table().table

    def pools(self, layer_idx: int) -> list[torch.Tensor]:
        """[k_pool, k_scales, v_pool, v_scales] of a layer."""
        return self._pools[layer_idx]

    def get_seq_lens(self, layer_idx: int) -> Optional[torch.Tensor]:
        return self._seq_lens.get(layer_idx)

    def get_quantized(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """Contiguous copies [B, H_kv, max_len, .] of a layer's codes and
        scales (rows past a sequence's length are unspecified), for callers
        that want the reference's tensor layout."""
        if layer_idx not in self._pools:
            raise KeyError(f"no cache state for layer {layer_idx}")
        S = max(self._lens[layer_idx], default=0)
        pt = self._page_table()
        t = torch.arange(S, device=pt.table.device)
        page = pt.table[:, (t // self.page_size).clamp(max=pt.table.shape[1] - 1)].to(torch.int64)
        rows = (page.clamp(min=0) * self.page_size + (t % self.page_size)[None, :])  # [B, S]
        return tuple(p[:, rows].permute(1, 0, 2, 3).contiguous() for p in self._pools[layer_idx])

    def get_dequantized(self, layer_idx: int, out_dtype: torch.dtype = torch.bfloat16
                        ) -> tuple[torch.Tensor, torch.Tensor]:
        pools = self._pools[layer_idx]
        pt = self._page_table()
        S = max(self._lens[layer_idx], default=0)
        B, D = self._shape[0], self._shape[2]
        return (ops.dequantize_paged(pools[0], pools[1], pt, B, S, self.group_size, D, out_dtype),
                ops.dequantize_paged(pools[2], pools[3], pt, B, S, self.group_size, D, out_dtype))

    # -- HF cache protocol ---------------------------------------------------
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: dict | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        del cache_kwargs
        self.append(key_states, value_states, layer_idx)
        return self.get_dequantized(layer_idx, out_dtype=key_states.dtype)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        lens = self._lens.get(layer_idx)
        return max(lens) if lens else 0

    def get_query_offset(self, layer_idx: int = 0) -> int:
        return self.get_seq_length(layer_idx)

    def get_mask_sizes(self, cache_position, layer_idx: int) -> tuple[int, int]:
        if isinstance(cache_position, torch.Tensor):
            q = int(cache_position.item()) if cache_position.dim() == 0 else int(cache_position.shape[0])
        else:
            q = int(cache_position)
        return self.get_seq_length(layer_idx) + q, 0

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return -1

    @property
    def is_initialized(self) -> bool:
        return len(self._pools) > 0

    @property
    def is_sliding(self) -> list[bool]:
        return [False for _ in self._pools]

    is_compileable = False

    def __len__(self) -> int:
        return len(self._pools)

    def has_layer(self, layer_idx: int) -> bool:
        return layer_idx in self._pools

    def nbytes(self) -> int:
        """Bytes of codes + scales of the stored tokens of all layers."""
        if self._shape is None:
            return 0
        _, H, D, _, sd, _ = self._shape
        row = ops.packed_width(D, self.group_size) + ops.num_groups(D, self.group_size) * torch.finfo(sd).bits // 8
        return sum(2 * H * row * sum(lens) for lens in self._lens.values())

    def capacity_nbytes(self) -> int:
        return sum(t.element_size() * t.numel() for pools in self._pools.values() for t in pools)
