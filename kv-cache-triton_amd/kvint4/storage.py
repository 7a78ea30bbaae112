"""On-disk format of the packed INT4 KV cache ("kvint4-cache", version 1).

The reference has no save/load for its cache; this is a stable layout for the
packed codes and scales so that a prompt's cache can be kept on disk or moved
between processes (prompt caching, KV offload) and read back into either the
contiguous ``QuantizedKVCache`` or the ``PagedQuantizedKVCache``.

A safetensors file holding, for every layer i = 0 .. n_layers - 1:

    layer.{i}.k_packed   uint8 [B, H_kv, S_i, W]      W = ceil(d/G) * ceil(G/2)
    layer.{i}.k_scales   [B, H_kv, S_i, ceil(d/G)]    bf16, fp16 or fp32
    layer.{i}.v_packed   uint8 [B, H_kv, S_i, W]
    layer.{i}.v_scales   [B, H_kv, S_i, ceil(d/G)]
    layer.{i}.seq_lens   int32 [B]                    valid rows of each sequence

Codes follow the reference quantizer (kernels/llama3/quantize.py:126-148):
per group of G elements along d, scale = max|x| / 7 (1 for an all-zero
group), code = clamp(round_half_even(x / scale), -8, 7) + 8, element 2j of a
group in the low nibble of byte j, groups padded to even length with code 0.
S_i is the longest sequence; rows at or past seq_lens[b] are unspecified.
String metadata: format = "kvint4-cache", version = "1", group_size, d_head,
n_layers.
"""

from __future__ import annotations

from typing import Union

import torch
from safetensors.torch import load_file, save_file

from . import ops
from .cache_base import QuantizedKVCacheBase, _LayerQuantizedKV
from .paged_cache import PagedQuantizedKVCache

FORMAT = "kvint4-cache"
VERSION = "1"
PARTS = ("k_packed", "k_scales", "v_packed", "v_scales")

Cache = Union[QuantizedKVCacheBase, PagedQuantizedKVCache]


def _layers_of(cache: Cache) -> list[int]:
    if isinstance(cache, PagedQuantizedKVCache):
        return sorted(cache._pools)
    return sorted(cache._layers)


def save_cache(cache: Cache, path: str) -> None:
    """Write every layer of `cache` (layers 0 .. n-1, all present) to `path`."""
    idx = _layers_of(cache)
    if idx != list(range(len(idx))):
        raise ValueError(f"layers must be 0 .. n-1 (got {idx})")
    tensors: dict[str, torch.Tensor] = {}
    d_head = 0
    for i in idx:
        parts = cache.get_quantized(i)
        lens = cache.get_seq_lens(i)
        if lens is None:
            lens = torch.full((parts[0].shape[0],), parts[0].shape[2], dtype=torch.int32)
        for name, t in zip(PARTS, parts):
            tensors[f"layer.{i}.{name}"] = t.detach().contiguous().cpu()
        tensors[f"layer.{i}.seq_lens"] = lens.detach().to(torch.int32).cpu()
        d_head = parts[1].shape[-1] * cache.group_size
    meta = {"format": FORMAT, "version": VERSION, "group_size": str(cache.group_size),
            "d_head": str(d_head), "n_layers": str(len(idx))}
    save_file(tensors, path, metadata=meta)


def read_cache_file(path: str) -> tuple[dict, list[dict[str, torch.Tensor]]]:
    """(metadata, per-layer dicts of CPU tensors) of a cache file, checked
    against the format."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        meta = dict(f.metadata() or {})
    if meta.get("format") != FORMAT:
        raise ValueError(f"{path}: not a {FORMAT} file (format={meta.get('format')!r})")
    if meta.get("version") != VERSION:
        raise ValueError(f"{path}: unsupported {FORMAT} version {meta.get('version')!r}")
    G, d, n = int(meta["group_size"]), int(meta["d_head"]), int(meta["n_layers"])
    if G <= 0 or d <= 0 or n < 0:
        raise ValueError(f"{path}: bad metadata {meta}")
    raw = load_file(path)
    w, ng = ops.packed_width(d, G), ops.num_groups(d, G)
    layers = []
    for i in range(n):
        try:
            lay = {name: raw[f"layer.{i}.{name}"] for name in (*PARTS, "seq_lens")}
        except KeyError as e:
            raise ValueError(f"{path}: layer {i} is incomplete ({e})") from None
        kp, ks, vp, vs, sl = (lay[k] for k in (*PARTS, "seq_lens"))
        B, H, S = kp.shape[:3]
        if (kp.dtype != torch.uint8 or vp.dtype != torch.uint8 or kp.shape != (B, H, S, w)
                or vp.shape != kp.shape or ks.shape != (B, H, S, ng) or vs.shape != ks.shape
                or ks.dtype != vs.dtype or ks.dtype not in ops.SUPPORTED_FLOATS
                or sl.dtype != torch.int32 or sl.shape != (B,)
                or bool((sl < 0).any()) or bool((sl > S).any())):
            raise ValueError(f"{path}: layer {i} tensors do not match the format")
        layers.append(lay)
    return meta, layers


def load_cache(path: str, cache: Cache, device: Union[str, torch.device] = "cuda") -> Cache:
    """Fill an empty cache (contiguous or paged) from a file written by
    save_cache; returns it. The group size must match the cache's."""
    meta, layers = read_cache_file(path)
    if int(meta["group_size"]) != cache.group_size:
        raise ValueError(f"file group size {meta['group_size']} != cache group size {cache.group_size}")
    if _layers_of(cache):
        raise ValueError("load_cache needs an empty cache")
    dev = torch.device(device)
    for i, lay in enumerate(layers):
        parts = [lay[name].to(dev) for name in PARTS]
        lens = lay["seq_lens"]
        if isinstance(cache, PagedQuantizedKVCache):
            cache._load_layer(i, parts, [int(n) for n in lens.tolist()], int(meta["d_head"]))
            continue
        S = parts[0].shape[2]
        ragged = bool((lens != S).any())
        cache._layers[i] = _LayerQuantizedKV(*parts, S, lens.to(dev) if ragged else None)
    return cache
