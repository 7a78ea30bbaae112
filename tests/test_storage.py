"""The on-disk cache format (kvint4.storage): CPU round trips and format
checks, plus GPU round trips through the contiguous and paged caches.

The codes written are the reference quantizer's (kernels/llama3/quantize.py:
126-148, restated in oracle/kvq_oracle.py); the file must give back every
stored code and scale bit for bit and refuse files that break the format.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from kvint4 import storage
from kvint4.cache_base import _LayerQuantizedKV
from kvint4.llama3.kv_cache import QuantizedKVCache
from oracle import kvq_oracle as O


def _cpu_cache(seed=0, B=2, H=3, S=40, D=64, G=32, lens=None):
    rng = np.random.default_rng(seed)
    c = QuantizedKVCache(group_size=G)
    for i in range(2):
        parts = []
        for _ in range(2):
            x = rng.standard_normal((B, H, S, D)).astype(np.float32)
            p, s = O.quantize_int4(x, G, "bf16")
            parts += [torch.from_numpy(p), torch.from_numpy(s).to(torch.bfloat16)]
        sl = None if lens is None else torch.tensor(lens, dtype=torch.int32)
        c._layers[i] = _LayerQuantizedKV(*parts, S, sl)
    return c


@pytest.mark.parametrize("lens", [None, [40, 17]])
def test_round_trip_on_cpu(tmp_path, lens):
    c = _cpu_cache(lens=lens)
    path = str(tmp_path / "kv.safetensors")
    storage.save_cache(c, path)
    meta, layers = storage.read_cache_file(path)
    assert meta["format"] == "kvint4-cache" and meta["version"] == "1"
    assert meta["group_size"] == "32" and meta["d_head"] == "64" and meta["n_layers"] == "2"
    back = storage.load_cache(path, QuantizedKVCache(group_size=32), device="cpu")
    for i in range(2):
        for x, y in zip(c.get_quantized(i), back.get_quantized(i)):
            assert x.dtype == y.dtype and torch.equal(x, y)
        want = c.get_seq_lens(i)
        got = back.get_seq_lens(i)
        assert (want is None and got is None) or torch.equal(want, got)


def test_format_checks(tmp_path):
    c = _cpu_cache()
    good = str(tmp_path / "good.safetensors")
    storage.save_cache(c, good)
    _, layers = storage.read_cache_file(good)
    base = {f"layer.{i}.{k}": v for i, lay in enumerate(layers) for k, v in lay.items()}
    meta = {"format": "kvint4-cache", "version": "1", "group_size": "32", "d_head": "64", "n_layers": "2"}

    def bad(tensors, md, what):
        p = str(tmp_path / f"{what}.safetensors")
        save_file(tensors, p, metadata=md)
        with pytest.raises(ValueError):
            storage.read_cache_file(p)

    bad(base, {**meta, "format": "other"}, "format")
    bad(base, {**meta, "version": "2"}, "version")
    bad({k: v for k, v in base.items() if k != "layer.1.v_scales"}, meta, "missing")
    t = dict(base)
    t["layer.0.seq_lens"] = torch.tensor([41, 3], dtype=torch.int32)  # past S
    bad(t, meta, "lens")
    t = dict(base)
    t["layer.0.k_scales"] = base["layer.0.k_scales"][..., :1].contiguous()  # wrong group count
    bad(t, meta, "groups")
    with pytest.raises(ValueError):
        storage.load_cache(good, QuantizedKVCache(group_size=64), device="cpu")  # group size mismatch


@pytest.mark.gpu
def test_round_trip_through_contiguous_and_paged_caches(tmp_path):
    from kvint4.paged_cache import PagedQuantizedKVCache

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, D = 2, 16, 4, 128
    k = torch.randn(B, Hkv, 500, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, Hkv, 500, D, generator=g).to(torch.bfloat16).to(dev)
    lens = torch.tensor([500, 333], dtype=torch.int32)
    src = PagedQuantizedKVCache(group_size=32, page_size=64)
    for i in range(2):
        src.load_ragged(k, v, i, lens)
    path = str(tmp_path / "kv.safetensors")
    storage.save_cache(src, path)
    for dst in (QuantizedKVCache(group_size=32), PagedQuantizedKVCache(group_size=32, page_size=128)):
        storage.load_cache(path, dst, device=dev)
        for i in range(2):
            a, b = src.get_quantized(i), dst.get_quantized(i)
            for x, y in zip(a, b):
                for s, n in enumerate(lens.tolist()):
                    assert torch.equal(x[s, :, :n], y[s, :, :n])
            assert dst.get_seq_lens(i).tolist() == lens.tolist()
        # both keep decoding after the load
        q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(dev)
        kn = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(dev)
        out = dst.append_and_attend(q, kn, kn, 0, n_kv_heads=Hkv, scale=D ** -0.5)
        assert out is not None and torch.isfinite(out).all()
        assert dst.get_seq_lens(0).tolist() == [501, 334]
