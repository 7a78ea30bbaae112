"""The reference's PyTorch CPU path, restated in torch — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and the ``cpu_baseline`` leg of ``bench.py`` may import this
module: it is the timed CPU baseline (the path a user of the reference runs
without a GPU), never part of the product. It follows the reference's CPU
operators step by step, in code of our own:

  quantize_int4     kernels/llama3/quantize.py:126-148 (_quantize_int4_torch):
                    zero-pad d to a multiple of G, per group amax, scale =
                    amax / 7 (1 where amax == 0), codes = clamp(round(x /
                    scale), -8, 7) + 8 with torch.round (half to even), element
                    2i in the low nibble of byte i, scales cast to x's dtype
                    (GPT-2: fp16, kernels/gpt2/quantize.py:111-133).
  dequantize_int4   kernels/llama3/quantize.py:210-234 (_dequantize_int4_torch):
                    (nibble - 8) * float(scale), cast to the output dtype.
  LayerCache.append models/llama3/kv_cache.py:76-102: quantize the new K and V
                    and torch.cat the four tensors onto the layer's along the
                    sequence axis (the whole layer is copied every step).
  decode_attention  models/llama3/llama3_quant.py:90-100,117-143 on the CPU:
                    dequantize the whole cache, repeat each KV head over its
                    GQA group (kv head h // ratio), scaled_dot_product_attention.

Pinned by tests/test_oracle_torch.py against the numpy oracle
(oracle/kvq_oracle.py, itself pinned by exact-rational known answers): codes
and scales bit for bit, dequantized values exactly, attention within 2e-2.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def quantize_int4(x: torch.Tensor, group_size: int, scale_dtype: torch.dtype | None = None):
    """x [..., d] -> (packed [..., ceil(d/G) * G/2] uint8, scales [..., ceil(d/G)])."""
    G = int(group_size)
    d = x.shape[-1]
    ng = -(-d // G)
    xf = x.float()
    if ng * G != d:
        xf = F.pad(xf, (0, ng * G - d))
    g = xf.reshape(*x.shape[:-1], ng, G)
    amax = g.abs().amax(dim=-1, keepdim=True)
    scale = torch.where(amax > 0, amax / 7.0, torch.ones_like(amax))
    codes = (torch.round(g / scale).clamp_(-8, 7) + 8).to(torch.uint8)  # [..., ng, G]
    if G % 2:  # each group packs into ceil(G / 2) bytes, its last high nibble zero
        codes = F.pad(codes, (0, 1))
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).reshape(*x.shape[:-1], -1)
    sd = x.dtype if scale_dtype is None else scale_dtype
    return packed.contiguous(), scale.squeeze(-1).to(sd)


def dequantize_int4(packed: torch.Tensor, scales: torch.Tensor, group_size: int, d_head: int,
                    out_dtype: torch.dtype) -> torch.Tensor:
    """(nibble - 8) * float(scale) -> out_dtype, first d_head columns."""
    G = int(group_size)
    ng = scales.shape[-1]
    lo = (packed & 0x0F).to(torch.int16)
    hi = (packed >> 4).to(torch.int16)
    codes = torch.stack((lo, hi), dim=-1).reshape(*packed.shape[:-1], ng, -1)[..., :G]
    vals = (codes - 8).float() * scales.float().unsqueeze(-1)
    return vals.reshape(*packed.shape[:-1], ng * G)[..., :d_head].to(out_dtype)


class LayerCache:
    """One layer of the reference's cache: four tensors grown by torch.cat."""

    def __init__(self, kp: torch.Tensor, ks: torch.Tensor, vp: torch.Tensor, vs: torch.Tensor, group_size: int):
        self.kp, self.ks, self.vp, self.vs = kp, ks, vp, vs
        self.group_size = int(group_size)

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        kp, ks = quantize_int4(k, self.group_size)
        vp, vs = quantize_int4(v, self.group_size)
        self.kp = torch.cat((self.kp, kp), dim=2)
        self.ks = torch.cat((self.ks, ks), dim=2)
        self.vp = torch.cat((self.vp, vp), dim=2)
        self.vs = torch.cat((self.vs, vs), dim=2)

    def decode_attention(self, q: torch.Tensor, scale: float) -> torch.Tensor:
        """q [B, Hq, 1, D] over every cached token."""
        D = q.shape[-1]
        k = dequantize_int4(self.kp, self.ks, self.group_size, D, q.dtype)
        v = dequantize_int4(self.vp, self.vs, self.group_size, D, q.dtype)
        ratio = q.shape[1] // k.shape[1]
        if ratio > 1:
            k = k.repeat_interleave(ratio, dim=1)
            v = v.repeat_interleave(ratio, dim=1)
        return F.scaled_dot_product_attention(q, k, v, scale=scale)


def decode_step(cache: LayerCache, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                scale: float) -> torch.Tensor:
    """One decode token of one layer on the reference's CPU path: append the
    new K/V (quantize + concatenate), then attend over the whole cache."""
    cache.append(k_new, v_new)
    return cache.decode_attention(q, scale)
