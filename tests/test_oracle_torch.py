"""The torch restatement of the reference's CPU path (oracle/kvq_torch.py),
which bench.py times as the CPU baseline, pinned against the numpy oracle:
codes and scales bit for bit (bf16 / fp16 / fp32 inputs, even, odd and padded
group sizes, exact ties), dequantized values exactly, the torch.cat append
equal to one-shot quantization of the whole history, and decode attention
within the bf16 bar of the fp64 oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kvq_oracle as O
from oracle import kvq_torch as T

_NP = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("G,d", [(32, 128), (32, 64), (64, 128), (128, 128), (7, 20), (16, 40), (33, 64)])
def test_quantize_matches_numpy_oracle(dtype, G, d):
    g = torch.Generator().manual_seed(G * 1000 + d)
    x = (torch.randn(2, 3, 17, d, generator=g) * 3).to(dtype)
    x[0, 0, 0] = 0  # an all-zero row: scale 1, codes 8
    x[1, 2, 3, :4] = torch.tensor([7.0, -7.0, 3.5, -0.5]).to(dtype)  # exact ties at scale 1
    p, s = T.quantize_int4(x, G)
    op, os_ = O.quantize_int4(x.float().numpy(), G, _NP[dtype])
    assert np.array_equal(p.numpy(), op)
    assert s.dtype == dtype
    assert np.array_equal(s.float().numpy(), os_)
    deq = T.dequantize_int4(p, s, G, d, torch.float32)
    assert np.array_equal(deq.numpy(), O.dequantize_int4(op, os_, G, d, "f32"))


def test_gpt2_policy_fp16_scales():
    x = torch.randn(1, 12, 9, 64, generator=torch.Generator().manual_seed(0))
    p, s = T.quantize_int4(x, 32, torch.float16)
    op, os_ = O.quantize_int4(x.numpy(), 32, "f16")
    assert np.array_equal(p.numpy(), op) and s.dtype == torch.float16
    assert np.array_equal(s.float().numpy(), os_)


def test_cat_append_equals_one_shot_and_attention_bar():
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, S, D, G = 1, 8, 2, 300, 128, 32
    k = torch.randn(B, Hkv, S + 3, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S + 3, D, generator=g).to(torch.bfloat16)
    kp, ks = T.quantize_int4(k[:, :, :S], G)
    vp, vs = T.quantize_int4(v[:, :, :S], G)
    cache = T.LayerCache(kp, ks, vp, vs, G)
    for t in range(3):
        q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
        out = T.decode_step(cache, q, k[:, :, S + t:S + t + 1], v[:, :, S + t:S + t + 1], D ** -0.5)
        n = S + t + 1
        okp, oks = O.quantize_int4(k[:, :, :n].float().numpy(), G, "bf16")
        ovp, ovs = O.quantize_int4(v[:, :, :n].float().numpy(), G, "bf16")
        assert np.array_equal(cache.kp.numpy(), okp) and np.array_equal(cache.vp.numpy(), ovp)
        assert np.array_equal(cache.ks.float().numpy(), oks) and np.array_equal(cache.vs.float().numpy(), ovs)
        want = O.attention_over_quantized(q.float().numpy(), okp, oks, ovp, ovs, group_size=G)
        assert float(np.abs(out.float().numpy() - want).max()) < 2e-2
