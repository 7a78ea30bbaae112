"""GPU: edge cases of the hot path — empty inputs, an empty cache, an empty
batch, and a context of a million keys.

Conventions where the reference has no defined result:
  * attention over zero keys (an empty cache, or a ragged sequence of length
    0) returns zeros. The reference's kernel divides the empty softmax sum by
    itself there (kernels/llama3/attention_quant.py:148, no guard), i.e. NaN;
  * empty tensors pass through every operator and come back empty.

The long-context case is checked against the C restatement (oracle/kvq_ref.c,
itself pinned against the fp64 numpy oracle in tests/test_oracle_attention.py)
at the attention bar, on codes written by the HIP quantizer (whose bytes are
pinned separately).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvint4 import ops
from kvint4.llama3.attention_quant import attention_forward_quant_gqa
from kvint4.llama3.quantize import dequantize_int4, quantize_int4
from oracle import kvq_ref as R

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _codes(B, Hkv, Sk, D, G, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn(B, Hkv, Sk, D, device=DEV, generator=g).to(dtype)
    kp, ks = quantize_int4(k, G)
    del k
    v = torch.randn(B, Hkv, Sk, D, device=DEV, generator=g).to(dtype)
    vp, vs = quantize_int4(v, G)
    return kp, ks, vp, vs


def test_empty_quantize_dequantize_and_append():
    x = torch.empty(2, 3, 0, 128, dtype=torch.bfloat16, device=DEV)
    p, s = quantize_int4(x, 32)
    assert p.shape == (2, 3, 0, 64) and s.shape == (2, 3, 0, 4) and s.dtype == torch.bfloat16
    out = dequantize_int4(p, s, 32, 128)
    assert out.shape == (2, 3, 0, 128)
    # appending zero rows at a position leaves the cache untouched
    kp = torch.randint(0, 256, (2, 3, 8, 64), dtype=torch.uint8, device=DEV)
    ks = torch.rand(2, 3, 8, 4, device=DEV).to(torch.bfloat16)
    kp0, ks0 = kp.clone(), ks.clone()
    ops.quantize_into(x, kp, ks, 32, 5)
    ops.quantize_into(x, kp, ks, 32, torch.tensor([1, 7], dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(kp, kp0) and torch.equal(ks, ks0)


def test_attention_empty_batch():
    kp, ks, vp, vs = _codes(1, 2, 16, 128, 32, seed=1)
    q = torch.empty(0, 8, 1, 128, dtype=torch.bfloat16, device=DEV)
    out = attention_forward_quant_gqa(q, kp[:0], ks[:0], vp[:0], vs[:0], n_q_heads=8, n_kv_heads=2)
    assert out.shape == (0, 8, 1, 128)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attention_over_an_empty_cache_is_zero(dtype):
    kp, ks, vp, vs = _codes(2, 2, 16, 128, 32, seed=2, dtype=dtype)
    q = torch.randn(2, 8, 1, 128, device=DEV).to(dtype)
    out = attention_forward_quant_gqa(q, kp[:, :, :0], ks[:, :, :0], vp[:, :, :0], vs[:, :, :0],
                                      n_q_heads=8, n_kv_heads=2)
    assert out.shape == q.shape and torch.all(out == 0)


def test_million_key_context_matches_c_oracle():
    B, Hq, Hkv, D, G = 1, 32, 8, 128, 32
    Sk = (1 << 20) + 3        # a split tail of a few keys at the end
    kp, ks, vp, vs = _codes(B, Hkv, Sk, D, G, seed=3)
    q = torch.randn(B, Hq, 1, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    out = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=Hq, n_kv_heads=Hkv)
    got = out.float().cpu().numpy()
    want = R.decode_attn(q.float().numpy(), kp.cpu().numpy(), ks.float().cpu().numpy(), vp.cpu().numpy(),
                         vs.float().cpu().numpy(), group_size=G, scale=D ** -0.5)
    err = np.abs(got - want).max()
    print(f"1M-key context: max-abs err {err:.2e}")
    assert err <= 2e-2, err
    # the new key written and attended in one launch at this length
    pos = Sk - 1
    kn = torch.randn(B, Hkv, 1, D, device=DEV).to(torch.bfloat16)
    vn = torch.randn(B, Hkv, 1, D, device=DEV).to(torch.bfloat16)
    step = ops.decode_step(q.to(DEV), kn, vn, kp, ks, vp, vs, pos, n_kv_heads=Hkv, group_size=G,
                           sm_scale=D ** -0.5)
    ref = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=Hq, n_kv_heads=Hkv)
    assert (step.float() - ref.float()).abs().max().item() <= 2e-2
