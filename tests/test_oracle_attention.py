"""Pin the attention oracle (oracle/kvq_oracle.attention) on the CPU.

  * equals torch's scaled_dot_product_attention (CPU, float64) with the GQA
    group expanded by repeat_interleave — the reference's own test oracle
    (tests/llama3/test_attention_quant_gqa.py:15-40);
  * closed forms: identical keys -> mean of the values; one key with a huge
    score -> that key's value; a single key -> its value;
  * GQA map h -> h // ratio (a transposed map h -> h % n_kv fails);
  * bottom-right causal alignment (a top-left alignment fails for Sq < Sk);
  * per-sequence lengths == running each sequence alone; empty rows are zero;
  * the C restatement agrees.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kvq_oracle as O
from oracle import kvq_ref as R


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.parametrize("Hq,Hkv,Sq,causal", [(8, 2, 1, False), (4, 4, 1, False), (8, 1, 5, True),
                                               (6, 3, 7, False), (4, 2, 16, True)])
def test_matches_torch_sdpa(Hq, Hkv, Sq, causal):
    q, k, v = _rand((2, Hq, Sq, 64), 1), _rand((2, Hkv, 40, 64), 2), _rand((2, Hkv, 40, 64), 3)
    scale = 64 ** -0.5
    got = O.attention(q, k, v, scale=scale, is_causal=causal)
    qt, kt, vt = (torch.from_numpy(a) for a in (q, k, v))
    kt = kt.repeat_interleave(Hq // Hkv, dim=1)
    vt = vt.repeat_interleave(Hq // Hkv, dim=1)
    mask = None
    if causal:  # bottom-right: query i sees keys j <= Sk - Sq + i
        i = torch.arange(Sq)[:, None]
        j = torch.arange(40)[None, :]
        mask = j <= (40 - Sq + i)
    want = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale).numpy()
    assert np.abs(got - want).max() < 1e-12


def test_closed_forms():
    q = _rand((1, 2, 1, 32), 4)
    v = _rand((1, 1, 10, 32), 5)
    k_same = np.repeat(_rand((1, 1, 1, 32), 6), 10, axis=2)
    out = O.attention(q, k_same, v, scale=1.0)
    assert np.allclose(out[0, 0, 0], v[0, 0].mean(0), atol=1e-12)
    k = np.zeros((1, 1, 10, 32))
    k[0, 0, 7] = 1000.0 * np.sign(q[0, 0, 0])
    out = O.attention(q[:, :1], k, v, scale=1.0)
    assert np.allclose(out[0, 0, 0], v[0, 0, 7], atol=1e-12)
    out = O.attention(q, v[:, :, :1], v[:, :, :1], scale=1.0)
    assert np.allclose(out[0, :, 0], np.repeat(v[0, 0, :1], 2, 0), atol=1e-12)


def test_gqa_map_is_h_div_ratio():
    q = _rand((1, 4, 1, 16), 7)
    k, v = _rand((1, 2, 12, 16), 8), _rand((1, 2, 12, 16), 9)
    out = O.attention(q, k, v, scale=0.25)
    for h in range(4):
        alone = O.attention(q[:, h:h + 1], k[:, h // 2:h // 2 + 1], v[:, h // 2:h // 2 + 1], scale=0.25)
        assert np.allclose(out[:, h:h + 1], alone, atol=1e-13)
    other = O.attention(q[:, 1:2], k[:, 1:2], v[:, 1:2], scale=0.25)  # h % n_kv map
    assert not np.allclose(out[:, 1:2], other, atol=1e-3)


def test_bottom_right_causal():
    q, k, v = _rand((1, 1, 3, 8), 10), _rand((1, 1, 10, 8), 11), _rand((1, 1, 10, 8), 12)
    out = O.attention(q, k, v, scale=1.0, is_causal=True)
    for i in range(3):
        lim = 10 - 3 + i + 1
        alone = O.attention(q[:, :, i:i + 1], k[:, :, :lim], v[:, :, :lim], scale=1.0)
        assert np.allclose(out[:, :, i:i + 1], alone, atol=1e-13)


def test_ragged_equals_separate_and_empty_is_zero():
    q, k, v = _rand((3, 4, 1, 16), 13), _rand((3, 2, 20, 16), 14), _rand((3, 2, 20, 16), 15)
    lens = [5, 20, 0]
    out = O.attention(q, k, v, scale=0.3, seq_lens=lens)
    for b in range(2):
        alone = O.attention(q[b:b + 1], k[b:b + 1, :, :lens[b]], v[b:b + 1, :, :lens[b]], scale=0.3)
        assert np.allclose(out[b:b + 1], alone, atol=1e-13)
    assert np.all(out[2] == 0)


@pytest.mark.parametrize("causal,lens", [(False, None), (True, None), (False, [33, 200, 1])])
def test_c_restatement_agrees(causal, lens):
    q = _rand((3, 8, 2, 128), 16).astype(np.float32)
    k = O.round_to(_rand((3, 2, 200, 128), 17).astype(np.float32), "bf16")
    v = O.round_to(_rand((3, 2, 200, 128), 18).astype(np.float32), "bf16")
    kp, ks = O.quantize_int4(k, 32, "bf16")
    vp, vs = O.quantize_int4(v, 32, "bf16")
    a = O.attention_over_quantized(q, kp, ks, vp, vs, group_size=32, is_causal=causal, seq_lens=lens)
    b = R.decode_attn(q, kp, ks, vp, vs, group_size=32, scale=128 ** -0.5, is_causal=causal,
                      seq_lens=lens, threads=4)
    assert np.abs(a - b).max() < 2e-6
