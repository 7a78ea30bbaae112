"""GPU parity: the matrix-core prefill kernel (kvq_prefill_attn) vs the fp64
oracle and vs the dequantize + dense SDPA route.

Reference semantics (kernels/llama3/attention_quant.py:24-152, Sq > 1): GQA
head map h // ratio, scores q.k * d^-1/2, causal mask aligned bottom-right
(key j admissible for query i iff j <= Sk - Sq + i), online softmax over
dequantized K/V. Bar: max-abs <= 2e-2 for bf16/fp16, as for the decode
kernel (tests/llama3/test_attention_quant_gqa.py:58-91 uses 5e-2 for its
prefill case). Cases: a prompt (Sq == Sk), prompt chunks after cached tokens,
GQA ratios 1/4/8, head dims 64/128, group sizes 32/64/128, fp16, more queries
than keys (rows with no admissible key are zero), an empty cache, and
non-contiguous views of a larger cache. Launches too small to fill the
device split the key range and merge the splits' partials (log-sum-exp)
in a second launch; those cases run through that path.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvint4 import ops
from oracle import kvq_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TDT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _inputs(B, Hq, Hkv, Sq, Sk, D, dtype, G, seed, cap=None):
    g = torch.Generator().manual_seed(seed)
    t = TDT[dtype]
    q = torch.randn(B, Hq, Sq, D, generator=g).to(t)
    cap = cap or Sk
    k = torch.randn(B, Hkv, cap, D, generator=g).to(t)
    v = torch.randn(B, Hkv, cap, D, generator=g).to(t)
    kp, ks = ops.quantize(k.to(DEV), G, t)
    vp, vs = ops.quantize(v.to(DEV), G, t)
    # views of the first Sk rows of a larger cache
    return q, kp[:, :, :Sk], ks[:, :, :Sk], vp[:, :, :Sk], vs[:, :, :Sk]


def _oracle(q, kp, ks, vp, vs, G, causal):
    return O.attention_over_quantized(
        q.float().numpy(), kp.cpu().numpy(), ks.float().cpu().numpy(), vp.cpu().numpy(),
        vs.float().cpu().numpy(), group_size=G, is_causal=causal)


CASES = [
    # B, Hq, Hkv, Sq, Sk, D, G, dtype, causal
    (2, 8, 2, 100, 100, 128, 32, "bf16", True),     # a prompt
    (1, 32, 8, 300, 1000, 128, 32, "bf16", True),   # a chunk after 700 cached tokens
    (1, 8, 8, 70, 200, 64, 64, "f16", False),       # MHA, D 64, G 64
    (2, 16, 2, 33, 500, 128, 128, "bf16", True),    # GQA 8, G 128
    (1, 4, 1, 129, 129, 64, 32, "f16", True),       # GQA 4, D 64, a row block cut short
    (1, 8, 2, 200, 150, 128, 32, "bf16", True),     # more queries than keys
    (1, 8, 2, 100, 3000, 128, 32, "bf16", True),    # split over keys (5 splits), merged
    (1, 8, 2, 1100, 1100, 128, 32, "bf16", True),   # a prompt split in two: early row blocks leave a split empty
]


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,G,dtype,causal", CASES)
def test_prefill_matches_oracle_and_dense_route(B, Hq, Hkv, Sq, Sk, D, G, dtype, causal):
    q, kp, ks, vp, vs = _inputs(B, Hq, Hkv, Sq, Sk, D, dtype, G, seed=Sq * 7 + Sk, cap=Sk + 37)
    out = ops.prefill_attention(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G,
                                is_causal=causal, sm_scale=D ** -0.5)
    got = out.float().cpu().numpy()
    want = _oracle(q, kp, ks, vp, vs, G, causal)
    err = np.abs(got - want).max()
    print(f"prefill B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} D={D} G={G} {dtype}: max-abs {err:.2e}")
    assert err <= 2e-2, err
    if causal and Sq > Sk:  # rows with no admissible key
        assert np.all(got[:, :, : Sq - Sk] == 0)
    dense = ops.dense_attention_over_quantized(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G,
                                               is_causal=causal, sm_scale=D ** -0.5)
    assert (out.float() - dense.float()).abs().max().item() <= 2e-2


def test_prefill_empty_cache_and_unsupported():
    q, kp, ks, vp, vs = _inputs(1, 8, 2, 16, 0, 128, "bf16", 32, seed=1, cap=8)
    out = ops.prefill_attention(q.to(DEV), kp, ks, vp, vs, n_kv_heads=2, group_size=32, is_causal=False,
                                sm_scale=0.1)
    assert torch.all(out == 0)
    from kvint4._native import KVQUnsupported

    q32 = torch.randn(1, 8, 16, 128, device=DEV)
    k = torch.randn(1, 2, 32, 128, device=DEV)
    kp, ks = ops.quantize(k, 32, torch.float32)
    with pytest.raises(KVQUnsupported):
        ops.prefill_attention(q32, kp, ks, kp, ks, n_kv_heads=2, group_size=32, is_causal=True, sm_scale=0.1)


@pytest.mark.parametrize("B", [1, 2])
def test_prefill_two_row_blocks_per_wave(B):
    """Launches of >= 256 workgroups of 128 rows take two 16-row blocks per
    wave (B = 2: 256 workgroups of eight waves and 256 rows, unsplit; B = 1:
    256 of four waves and 128 rows, split in two over keys):
    the whole output against the dense route, and rows across the block
    against the fp64 oracle (row i of a causal block after cached tokens
    attends keys [0, Sk - Sq + i])."""
    Hq, Hkv, Sq, Sk, D, G = 32, 8, 1024, 3000, 128, 32
    assert B * Hkv * (Sq * (Hq // Hkv) // 128) >= 256
    q, kp, ks, vp, vs = _inputs(B, Hq, Hkv, Sq, Sk, D, "bf16", G, seed=11)
    out = ops.prefill_attention(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G, is_causal=True,
                                sm_scale=D ** -0.5)
    dense = ops.dense_attention_over_quantized(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G,
                                               is_causal=True, sm_scale=D ** -0.5)
    assert (out.float() - dense.float()).abs().max().item() <= 2e-2
    got = out.float().cpu().numpy()
    for i in (0, 1, 37, 500, 1023):
        n = Sk - Sq + i + 1
        want = O.attention_over_quantized(
            q[:, :, i:i + 1].float().numpy(), kp[:, :, :n].cpu().numpy(), ks[:, :, :n].float().cpu().numpy(),
            vp[:, :, :n].cpu().numpy(), vs[:, :, :n].float().cpu().numpy(), group_size=G, is_causal=False)
        assert np.abs(got[:, :, i:i + 1] - want).max() <= 2e-2, i


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_prefill_eight_waves_per_workgroup(dtype):
    """D = 128 launches of at least 256 workgroups of 256 rows take eight
    waves per workgroup (each thread dequantizes half as much of a K/V tile):
    here 8 KV heads x 4096 query positions x GQA 4 (512). The whole output against
    the dense route, and rows across the block (including the first and last
    of a workgroup and of its waves) against the fp64 oracle."""
    Hq, Hkv, Sq, Sk, D, G = 32, 8, 4096, 4160, 128, 32
    assert Hkv * (Sq * (Hq // Hkv) // 256) >= 512
    q, kp, ks, vp, vs = _inputs(1, Hq, Hkv, Sq, Sk, D, dtype, G, seed=23)
    out = ops.prefill_attention(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G, is_causal=True,
                                sm_scale=D ** -0.5)
    dense = ops.dense_attention_over_quantized(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G,
                                               is_causal=True, sm_scale=D ** -0.5)
    assert (out.float() - dense.float()).abs().max().item() <= 2e-2
    got = out.float().cpu().numpy()
    for i in (0, 1, 7, 8, 63, 64, 2047, 4095):
        n = Sk - Sq + i + 1
        want = O.attention_over_quantized(
            q[:, :, i:i + 1].float().numpy(), kp[:, :, :n].cpu().numpy(), ks[:, :, :n].float().cpu().numpy(),
            vp[:, :, :n].cpu().numpy(), vs[:, :, :n].float().cpu().numpy(), group_size=G, is_causal=False)
        assert np.abs(got[:, :, i:i + 1] - want).max() <= 2e-2, i


def _random_prefill_case(seed):
    r = np.random.default_rng(6000 + seed)
    dtype = ["bf16", "f16"][r.integers(2)]
    B = int(r.integers(1, 3))
    Hkv = int(r.choice([1, 2, 4, 8]))
    ratio = int(r.choice([1, 2, 4, 8]))
    D = int(r.choice([64, 128]))
    G = min(int(r.choice([32, 64, 128])), D)  # the kernel takes groups that divide D
    Sk = int(r.integers(1, 2500))
    Sq = int(r.integers(1, min(Sk, 700) + 1)) if r.random() < 0.8 else int(r.integers(Sk, Sk + 200))
    causal = bool(r.random() < 0.7)
    return dtype, B, Hkv, ratio, D, G, Sq, Sk, causal


@pytest.mark.parametrize("seed", range(16))
def test_prefill_random_shapes(seed):
    """Seeded random query blocks on the prefill kernel (GQA ratios, D, G,
    fp16/bf16, prompts, chunks after cached tokens, more queries than keys,
    causal or not, launches that split over keys): within 2e-2 of the float64
    oracle."""
    dtype, B, Hkv, ratio, D, G, Sq, Sk, causal = _random_prefill_case(seed)
    Hq = Hkv * ratio
    print(f"random prefill {seed}: {dtype} B {B} Hq {Hq} Hkv {Hkv} D {D} G {G} Sq {Sq} Sk {Sk} causal {causal}",
          flush=True)
    q, kp, ks, vp, vs = _inputs(B, Hq, Hkv, Sq, Sk, D, dtype, G, seed=7000 + seed, cap=Sk + 17)
    out = ops.prefill_attention(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G, is_causal=causal,
                                sm_scale=D ** -0.5)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - _oracle(q, kp, ks, vp, vs, G, causal)).max()
    assert err <= 2e-2, err


@pytest.mark.parametrize("sm_scale", [-(128 ** -0.5), 0.0, 0.02])
def test_prefill_any_softmax_scale(sm_scale):
    """The kernel takes the row max over unscaled scores and scales with
    fma(s, |c|, -m); a negative sm_scale negates the queries instead, and 0
    weighs every admissible key alike. Causal prompt chunk (diagonal tiles
    masked, the rest not) against the fp64 oracle at the same scale."""
    B, Hq, Hkv, Sq, Sk, D, G = 1, 8, 2, 150, 300, 128, 32
    print(f"prefill sm_scale {sm_scale}", flush=True)
    q, kp, ks, vp, vs = _inputs(B, Hq, Hkv, Sq, Sk, D, "bf16", G, seed=91)
    out = ops.prefill_attention(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G, is_causal=True,
                                sm_scale=sm_scale)
    want = O.attention_over_quantized(
        q.float().numpy(), kp.cpu().numpy(), ks.float().cpu().numpy(), vp.cpu().numpy(),
        vs.float().cpu().numpy(), group_size=G, scale=sm_scale, is_causal=True)
    err = np.abs(out.float().cpu().numpy() - want).max()
    print(f"prefill sm_scale {sm_scale}: max-abs {err:.2e}")
    assert err <= 2e-2, err
    dense = ops.dense_attention_over_quantized(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G,
                                               is_causal=True, sm_scale=sm_scale)
    assert (out.float() - dense.float()).abs().max().item() <= 2e-2


def test_prefill_scales_beyond_2_pow_125():
    """Dequantization runs as fma(n, sc, -8 sc), exact while -8 sc does not
    overflow; a tile holding a scale above 2^125 is written again as
    (n - 8) sc. One key's values carry a bf16 scale of 4.5e37 (codes 1..15:
    |(n - 8) sc| <= 3.2e38, finite) and a key row of -2 that keeps its weight
    near 1e-7, so that its values dominate every output without overflowing.
    The fma form would turn that key's values into -inf."""
    B, Hq, Hkv, Sq, Sk, D, G = 1, 4, 1, 64, 128, 128, 32
    g = torch.Generator().manual_seed(5)
    q = torch.full((B, Hq, Sq, D), 0.5).to(torch.bfloat16)
    k = torch.randn(B, Hkv, Sk, D, generator=g)
    k[:, :, 77] = -2.0
    v = torch.randn(B, Hkv, Sk, D, generator=g)
    kp, ks = ops.quantize(k.to(torch.bfloat16).to(DEV), G, torch.bfloat16)
    vp, vs = ops.quantize(v.to(torch.bfloat16).to(DEV), G, torch.bfloat16)
    codes = torch.randint(1, 16, (B, Hkv, D), generator=g, dtype=torch.int32)
    vp[:, :, 77] = (codes[..., 0::2] | (codes[..., 1::2] << 4)).to(torch.uint8).to(DEV)
    vs[:, :, 77] = torch.tensor(4.5e37, dtype=torch.bfloat16)
    assert float(vs[0, 0, 77, 0]) > 2.0 ** 125
    out = ops.prefill_attention(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G, is_causal=False,
                                sm_scale=D ** -0.5)
    got = out.float().cpu().numpy()
    want = O.attention_over_quantized(
        q.float().numpy(), kp.cpu().numpy(), ks.float().cpu().numpy(), vp.cpu().numpy(),
        vs.float().cpu().numpy(), group_size=G, is_causal=False)
    assert np.isfinite(want).all() and np.abs(want).max() > 1e25
    assert np.isfinite(got).all()
    assert np.all(np.abs(got - want) <= 2e-2 + 3e-2 * np.abs(want))
