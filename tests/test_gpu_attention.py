"""GPU parity: fused INT4 decode attention vs the CPU oracle.

Bars (the parity targets of this path):
  * bf16 / fp16 inputs: max-abs <= 2e-2 against the reference's own oracle as
    written (dequantize to the scale dtype, repeat_interleave over the GQA
    group, SDPA in the input dtype — tests/llama3/test_attention_quant_gqa.py:
    21-40), here evaluated with torch on the CPU; and max-abs <= 2e-2 against
    the float64 oracle over exactly dequantized K/V;
  * fp32 inputs: max-abs <= 1e-4 against the float64 oracle.
Cases cover GQA ratios 1/4/8, head dims 64/128, group sizes 32/64/128,
contexts from 1 token to 16K, bottom-right causal query blocks, ragged
per-sequence lengths (including 0), the prefill route, a shape outside the
fused kernel, repeat calls (workspace reuse) and the reference's validation
errors.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kvint4 import ops
from kvint4.gpt2.attention_quant import attention_forward_quant
from kvint4.llama3.attention_quant import attention_forward_quant_gqa
from oracle import kvq_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TDT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _inputs(B, Hq, Hkv, Sq, Sk, D, dtype, seed, scale_dtype=None, G=32, outliers=()):
    """Seeded ~N(0, 1) q, K, V (K channels listed in `outliers` scaled x8),
    K and V quantized on the GPU."""
    g = torch.Generator().manual_seed(seed)
    t = TDT[dtype]
    q = torch.randn(B, Hq, Sq, D, generator=g).to(t)
    k = torch.randn(B, Hkv, Sk, D, generator=g)
    if len(outliers):
        k[..., list(outliers)] *= 8.0
    k = k.to(t)
    v = torch.randn(B, Hkv, Sk, D, generator=g).to(t)
    sd = scale_dtype or dtype
    kp, ks = ops.quantize(k.to(DEV), G, TDT[sd])
    vp, vs = ops.quantize(v.to(DEV), G, TDT[sd])
    return q, kp, ks, vp, vs


def _oracle(q, kp, ks, vp, vs, G, causal=False, seq_lens=None, scale=None):
    return O.attention_over_quantized(
        q.float().numpy(), kp.cpu().numpy(), ks.float().cpu().numpy(), vp.cpu().numpy(),
        vs.float().cpu().numpy(), group_size=G, is_causal=causal, seq_lens=seq_lens, scale=scale)


def _as_written(q, kp, ks, vp, vs, G, n_rep, causal=False):
    """The reference test's oracle (dequantize -> repeat_interleave -> SDPA in
    q's dtype), on the CPU with torch."""
    D = q.shape[-1]
    sd = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[ks.dtype]
    k = torch.from_numpy(O.dequantize_int4(kp.cpu().numpy(), ks.float().cpu().numpy(), G, D, sd))
    v = torch.from_numpy(O.dequantize_int4(vp.cpu().numpy(), vs.float().cpu().numpy(), G, D, sd))
    k = k.to(ks.dtype).to(q.dtype).repeat_interleave(n_rep, dim=1)
    v = v.to(ks.dtype).to(q.dtype).repeat_interleave(n_rep, dim=1)
    mask = None
    if causal:
        Sq, Sk = q.shape[2], k.shape[2]
        mask = torch.arange(Sk)[None, :] <= (Sk - Sq + torch.arange(Sq)[:, None])
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask).float().numpy()


DECODE_CASES = [
    # B, Hq, Hkv, Sk, D, G, dtype
    (1, 32, 8, 1, 128, 32, "bf16"),
    (1, 32, 8, 17, 128, 32, "bf16"),
    (1, 32, 8, 300, 128, 32, "bf16"),
    (1, 32, 8, 4097, 128, 32, "bf16"),
    (1, 8, 2, 1024, 128, 64, "bf16"),
    (1, 8, 2, 128, 128, 128, "bf16"),
    (2, 64, 8, 2000, 128, 32, "bf16"),
    (3, 12, 12, 1024, 64, 32, "f16"),
    (2, 16, 4, 777, 64, 32, "f16"),
    (1, 4, 4, 96, 128, 32, "bf16"),
]


@pytest.mark.parametrize("B,Hq,Hkv,Sk,D,G,dtype", DECODE_CASES)
def test_decode_matches_oracle(B, Hq, Hkv, Sk, D, G, dtype):
    q, kp, ks, vp, vs = _inputs(B, Hq, Hkv, 1, Sk, D, dtype, seed=Sk + Hq, G=G)
    out = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=Hq, n_kv_heads=Hkv, group_size=G)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    exact = _oracle(q, kp, ks, vp, vs, G)
    err = np.abs(got - exact).max()
    assert err <= 2e-2, f"vs float64 oracle: {err}"
    written = _as_written(q, kp, ks, vp, vs, G, Hq // Hkv)
    err_w = np.abs(got - written).max()
    assert err_w <= 2e-2, f"vs as-written oracle: {err_w}"


# eight fixed head-dim channels of K scaled x8 (the Llama decode configuration's outliers)
OUTLIER_CHANNELS = (3, 17, 29, 46, 64, 81, 100, 122)


def test_north_star_shape_16k():
    """Llama-3.1-8B decode shape at 16K keys with eight x8 outlier key
    channels, against both oracles (float64 over the exact dequantized
    values, and the reference's as-written bf16 dequantize -> SDPA)."""
    q, kp, ks, vp, vs = _inputs(1, 32, 8, 1, 16384, 128, "bf16", seed=16, outliers=OUTLIER_CHANNELS)
    out = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=32, n_kv_heads=8)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - _oracle(q, kp, ks, vp, vs, 32)).max()
    err_w = np.abs(got - _as_written(q, kp, ks, vp, vs, 32, 4)).max()
    print(f"NS 16K with outliers: max-abs vs float64 oracle {err:.2e}, vs as-written oracle {err_w:.2e}")
    assert err <= 2e-2, f"vs float64 oracle: {err}"
    assert err_w <= 2e-2, f"vs as-written oracle: {err_w}"


@pytest.mark.parametrize("Sk", [1, 64, 1024, 3000])
def test_fp32_inputs_1e4(Sk):
    # GPT-2 config 1 semantics: fp32 q, fp16 scales (GPT-2 quantizer)
    q, kp, ks, vp, vs = _inputs(1, 12, 12, 1, Sk, 64, "f32", seed=Sk, scale_dtype="f16")
    out = attention_forward_quant(q.to(DEV), kp, ks, vp, vs, group_size=32)
    got = out.cpu().numpy()
    err = np.abs(got - _oracle(q, kp, ks, vp, vs, 32)).max()
    assert err <= 1e-4, err


@pytest.mark.parametrize("Sq,Sk,ratio", [(2, 50, 4), (4, 300, 4), (16, 100, 4), (3, 3, 2), (8, 1030, 8)])
def test_causal_query_blocks_bottom_right(Sq, Sk, ratio):
    Hkv = 2
    q, kp, ks, vp, vs = _inputs(1, Hkv * ratio, Hkv, Sq, Sk, 128, "bf16", seed=Sq * Sk)
    out = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=Hkv * ratio, n_kv_heads=Hkv,
                                      is_causal=True)
    got = out.float().cpu().numpy()
    err = np.abs(got - _oracle(q, kp, ks, vp, vs, 32, causal=True)).max()
    assert err <= 2e-2, err


def test_ragged_seq_lens():
    B, Hq, Hkv, Sk, D = 5, 16, 4, 700, 64
    q, kp, ks, vp, vs = _inputs(B, Hq, Hkv, 1, Sk, D, "f16", seed=5)
    lens = [0, 1, 129, 700, 450]
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=Hq, n_kv_heads=Hkv, seq_lens=sl)
    got = out.float().cpu().numpy()
    want = _oracle(q, kp, ks, vp, vs, 32, seq_lens=lens)
    assert np.abs(got - want).max() <= 2e-2
    assert np.all(got[0] == 0)


def test_prefill_route_matches_oracle():
    # tests/llama3/test_attention_quant_gqa.py:58-91 (s=64, causal, 5e-2 there)
    q, kp, ks, vp, vs = _inputs(1, 4, 2, 64, 64, 128, "bf16", seed=1)
    out = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=4, n_kv_heads=2, is_causal=True)
    got = out.float().cpu().numpy()
    assert np.abs(got - _oracle(q, kp, ks, vp, vs, 32, causal=True)).max() <= 2e-2
    assert np.abs(got - _as_written(q, kp, ks, vp, vs, 32, 2, causal=True)).max() <= 2e-2


@pytest.mark.parametrize("Sq,causal", [(100, True), (100, False), (300, True), (300, False)])
def test_query_blocks_on_both_routes(Sq, causal):
    """Over 1000 keys, blocks of 400 query rows per KV head take the fused
    decode kernel; 1200 rows take the matrix-core prefill kernel. A causal
    block after cached tokens (a prompt chunk, a speculative block) is
    aligned bottom-right on both."""
    Hq, Hkv, Sk = 8, 2, 1000
    assert not ops.use_prefill_kernel((Hq // Hkv) * 100, Sk) and ops.use_prefill_kernel((Hq // Hkv) * 300, Sk)
    q, kp, ks, vp, vs = _inputs(1, Hq, Hkv, Sq, Sk, 128, "bf16", seed=Sq + causal)
    out = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=Hq, n_kv_heads=Hkv, is_causal=causal)
    got = out.float().cpu().numpy()
    assert np.abs(got - _oracle(q, kp, ks, vp, vs, 32, causal=causal)).max() <= 2e-2
    assert np.abs(got - _as_written(q, kp, ks, vp, vs, 32, Hq // Hkv, causal=causal)).max() <= 2e-2


def test_shape_outside_fused_kernel():
    q, kp, ks, vp, vs = _inputs(1, 4, 2, 1, 50, 96, "bf16", seed=3, G=16)
    out = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=4, n_kv_heads=2, group_size=16)
    got = out.float().cpu().numpy()
    assert np.abs(got - _oracle(q, kp, ks, vp, vs, 16)).max() <= 2e-2


def test_repeat_calls_are_identical():
    q, kp, ks, vp, vs = _inputs(1, 32, 8, 1, 8192, 128, "bf16", seed=9)
    qd = q.to(DEV)
    a = attention_forward_quant_gqa(qd, kp, ks, vp, vs, n_q_heads=32, n_kv_heads=8)
    b = attention_forward_quant_gqa(qd, kp, ks, vp, vs, n_q_heads=32, n_kv_heads=8)
    c = attention_forward_quant_gqa(qd, kp[:, :, :100], ks[:, :, :100], vp[:, :, :100], vs[:, :, :100],
                                    n_q_heads=32, n_kv_heads=8)
    d = attention_forward_quant_gqa(qd, kp, ks, vp, vs, n_q_heads=32, n_kv_heads=8)
    assert torch.equal(a, b) and torch.equal(a, d)
    want = _oracle(q, kp[:, :, :100], ks[:, :, :100], vp[:, :, :100], vs[:, :, :100], 32)
    assert np.abs(c.float().cpu().numpy() - want).max() <= 2e-2


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,dtype,causal", [
    (1, 32, 8, 1, 16385, 128, "bf16", False),   # one split of 512 + 1 keys
    (1, 32, 8, 1, 16640, 128, "bf16", False),   # every split 512 + 8 keys (one per wave)
    (1, 64, 8, 1, 8288, 128, "bf16", False),    # 8 query rows, 4 waves: splits of 256 + 3
    (1, 8, 4, 2, 32896, 128, "bf16", True),     # causal query block, splits of 512 + 2
    (1, 16, 4, 1, 32832, 64, "f16", False),     # D = 64, splits of 512 + 1
])
def test_split_tail_keys(B, Hq, Hkv, Sq, Sk, D, dtype, causal):
    """Splits of whole passes plus at most one key per wave fold those keys in
    with the per-wave tail path instead of another tile pass."""
    q, kp, ks, vp, vs = _inputs(B, Hq, Hkv, Sq, Sk, D, dtype, seed=Sk % 97)
    out = attention_forward_quant_gqa(q.to(DEV), kp, ks, vp, vs, n_q_heads=Hq, n_kv_heads=Hkv,
                                      is_causal=causal)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - _oracle(q, kp, ks, vp, vs, 32, causal=causal)).max()
    assert err <= 2e-2, err


def test_validation_errors():
    # tests/llama3/test_attention_quant_gqa.py:123-141
    q, kp, ks, vp, vs = _inputs(1, 8, 4, 1, 32, 128, "bf16", seed=0)
    qd = q.to(DEV)
    with pytest.raises(ValueError):
        attention_forward_quant_gqa(qd, kp, ks, vp, vs, n_q_heads=7, n_kv_heads=4)
    with pytest.raises(ValueError):
        attention_forward_quant_gqa(qd, kp, ks, vp, vs, n_q_heads=8, n_kv_heads=3)
    with pytest.raises(ValueError):
        attention_forward_quant_gqa(q, kp, ks, vp, vs, n_q_heads=8, n_kv_heads=4)
    with pytest.raises(ValueError):
        attention_forward_quant(qd.to(torch.bfloat16), kp, ks, vp, vs)


def _random_attn_case(seed):
    r = np.random.default_rng(1000 + seed)
    dtype = ["bf16", "f16", "f32"][r.integers(3)]
    sdt = ["bf16", "f16", "f32"][r.integers(3)]
    B = int(r.integers(1, 4))
    Hkv = int(r.choice([1, 2, 4, 8]))
    ratio = int(r.choice([1, 2, 4, 8]))
    Sq = int(r.choice([1, 1, 2, 3, 5, 8]))
    causal = bool(r.random() < 0.5) and Sq > 1
    D = int(r.choice([64, 128]))
    G = int(r.choice([32, 64, 128]))
    Sk = int(r.integers(1, 2200))
    lens = None
    if r.random() < 0.5:
        lens = [int(r.integers(0, Sk + 1)) for _ in range(B)]
    n_split = None if r.random() < 0.5 else int(r.integers(1, 12))
    return dtype, sdt, B, Hkv, ratio, Sq, causal, D, G, Sk, lens, n_split


@pytest.mark.parametrize("seed", range(24))
def test_fused_attention_random_shapes(seed):
    """Seeded random calls of the fused kernel itself (both kernels by query
    and scale dtype): multi-token query blocks with and without the
    bottom-right causal mask (the row-masked instances), GQA ratios that split
    the rows into several chunks, ragged lengths including 0, forced split
    counts. Bar: 1e-4 (fp32 queries) or 2e-2 against the float64 oracle."""
    dtype, sdt, B, Hkv, ratio, Sq, causal, D, G, Sk, lens, n_split = _random_attn_case(seed)
    Hq = Hkv * ratio
    print(f"random fused attention {seed}: {dtype}/{sdt} B {B} Hq {Hq} Hkv {Hkv} Sq {Sq} causal {causal} "
          f"D {D} G {G} Sk {Sk} lens {lens} n_split {n_split}", flush=True)
    q, kp, ks, vp, vs = _inputs(B, Hq, Hkv, Sq, Sk, D, dtype, seed=2000 + seed, scale_dtype=sdt, G=G)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV) if lens is not None else None
    if n_split is not None:
        n_split = max(1, min(n_split, Sk // 128))
    sm = D ** -0.5
    out = ops.fused_decode_attention(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=G, is_causal=causal,
                                     sm_scale=sm, seq_lens=sl, n_split=n_split)
    got = out.float().cpu().numpy()
    want = _oracle(q, kp, ks, vp, vs, G, causal=causal, seq_lens=lens, scale=sm)
    tol = 1e-4 if dtype == "f32" else 2e-2
    assert np.isfinite(got).all()
    err = np.abs(got - want).max()
    assert err <= tol, err


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("ratio", [1, 2, 4, 8])
def test_split_merge_every_group_size(dtype, D, ratio):
    """The cross-split merge at every lane-group size it has: a piece of the
    partials (4 dims of one query row) is shared by P = threads / (rows * D /
    4) threads, lanes 64 / P apart, combined with shuffles: P = 2, 4 or 8 in
    the matrix kernel (D 64/128, 4 or 8 rows), 1 to 16 in the fp32 kernel (1
    to 8 rows). Seven splits (not a multiple of any P, so some groups fold
    fewer splits), ragged lengths, against the float64 oracle."""
    B, Hkv, Sk = 2, 2, 1500
    Hq = Hkv * ratio
    lens = [1500, 700]
    print(f"merge groups: {dtype} D {D} ratio {ratio}", flush=True)
    q, kp, ks, vp, vs = _inputs(B, Hq, Hkv, 1, Sk, D, dtype, seed=77 + D + ratio, G=32)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    sm = D ** -0.5
    out = ops.fused_decode_attention(q.to(DEV), kp, ks, vp, vs, n_kv_heads=Hkv, group_size=32, is_causal=False,
                                     sm_scale=sm, seq_lens=sl, n_split=7)
    got = out.float().cpu().numpy()
    want = _oracle(q, kp, ks, vp, vs, 32, seq_lens=lens, scale=sm)
    tol = 1e-4 if dtype == "f32" else 2e-2
    assert np.isfinite(got).all()
    err = np.abs(got - want).max()
    assert err <= tol, err
