"""GPU parity: HIP quantize / dequantize / in-place append vs the CPU oracle.

Bar: bit-exact packed codes and scales (and dequantized values) — integer and
byte work. Shapes cover every BASELINE config's K/V tensors (full size where
the oracle is fast; C4's 268M-element K/V is checked on a 4-sequence slice),
the exact-rational KATs, and the reference's own quantize tests
(tests/llama3/test_quantize.py, tests/gpt2/test_quantize.py).
"""

from __future__ import annotations

import json
import os
import zlib

import numpy as np
import pytest
import torch

from kvint4 import ops
from kvint4.gpt2 import quantize as gq
from kvint4.llama3 import quantize as lq
from oracle import kvq_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TDT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "int4_kat.json")))["cases"]


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def _assert_codes_equal(packed_gpu, scales_gpu, x_np, G, scale_dtype):
    want_p, want_s = O.quantize_int4(x_np, G, scale_dtype)
    got_p = packed_gpu.cpu().numpy()
    assert got_p.shape == want_p.shape
    mism = int((got_p != want_p).sum())
    assert mism == 0, f"{mism} packed bytes differ from the oracle"
    assert np.array_equal(O.bits(_np(scales_gpu), scale_dtype), O.bits(want_s, scale_dtype))


@pytest.mark.parametrize("case", KAT, ids=[c["name"] for c in KAT])
def test_kat_quantize_dequantize(case):
    x = np.array(case["x_f32_bits"], dtype=np.uint32).view(np.float32)
    xt = torch.from_numpy(x).to(TDT[case["x_dtype"]]).to(DEV)
    G = case["group_size"]
    packed, scales = ops.quantize(xt, G, TDT[case["scale_dtype"]])
    want = np.array([list(bytes.fromhex(h)) for h in case["packed"]], dtype=np.uint8)
    assert np.array_equal(packed.cpu().numpy(), want)
    assert np.array_equal(O.bits(_np(scales), case["scale_dtype"]).astype(np.int64),
                          np.array(case["scale_bits"], dtype=np.int64))
    out = ops.dequantize(packed, scales, G, x.shape[-1], TDT[case["out_dtype"]])
    assert np.array_equal(O.bits(_np(out), case["out_dtype"]).astype(np.int64),
                          np.array(case["dequant_bits"], dtype=np.int64))


# (name, shape, input dtype, scale dtype policy, outlier channels)
CONFIG_TENSORS = [
    ("c1_gpt2_small_fp32", (1, 12, 1024, 64), "f32", "gpt2", None),
    ("c2_llama8b_4k_bf16_outliers", (1, 8, 4096, 128), "bf16", "llama", "x8"),
    ("c4_llama70b_slice_bf16_t3", (4, 8, 2048, 128), "bf16", "llama", "t3"),
    ("c5_gpt2xl_fp16", (16, 25, 1024, 64), "f16", "gpt2", None),
    ("ns_llama8b_16k_bf16", (1, 8, 16384, 128), "bf16", "llama", None),
]


def _config_tensor(shape, dtype, outliers, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if outliers == "x8":
        idx = torch.tensor([3, 17, 40, 63, 77, 90, 101, 126])
        x[..., idx] *= 8
    elif outliers == "t3":
        idx = torch.tensor([5, 33, 60, 96])
        t = np.random.default_rng(seed).standard_t(3.0, size=(*shape[:-1], len(idx)))
        x[..., idx] = torch.from_numpy(t.astype(np.float32))
    return x.to(TDT[dtype])


@pytest.mark.parametrize("name,shape,dtype,policy,outliers", CONFIG_TENSORS, ids=[c[0] for c in CONFIG_TENSORS])
def test_config_tensors_bit_exact(name, shape, dtype, policy, outliers):
    x = _config_tensor(shape, dtype, outliers, seed=zlib.crc32(name.encode()) % 1000)
    quant = lq.quantize_int4 if policy == "llama" else gq.quantize_int4
    scale_dtype = dtype if policy == "llama" else "f16"
    packed, scales = quant(x.to(DEV), group_size=32)
    torch.cuda.synchronize()
    assert scales.dtype == TDT[scale_dtype]
    _assert_codes_equal(packed, scales, x.float().numpy(), 32, scale_dtype)
    deq = (lq.dequantize_int4(packed, scales, group_size=32, d_head=shape[-1]) if policy == "llama"
           else gq.dequantize_int4(packed, scales, group_size=32, d_head=shape[-1]))
    want = O.dequantize_int4(packed.cpu().numpy(), _np(scales), 32, shape[-1], scale_dtype)
    assert np.array_equal(O.bits(_np(deq), scale_dtype), O.bits(want, scale_dtype))


@pytest.mark.parametrize("G", [16, 32, 64, 128, 5, 7, 33])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_group_sizes_and_padding(G, dtype):
    x = _config_tensor((2, 3, 9, 70), dtype, None, seed=G)
    packed, scales = lq.quantize_int4(x.to(DEV), group_size=G)
    _assert_codes_equal(packed, scales, x.float().numpy(), G, dtype)
    out = lq.dequantize_int4(packed, scales, group_size=G, d_head=70, out_dtype=torch.float32)
    want = O.dequantize_int4(packed.cpu().numpy(), _np(scales), G, 70, "f32")
    assert np.array_equal(_np(out), want)


def test_strided_input_and_leading_ranks():
    x = _config_tensor((2, 5, 4, 64), "bf16", None, seed=11)  # [B, S, H, D] like a projection output
    xt = x.to(DEV).transpose(1, 2)                                   # [B, H, S, D] view, not contiguous
    packed, scales = lq.quantize_int4(xt)
    _assert_codes_equal(packed, scales, x.transpose(1, 2).float().numpy(), 32, "bf16")
    for shape in [(128,), (3, 128), (2, 2, 2, 2, 64)]:
        y = _config_tensor(shape, "f16", None, seed=len(shape))
        p, s = lq.quantize_int4(y.to(DEV))
        _assert_codes_equal(p, s, y.float().numpy(), 32, "f16")


def test_append_in_place_scalar_and_ragged_positions():
    B, H, D, cap = 3, 4, 128, 64
    kp = torch.zeros(B, H, cap, 64, dtype=torch.uint8, device=DEV)
    ks = torch.zeros(B, H, cap, 4, dtype=torch.bfloat16, device=DEV)
    x1 = _config_tensor((B, H, 10, D), "bf16", None, seed=1)
    ops.quantize_into(x1.to(DEV), kp, ks, 32, 5)
    p1, s1 = O.quantize_int4(x1.float().numpy(), 32, "bf16")
    assert np.array_equal(kp[:, :, 5:15].cpu().numpy(), p1)
    assert (kp[:, :, :5] == 0).all() and (kp[:, :, 15:] == 0).all()
    pos = torch.tensor([0, 20, 40], dtype=torch.int32, device=DEV)
    x2 = _config_tensor((B, H, 2, D), "bf16", None, seed=2)
    ops.quantize_into(x2.to(DEV), kp, ks, 32, pos)
    p2, s2 = O.quantize_int4(x2.float().numpy(), 32, "bf16")
    for b, p0 in enumerate([0, 20, 40]):
        assert np.array_equal(kp[b, :, p0:p0 + 2].cpu().numpy(), p2[b])
        assert np.array_equal(O.bits(_np(ks[b, :, p0:p0 + 2]), "bf16"), O.bits(s2[b], "bf16"))


@pytest.mark.parametrize("G", [32, 33])  # the vector kernel and the general one
def test_append_drops_rows_past_the_capacity(G):
    """Device positions: rows that land at or past the capacity are dropped,
    the rest written bit-exact. The destination is a view of a taller buffer,
    so a row written past the capacity would land in the (zero) rows below it
    rather than outside the allocation."""
    print(f"quantize past capacity: G {G}", flush=True)
    B, H, D, cap, S, pad = 4, 2, 128, 64, 4, 16
    W, NG = ops.packed_width(D, G), ops.num_groups(D, G)
    kp_full = torch.zeros(B, H, cap + pad, W, dtype=torch.uint8, device=DEV)
    ks_full = torch.zeros(B, H, cap + pad, NG, dtype=torch.bfloat16, device=DEV)
    kp, ks = kp_full[:, :, :cap], ks_full[:, :, :cap]
    starts = [62, 64, 70, 30]
    x = _config_tensor((B, H, S, D), "bf16", None, seed=9)
    ops.quantize_into(x.to(DEV), kp, ks, G, torch.tensor(starts, dtype=torch.int32, device=DEV))
    p, sc = O.quantize_int4(x.float().numpy(), G, "bf16")
    got_p, got_s = kp_full.cpu().numpy(), O.bits(_np(ks_full), "bf16")
    want_s = O.bits(sc, "bf16")
    for b, p0 in enumerate(starts):
        n = max(0, min(S, cap - p0))  # rows that fit
        assert np.array_equal(got_p[b, :, p0:p0 + n], p[b, :, :n])
        assert np.array_equal(got_s[b, :, p0:p0 + n], want_s[b, :, :n])
        rest = np.ones(cap + pad, dtype=bool)
        rest[p0:p0 + n] = False
        assert (got_p[b][:, rest] == 0).all() and (got_s[b][:, rest] == 0).all()
    with pytest.raises(ValueError):  # a scalar position whose rows do not fit
        ops.quantize_into(x.to(DEV), kp, ks, G, 61)


def test_reference_properties():
    # tests/llama3/test_quantize.py:57-83, tests/gpt2/test_quantize.py:25-40
    x = torch.randn(1, 4, 16, 128, device=DEV, dtype=torch.bfloat16)
    assert lq.quantize_int4(x)[1].dtype == torch.bfloat16
    assert lq.quantize_int4(x.half())[1].dtype == torch.float16
    assert gq.quantize_int4(x)[1].dtype == torch.float16
    z = torch.zeros(1, 2, 4, 64, dtype=torch.float16, device=DEV)
    p, s = gq.quantize_int4(z)
    assert (p == 0x88).all() and (s == 1).all()
    assert torch.equal(gq.dequantize_int4(p, s, d_head=64), z)
    p, s = lq.quantize_int4(x)
    bf = lq.dequantize_int4(p, s, d_head=128)
    hf = lq.dequantize_int4(p, s, d_head=128, out_dtype=torch.float16)
    assert bf.dtype == torch.bfloat16 and hf.dtype == torch.float16
    assert torch.allclose(bf.float(), hf.float(), rtol=5e-3, atol=5e-3)
    with pytest.raises(ValueError):
        lq.quantize_int4(x, group_size=0)
    with pytest.raises(ValueError):
        lq.quantize_int4(torch.randint(0, 5, (4, 128), dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError):
        lq.quantize_int4(torch.randn(4, 128))  # CPU tensors are not served


@pytest.mark.parametrize("seed", range(24))
def test_quantize_random_shapes(seed):
    """Seeded random quantize / dequantize calls: any head dim, group sizes
    that divide it or not (odd ones included), every input and scale dtype,
    contiguous or transposed inputs, outlier channels. Codes and scale bits
    equal the oracle's; dequantized values equal the oracle's bit for bit."""
    r = np.random.default_rng(8000 + seed)
    B, H, S = int(r.integers(1, 4)), int(r.integers(1, 6)), int(r.integers(1, 200))
    D = int(r.integers(1, 257))
    G = int(r.choice([3, 5, 7, 16, 32, 33, 48, 64, 96, 128, 200]))
    xdt = ["bf16", "f16", "f32"][r.integers(3)]
    sdt = ["bf16", "f16", "f32"][r.integers(3)]
    transposed = bool(r.random() < 0.5)
    outliers = [int(c) for c in r.choice(D, size=min(D, 3), replace=False)] if r.random() < 0.5 else None
    print(f"random quantize {seed}: B {B} H {H} S {S} D {D} G {G} {xdt}/{sdt} transposed {transposed} "
          f"outliers {outliers}", flush=True)
    g = torch.Generator().manual_seed(9000 + seed)
    x = torch.randn(*((B, S, H, D) if transposed else (B, H, S, D)), generator=g)
    if outliers:
        x[..., outliers] *= 8.0
    x = x.to(TDT[xdt])
    xd = x.to(DEV)
    if transposed:
        xd, x = xd.transpose(1, 2), x.transpose(1, 2)  # [B, H, S, D] views, not contiguous
    packed, scales = ops.quantize(xd, G, TDT[sdt])
    _assert_codes_equal(packed, scales, x.float().numpy(), G, sdt)
    out = ops.dequantize(packed, scales, G, D, torch.float32)
    want = O.dequantize_int4(packed.cpu().numpy(), _np(scales), G, D, "f32")
    assert np.array_equal(_np(out), want)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_non_finite_and_extreme_groups_agree_across_kernels(dtype):
    """Groups with a NaN element, +-inf, all zeros, values near the format's
    largest and smallest normals (scales outside [2^-100, 2^100], where the
    kernels divide for every element): the vector quantize kernel, the
    general one (taken for a strided input) and the decode step's in-kernel
    append write the same bytes. The reference defines no codes for
    non-finite inputs (its fp32 division and round give NaN before the int
    cast), so this pins the three HIP paths to each other; the finite groups
    of the same rows are also checked against the oracle."""
    B, H, D, G = 2, 4, 128, 32
    tdt = TDT[dtype]
    g = torch.Generator().manual_seed(31)
    x = (torch.randn(B, H, 1, D, generator=g) * 2).to(tdt)
    big = 3.0e38 if dtype == "bf16" else 6.0e4
    tiny = 2.0e-38 if dtype == "bf16" else 7.0e-5
    x[0, 0, 0, 3] = float("nan")
    x[0, 1, 0, 40] = float("inf")
    x[1, 2, 0, 70] = float("-inf")
    x[1, 3, 0, 96:128] = 0
    x[0, 2, 0, 0:32] = torch.linspace(-big, big, 32).to(tdt)
    x[1, 0, 0, 32:64] = torch.linspace(-tiny, tiny, 32).to(tdt)
    xd = x.to(DEV)
    special = {(0, 0, 0), (0, 1, 1), (1, 2, 2), (0, 2, 0), (1, 0, 1)}  # (b, h, group) with non-finite / extreme values

    kp_a = torch.zeros(B, H, 4, D // 2, dtype=torch.uint8, device=DEV)
    ks_a = torch.zeros(B, H, 4, D // G, dtype=tdt, device=DEV)
    ops.quantize_into(xd, kp_a, ks_a, G, 0)  # contiguous rows: the vector kernel
    xs = torch.zeros(B, H, 1, 2 * D, dtype=tdt, device=DEV)
    xs[..., ::2] = xd
    kp_b = torch.zeros_like(kp_a)
    ks_b = torch.zeros_like(ks_a)
    ops.quantize_into(xs[..., ::2], kp_b, ks_b, G, 0)  # element stride 2: the general kernel
    kp_c, vp_c = torch.zeros_like(kp_a), torch.zeros_like(kp_a)
    ks_c, vs_c = torch.zeros_like(ks_a), torch.zeros_like(ks_a)
    q = torch.randn(B, H, 1, D, generator=g).to(tdt).to(DEV)
    ops.decode_step(q, xd, xd, kp_c, ks_c, vp_c, vs_c, 0, n_kv_heads=H, group_size=G, sm_scale=D ** -0.5)
    torch.cuda.synchronize()
    row = lambda t: t[:, :, 0].cpu()
    bits = lambda t: row(t).view(torch.int16)
    assert torch.equal(row(kp_a), row(kp_b)) and torch.equal(bits(ks_a), bits(ks_b))
    assert torch.equal(row(kp_a), row(kp_c)) and torch.equal(bits(ks_a), bits(ks_c))
    assert torch.equal(row(kp_a), row(vp_c)) and torch.equal(bits(ks_a), bits(vs_c))
    # a NaN element codes as -8 (byte nibble 0) in a group whose scale the
    # finite elements set; +-inf gives an infinite scale, NaN quotients, code 0
    # for the inf element and 8 for the finite ones (x / inf = 0)
    codes = row(kp_a).numpy()
    nib = lambda b, h, d: (codes[b, h, d // 2] >> (4 * (d % 2))) & 15
    assert nib(0, 0, 3) == 0
    assert nib(0, 1, 40) == 0 and nib(0, 1, 41) == 8
    assert nib(1, 3, 100) == 8  # an all-zero group: scale 1, codes 8
    # the finite groups against the oracle
    with np.errstate(invalid="ignore"):  # the special groups' NaN quotients (not compared)
        want_p, want_s = O.quantize_int4(x.float().numpy(), G, dtype)
    got_s = O.bits(_np(ks_a[:, :, :1]), dtype)
    want_sb = O.bits(want_s, dtype)
    for b in range(B):
        for h in range(H):
            for grp in range(D // G):
                if (b, h, grp) in special:
                    continue
                sl = slice(grp * G // 2, (grp + 1) * G // 2)
                assert np.array_equal(codes[b, h, sl], want_p[b, h, 0, sl]), (b, h, grp)
                assert got_s[b, h, 0, grp] == want_sb[b, h, 0, grp], (b, h, grp)
