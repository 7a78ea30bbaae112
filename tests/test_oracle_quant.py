"""Pin the CPU oracle's quantizer (oracle/kvq_oracle.py, oracle/kvq_ref.c).

Checks, each chosen so that a plausible mistake fails at least one:
  * exact-rational known answers (tests/golden/int4_kat.json, no floats used
    to produce them): wrong rounding rule (half-away vs half-even), reciprocal
    multiply instead of IEEE division, scale rounded before use, wrong nibble
    order, wrong padding nibble;
  * closed forms and invariants: zero group -> 0x88 and scale 1, max -> 15,
    -max -> 1, codes in 1..15, |x - deq| <= scale/2, concat == one-shot;
  * brute force: each code minimises |x/scale - (c - 8)| over all 16 codes;
  * the reference tests' own properties (tests/gpt2/test_quantize.py:11-40,
    tests/llama3/test_quantize.py:18-32);
  * the independent C restatement agrees bit for bit.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import kvq_oracle as O
from oracle import kvq_ref as R

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "int4_kat.json")))["cases"]


def _x(case) -> np.ndarray:
    return np.array(case["x_f32_bits"], dtype=np.uint32).view(np.float32)


@pytest.mark.parametrize("case", KAT, ids=[c["name"] for c in KAT])
@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_quantize_matches_exact_kat(case, impl):
    x = _x(case)
    G = case["group_size"]
    q = O.quantize_int4 if impl == "numpy" else R.quantize_int4
    packed, scales = q(x, G, case["scale_dtype"])
    want_packed = np.array([list(bytes.fromhex(h)) for h in case["packed"]], dtype=np.uint8)
    assert np.array_equal(packed, want_packed)
    assert np.array_equal(O.bits(scales, case["scale_dtype"]).astype(np.int64),
                          np.array(case["scale_bits"], dtype=np.int64))


@pytest.mark.parametrize("case", KAT, ids=[c["name"] for c in KAT])
@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_dequantize_matches_exact_kat(case, impl):
    x = _x(case)
    G = case["group_size"]
    packed = np.array([list(bytes.fromhex(h)) for h in case["packed"]], dtype=np.uint8)
    scales = O.from_bits(np.array(case["scale_bits"]), case["scale_dtype"])
    dq = O.dequantize_int4 if impl == "numpy" else R.dequantize_int4
    out = dq(packed, scales, G, x.shape[-1], case["out_dtype"])
    assert np.array_equal(O.bits(out, case["out_dtype"]).astype(np.int64),
                          np.array(case["dequant_bits"], dtype=np.int64))


def test_half_even_not_half_away():
    # x/scale = 2.5, 3.5, -2.5 exactly (scale = 1): half-even gives 2, 4, -2.
    x = np.zeros(32, np.float32)
    x[:4] = [7.0, 2.5, 3.5, -2.5]
    packed, scales = O.quantize_int4(x, 32, "f32")
    assert scales[0] == 1.0
    codes = np.stack([packed & 15, packed >> 4], -1).reshape(-1)
    assert list(codes[:4]) == [15, 10, 12, 6]


def test_zero_group_is_0x88_and_scale_one():
    packed, scales = O.quantize_int4(np.zeros((2, 64), np.float32), 32, "bf16")
    assert (packed == 0x88).all() and (scales == 1.0).all()


def test_extremes_and_code_range():
    rng = np.random.default_rng(3)
    x = O.round_to(rng.standard_normal((64, 128)).astype(np.float32), "bf16")
    packed, scales = O.quantize_int4(x, 32, "bf16")
    codes = np.stack([packed & 15, packed >> 4], -1).reshape(64, 4, 32)
    assert codes.min() >= 1 and codes.max() <= 15  # |x/scale| <= 7 -> no code 0
    g = x.reshape(64, 4, 32)
    imax = np.abs(g).argmax(-1)
    picked = np.take_along_axis(codes, imax[..., None], -1)[..., 0]
    sign = np.sign(np.take_along_axis(g, imax[..., None], -1)[..., 0])
    assert np.all(np.where(sign > 0, picked == 15, picked == 1))


def test_bruteforce_nearest_code():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((16, 64)) * 5).astype(np.float32)
    packed, _ = O.quantize_int4(x, 32, "f32")
    g = x.reshape(16, 2, 32).astype(np.float64)
    amax = np.abs(g).max(-1, keepdims=True)
    scale = np.float32(amax / 7.0).astype(np.float64)  # fp32 scale, as the codes use
    q = g / scale
    cand = np.arange(-8, 8)[None, None, None, :]
    dist = np.abs(q[..., None] - cand)
    best = dist.min(-1, keepdims=True)
    codes = np.stack([packed & 15, packed >> 4], -1).reshape(16, 2, 32).astype(np.int64) - 8
    chosen = np.take_along_axis(dist, (codes + 8)[..., None], -1)
    assert np.all(chosen <= best + 1e-6)


def test_roundtrip_error_bounds_reference_properties():
    # tests/llama3/test_quantize.py:18-32 and tests/gpt2/test_quantize.py:11-40
    rng = np.random.default_rng(0)
    for G in (32, 64, 128):
        x = O.round_to(rng.standard_normal((2, 8, 64, 128)).astype(np.float32), "bf16")
        packed, scales = O.quantize_int4(x, G, "bf16")
        assert packed.shape[-1] == 64 and scales.shape[-1] == 128 // G
        xh = O.dequantize_int4(packed, scales, G, 128, "bf16")
        assert np.abs(x - xh).mean() < np.abs(scales).mean()
        # per-element bound: half a step, plus |n-8| <= 8 times the bf16 rounding
        # of the stored scale, plus the bf16 rounding of the product (a half ulp
        # of an 8-bit significand is at most 2^-8 relative)
        s_full = np.repeat(scales, G, axis=-1)
        assert np.all(np.abs(x - xh) <= s_full * (0.5 + 8 * 2.0**-8 + 8 * 2.0**-8))
    x = O.round_to(rng.standard_normal((2, 3, 5, 64)).astype(np.float32), "f16")
    p, s = O.quantize_int4(x, 32, "f16")
    assert np.abs(x - O.dequantize_int4(p, s, 32, 64, "f16")).mean() < 0.2
    x = rng.standard_normal((2, 2, 3, 70)).astype(np.float32)
    p, s = O.quantize_int4(x, 32, "f16")
    assert p.shape[-1] == 48 and s.shape[-1] == 3
    assert O.dequantize_int4(p, s, 32, 70, "f16").shape[-1] == 70


def test_concat_equals_one_shot():
    # cf. tests/llama3/test_quantize_sm70.py:145-168 (here exact, since rows are independent)
    rng = np.random.default_rng(5)
    x = O.round_to(rng.standard_normal((1, 4, 64, 128)).astype(np.float32), "bf16")
    cache = None
    for a, b in ((0, 37), (37, 38), (38, 64)):
        cache = O.cache_append(cache, x[:, :, a:b], x[:, :, a:b], 32, "bf16")
    p0, s0 = O.quantize_int4(x, 32, "bf16")
    assert np.array_equal(cache[0], p0) and np.array_equal(cache[1], s0)


def test_c_matches_numpy_large():
    rng = np.random.default_rng(6)
    for dt in ("bf16", "f16", "f32"):
        x = O.round_to((rng.standard_normal((8, 1024, 128)) * 4).astype(np.float32), dt)
        x[0, :, [3, 17, 40, 77]] *= 8
        x = O.round_to(x, dt)
        p1, s1 = O.quantize_int4(x, 32, dt)
        p2, s2 = R.quantize_int4(x, 32, dt)
        assert np.array_equal(p1, p2)
        assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


def test_group_scale_without_division_is_exact():
    """The HIP kernels form the group scale absmax / 7 without a division
    (kv-cache-triton_amd/csrc/kvq_common.h group_scale: am * RN(1/7) corrected
    once with an fma). Checked against the IEEE quotient the reference computes
    (kernels/llama3/quantize.py:137-141) for every non-negative finite float:
    zero, all subnormals and all normal values (oracle/kvq_ref.c
    kvqref_check_div7)."""
    assert R.lib().kvqref_check_div7(0, 0x7F800000) == 0


def test_rint_with_approximate_inverse_is_exact_outside_the_tie_margin():
    """The quantize kernels round x / s as rint(RN(x * inv)) with inv =
    v_rcp_f32(s) (1 ulp), and divide only when RN(x * inv) lies within 2^-17
    of a half-integer (kv-cache-triton_amd/csrc/kvq_common.h rint_quotient).
    Sampled scales and elements, random and a few ulps from every tie, with
    inverses up to 8 ulps off: no element outside the margin rounds
    differently from rint of the correctly rounded quotient. The same check
    with a margin below the error bound (2^-20 at 1 ulp, 2^-19 at 2 ulps)
    finds such elements, so the sampling reaches the ties."""
    lib = R.lib()
    assert lib.kvqref_check_rint_margin(11, 4_000_000, 2, 17) == 0
    assert lib.kvqref_check_rint_margin(12, 1_000_000, 8, 17) == 0
    assert lib.kvqref_check_rint_margin(13, 1_000_000, 1, 20) > 0
    assert lib.kvqref_check_rint_margin(13, 1_000_000, 2, 19) > 0


def test_packed_rint_with_magic_add_is_exact_outside_the_tie_margin():
    """The vector quantize kernel computes code + 8 as u - 2^23 with
    u = RN(RN(x * inv + 8) + 2^23) (one fma, one add that rounds to an
    integer, ties to even), and divides only when the exact residual
    t - (u - 2^23) is within 2^-17 of 1/2
    (kv-cache-triton_amd/csrc/kvq_quant.hip quantize_vec_kernel). Sampled as
    above, plus the group extremes +-absmax with s = RN(absmax / 7): every
    element outside the margin gets rint of the correctly rounded quotient,
    and a code in [1, 15] (so the kernel needs no clamp there). A margin
    below the error bound finds misses, so the sampling reaches the ties."""
    lib = R.lib()
    assert lib.kvqref_check_rint_margin_fma8(11, 4_000_000, 2, 17) == 0
    assert lib.kvqref_check_rint_margin_fma8(12, 1_000_000, 8, 17) == 0
    assert lib.kvqref_check_rint_margin_fma8(13, 1_000_000, 1, 20) > 0
    assert lib.kvqref_check_rint_margin_fma8(13, 1_000_000, 2, 20) > 0
