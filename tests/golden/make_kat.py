"""Write tests/golden/int4_kat.json: known-answer vectors for the INT4 quantizer.

The expected outputs are computed in exact rational arithmetic
(fractions.Fraction) from the quantizer's mathematical definition
(kernels/llama3/quantize.py:126-148, kernels/gpt2/quantize.py:111-133):

    scale  = fp32(max|x_g| / 7)           (1 when the group is all zero)
    code   = round_half_even(fp32(x / scale)) clamped to [-8, 7], plus 8
    stored = scale rounded to the scale dtype (nearest, ties to even)
    deq    = out_dtype(fp32((code - 8) * scale))

where fp32(.)/bf16(.)/fp16(.) are exact round-to-nearest-even of a rational.
No floating-point operation is used to produce an expected value, so these
vectors pin the float implementations (numpy oracle, C oracle, HIP kernels)
independently of any of them. Inputs are drawn with numpy only to pick
representable values; cases include exact ties, near-ties decided by the fp32
rounding of the quotient, all-zero groups, padding (d % G != 0) and odd G.

    python tests/golden/make_kat.py      # rewrites int4_kat.json
"""

from __future__ import annotations

import json
import math
import os
import struct
from fractions import Fraction as Fr

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "int4_kat.json")

# (significand bits incl. implicit one, min normal exponent, max exponent)
FORMATS = {"f32": (24, -126, 127), "bf16": (8, -126, 127), "f16": (11, -14, 15)}


def rne(x: Fr, fmt: str) -> Fr:
    """Exact round-to-nearest-even of rational x into a binary format."""
    p, emin, emax = FORMATS[fmt]
    if x == 0:
        return Fr(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fr(2) ** e > a:
        e -= 1
    while Fr(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    quantum = Fr(2) ** (e - (p - 1))
    n = round(a / quantum)  # Fraction.__round__: ties to even
    r = n * quantum
    if r >= Fr(2) ** (emax + 1):
        raise OverflowError("rounds to infinity")
    return sign * r


def f32_bits(v: Fr) -> int:
    return struct.unpack("<I", struct.pack("<f", float(v)))[0]


def to_bits(v: Fr, fmt: str) -> int:
    if fmt == "f32":
        return f32_bits(v)
    if fmt == "bf16":
        return f32_bits(v) >> 16
    return int(np.float16(float(v)).view(np.uint16))  # v is exactly representable


def from_f32_bits(b: int) -> Fr:
    return Fr(struct.unpack("<f", struct.pack("<I", b))[0])


def quantize_exact(row: list[Fr], G: int):
    d = len(row)
    ng = math.ceil(d / G)
    codes_all, scales = [], []
    for g in range(ng):
        grp = [row[c] if c < d else Fr(0) for c in range(g * G, g * G + G)]
        amax = max(abs(v) for v in grp)
        scale = rne(amax / 7, "f32") if amax > 0 else Fr(1)
        codes = []
        for v in grp:
            qf = rne(v / scale, "f32")
            c = max(-8, min(7, round(qf)))
            codes.append(c + 8)
        if G % 2:
            codes.append(0)
        codes_all.append(codes)
        scales.append(scale)
    packed = []
    for codes in codes_all:
        for j in range(0, len(codes), 2):
            packed.append(codes[j] | (codes[j + 1] << 4))
    return packed, scales, codes_all


def case(name, x_fmt, scale_fmt, G, rows: list[list[Fr]], out_fmt):
    packed_rows, scale_rows, deq_rows = [], [], []
    for row in rows:
        packed, scales, codes_all = quantize_exact(row, G)
        packed_rows.append(packed)
        stored = [rne(s, scale_fmt) for s in scales]
        scale_rows.append([to_bits(s, scale_fmt) for s in stored])
        deq = []
        for c in range(len(row)):
            g, k = divmod(c, G)
            n = codes_all[g][k]
            deq.append(to_bits(rne(rne((n - 8) * stored[g], "f32"), out_fmt), out_fmt))
        deq_rows.append(deq)
    return {
        "name": name,
        "x_dtype": x_fmt,
        "scale_dtype": scale_fmt,
        "out_dtype": out_fmt,
        "group_size": G,
        "x_f32_bits": [[f32_bits(v) for v in row] for row in rows],
        "packed": [bytes(p).hex() for p in packed_rows],
        "scale_bits": scale_rows,
        "dequant_bits": deq_rows,
    }


def representable(vals: np.ndarray, fmt: str) -> list[Fr]:
    vals = np.asarray(vals, dtype=np.float32)
    if fmt == "bf16":
        u = vals.view(np.uint32).astype(np.uint64)
        vals = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    elif fmt == "f16":
        vals = vals.astype(np.float16).astype(np.float32)
    return [Fr(float(v)) for v in vals]


def near_tie_rows(rng: np.random.Generator, G: int, want: int) -> list[list[Fr]]:
    """fp32 rows in which up to 8 elements sit within +-2 ulps of
    (k + 1/2) * scale, so the code depends on the correctly rounded fp32
    quotient x / scale (a reciprocal-multiply or a wider division can differ)."""
    rows = []
    while len(rows) < want:
        base = [Fr(float(v)) for v in (rng.standard_normal(G) * rng.uniform(0.05, 20)).astype(np.float32)]
        amax = max(abs(v) for v in base)
        imax = max(range(G), key=lambda i: abs(base[i]))
        scale = rne(amax / 7, "f32")
        row = list(base)
        for i in [i for i in range(G) if i != imax][:8]:
            k = int(rng.integers(-7, 7)) + Fr(1, 2)
            xf = np.float32(float(rne(k * scale, "f32")))
            steps = int(rng.integers(-2, 3))
            for _ in range(abs(steps)):
                xf = np.nextafter(xf, np.float32(np.inf if steps > 0 else -np.inf))
            x = Fr(float(xf))
            if abs(x) < amax:
                row[i] = x
        rows.append(row)
    return rows


def main() -> None:
    rng = np.random.default_rng(20261201)
    cases = []
    # exact ties with an exactly representable scale (amax = 7 * 2^k)
    for fmt in ("bf16", "f16", "f32"):
        s = Fr(1, 4)
        row = [7 * s, -7 * s] + [Fr(h, 2) * s for h in (1, 3, 5, 7, 9, 11, 13, -1, -3, -5, -7, -9, -11, -13)]
        row += [Fr(0)] * (32 - len(row))
        cases.append(case(f"ties_{fmt}", fmt, fmt, 32, [row], fmt))
    # all-zero groups, mixed with a live group; padding d=70; odd group sizes
    cases.append(case("zero_groups_f16", "f16", "f16", 32,
                      [[Fr(0)] * 64, [Fr(0)] * 32 + representable(rng.standard_normal(32), "f16")], "f16"))
    for fmt, scale_fmt, out_fmt in (("bf16", "bf16", "bf16"), ("f16", "f16", "f16"), ("f32", "f16", "f16"),
                                    ("f32", "f32", "f32"), ("bf16", "f16", "bf16")):
        for G in (32, 64, 128):
            rows = [representable(rng.standard_normal(128) * rng.uniform(0.01, 50), fmt) for _ in range(3)]
            cases.append(case(f"rand_{fmt}_{scale_fmt}_G{G}", fmt, scale_fmt, G, rows, out_fmt))
        rows = [representable(rng.standard_normal(70) * 3, fmt) for _ in range(2)]
        cases.append(case(f"pad70_{fmt}_{scale_fmt}", fmt, scale_fmt, 32, rows, out_fmt))
        for G in (5, 7):
            rows = [representable(rng.standard_normal(24), fmt) for _ in range(2)]
            cases.append(case(f"oddG{G}_{fmt}_{scale_fmt}", fmt, scale_fmt, G, rows, out_fmt))
        # outlier channels (x8), as in the Llama decode config
        rows = []
        for _ in range(2):
            v = rng.standard_normal(128)
            v[[3, 17, 40, 77, 90, 101, 115, 126]] *= 8
            rows.append(representable(v, fmt))
        cases.append(case(f"outliers_{fmt}_{scale_fmt}", fmt, scale_fmt, 32, rows, out_fmt))
    cases.append(case("near_ties_f32", "f32", "f32", 32, near_tie_rows(rng, 32, 8), "f32"))
    cases.append(case("near_ties_f32_f16scale", "f32", "f16", 32, near_tie_rows(rng, 32, 8), "f16"))
    with open(OUT, "w") as f:
        json.dump({"generator": "tests/golden/make_kat.py", "cases": cases}, f, indent=0)
    print(f"wrote {len(cases)} cases to {OUT}")


if __name__ == "__main__":
    main()
