"""Writes tests/golden/kats.json: known-answer vectors for the hot path.

The reference (github.com/giraffesyo/ingot) stores no golden files for this
path: its tests compute expectations in-test. This script restates those
tests' inputs and derives the expected outputs with exact Python integer /
rational arithmetic, independent of oracle/oracle.c:

- gemm_transb      TestGemmTransB        ops/compute_optest_test.go:232-252
- matmul_batched   TestMatMulBatched     ops/compute_optest_test.go:254-274
- dequantize_*     TestDequantizeLinear  ops/quant_optest_test.go:60-73
- matmul_integer   the closed form of TestQLinearMatMulAndMatMulInteger
                   (ops/quant_optest_test.go:194-223: m=7, k=33, n=12,
                   za=110); inputs come from a seeded numpy generator because
                   Go's PCG stream is not reproduced here
- qlinear_ref      QLinearMatMul's requantisation (ops/quant.go:902-928) of
                   the matmul_integer product with the scales of the same
                   reference test; qlinear_ties a power-of-two-scale case that
                   hits exact .5 ties and both s8 saturation ends
- bf16_rne         F32ToBF16 (kernels/gemm/bgemm.go:20-26) special cases,
                   expected bits from exact round-half-to-even on rationals
                   plus the NaN rule (quiet bit set, sign kept)

Run: python tests/golden/make_kats.py
"""
from __future__ import annotations

import json
import os
import struct
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def iota(*shape):
    n = 1
    for d in shape:
        n *= d
    return list(range(n))


def f32_bits_to_fraction(bits: int):
    f = struct.unpack("<f", struct.pack("<I", bits))[0]
    return Fraction(f)


def bf16_rne_exact(bits: int) -> int:
    """Round the float32 with these bits to bfloat16 by exact arithmetic."""
    exp = (bits >> 23) & 0xFF
    if exp == 0xFF:
        if bits & 0x7FFFFF:  # NaN: the reference keeps it a quiet NaN, sign kept
            return ((bits >> 16) | 0x40) & 0xFFFF
        return bits >> 16  # ±Inf
    sign = bits >> 31
    x = abs(f32_bits_to_fraction(bits))
    lo = (bits & 0x7FFFFFFF) >> 16  # truncated magnitude bits
    lo_val = f32_bits_to_fraction(lo << 16)
    hi_val = f32_bits_to_fraction((lo + 1) << 16) if lo + 1 < 0x7F80 else None
    if hi_val is None:  # next step is infinity: halfway point is 2^128 - 2^119·... use bit distance
        ulp = lo_val - f32_bits_to_fraction((lo - 1) << 16)
        hi_val = lo_val + ulp
    d_lo, d_hi = x - lo_val, hi_val - x
    if d_lo < d_hi or (d_lo == d_hi and lo % 2 == 0):
        r = lo
    else:
        r = lo + 1
    return (sign << 15) | r


def requant(raw, sa, sb, sy, zy, u8):
    """satU8/satI8(RoundToEven(fl32(fl32(float32(v)·mult) + zy))), mult = fl32(fl32(sa·sb)/sy): each f32
    operation rounded by numpy float32 scalars, the integer rounding by Python's round (half to even)."""
    f = np.float32
    mult = f(f(f(sa) * f(sb)) / f(sy))
    lo, hi = (0, 255) if u8 else (-128, 127)
    out = []
    for v in raw:
        u = f(f(f(v) * mult) + f(zy))
        out.append(min(max(round(float(u)), lo), hi))
    return out


def main():
    kats = {}
    # TestGemmTransB: A=iota(2,3), B=iota(4,3), C=[100..400], alpha=2, beta=1, transB
    a, b, c = iota(2, 3), iota(4, 3), [100, 200, 300, 400]
    y = [[2 * sum(a[i * 3 + k] * b[j * 3 + k] for k in range(3)) + c[j] for j in range(4)] for i in range(2)]
    kats["gemm_transb"] = {"A": a, "A_shape": [2, 3], "B": b, "B_shape": [4, 3], "C": c, "alpha": 2.0, "beta": 1.0,
                           "transB": 1, "Y": y}
    # TestMatMulBatched: [2,2,3] x [2,3,2]
    a, b = iota(2, 2, 3), iota(2, 3, 2)
    y = [[[sum(a[(bt * 2 + i) * 3 + k] * b[(bt * 3 + k) * 2 + j] for k in range(3)) for j in range(2)]
          for i in range(2)] for bt in range(2)]
    kats["matmul_batched"] = {"A": a, "A_shape": [2, 2, 3], "B": b, "B_shape": [2, 3, 2], "Y": y}
    # TestDequantizeLinear
    kats["dequantize_u8"] = {"x": [0, 128, 255], "x_dtype": "u8", "scale": [0.5], "zp": [128], "zp_dtype": "u8",
                             "y": [-64.0, 0.0, 63.5]}
    kats["dequantize_i8"] = {"x": [-128, 127], "x_dtype": "i8", "scale": [2.0], "zp": [-8], "zp_dtype": "i8",
                             "y": [-240.0, 270.0]}
    # MatMulInteger closed form, m=7 k=33 n=12 za=110
    rng = np.random.default_rng(2526)
    m, k, n, za = 7, 33, 12, 110
    av = rng.integers(0, 256, size=m * k).tolist()
    bv = (rng.integers(0, 256, size=k * n).astype(np.uint8).view(np.int8)).tolist()
    y = [[sum((av[i * k + p] - za) * bv[p * n + j] for p in range(k)) for j in range(n)] for i in range(m)]
    kats["matmul_integer"] = {"m": m, "k": k, "n": n, "za": za, "A": av, "B": bv, "Y": y}
    # QLinearMatMul requant (ops/quant.go:902-928): the reference test's scales on the same product, and a
    # power-of-two scale case whose products land on .5 (round half to even) and saturate the s8 range
    raw = [v for row in y for v in row]
    kats["qlinear_ref"] = {"raw": raw, "sa": 0.1, "sb": 0.05, "sy": 0.7, "zy": 3, "u8": True,
                           "Y": requant(raw, 0.1, 0.05, 0.7, 3, True)}
    rng = np.random.default_rng(2627)
    m2, k2, n2, za2 = 9, 40, 11, 17
    a2 = rng.integers(za2 - 3, za2 + 4, size=m2 * k2).tolist()
    b2 = rng.integers(-3, 4, size=k2 * n2).tolist()
    raw2 = [sum((a2[i * k2 + p] - za2) * b2[p * n2 + j] for p in range(k2)) for i in range(m2) for j in range(n2)]
    raw2 += [8, -8, 24, -24, 2040, -2056, 40, 56]  # exact ties and both saturation ends
    kats["qlinear_ties"] = {"m": m2, "k": k2, "n": n2, "za": za2, "A": a2, "B": b2, "raw": raw2, "sa": 0.25,
                            "sb": 0.125, "sy": 0.5, "zy": -5, "u8": False,
                            "Y": requant(raw2, 0.25, 0.125, 0.5, -5, False)}
    # F32ToBF16 special cases
    cases = [0x3F800000, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F807FFF, 0x3F817FFF, 0x00000000, 0x80000000,
             0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0xFF800001, 0x7FBFFFFF, 0x7F7FFFFF, 0xFF7FFFFF,
             0x00000001, 0x00008000, 0x00018000, 0x00010000, 0x807FFFFF, 0x3EAAAAAB, 0xC0490FDB, 0x477FE000,
             0x477FF000, 0x33800000]
    kats["bf16_rne"] = [[x, bf16_rne_exact(x)] for x in cases]
    with open(os.path.join(HERE, "kats.json"), "w") as f:
        json.dump(kats, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
