"""Writes tests/golden/known_answers.json: exact-rational known answers for the W4 path's arithmetic.

The reference ships no golden vectors for this path (its GPU tests are manual tools with inline CPU references:
engine/tools/qa8_dbg.mm, gemm_dbg.mm, micro/qtest.mm). These vectors are computed here with Python's
fractions.Fraction, i.e. exactly, from the definitions the reference kernels implement:
  * MLX affine 4-bit layout: element j of a little-endian uint32 at bits 4j (engine/kernels/core.metal:13-15);
  * decode GEMV (qmv4, core.metal:85-171):        y = sum_k (s q + b) x                      (exact value);
  * prefill GEMM (MLX qmm, quantized.h:528-535):  y = sum_k bf16(fp32(s q + b)) x            (exact value);
  * activation quantizer (w4a8.metal:24-41):      sx = fp32(amax / 127), xq = rint(fp32(x / sx));
  * W4A8 (w4a8.metal:7-8, 78-87):                 y = sum_g [s sx P + b sx sum xq], P = sum_k q xq.
Rounding to fp32 / bf16 is done on the exact rationals with round-half-even, so the expected values carry no
floating-point summation error; the oracle (fp32 accumulation) must land within a small tolerance of them, and its
integer outputs (codes, xq, P) must match exactly.

Inputs come from a stated 32-bit LCG so the file can be regenerated bit-for-bit: `python tests/golden/make_golden.py`.
"""
from __future__ import annotations

import json
import os
import struct
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))


class LCG:
    """x <- (1664525 x + 1013904223) mod 2^32 (Numerical Recipes)."""

    def __init__(self, seed: int):
        self.x = seed & 0xFFFFFFFF

    def next(self) -> int:
        self.x = (1664525 * self.x + 1013904223) & 0xFFFFFFFF
        return self.x

    def uniform(self) -> Fraction:  # in [0, 1), 24-bit grid
        return Fraction(self.next() >> 8, 1 << 24)


def round_bits(v: Fraction, bits: int) -> Fraction:
    """Round a rational to `bits` significant bits, ties to even (normal range only)."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    # a in [2^e, 2^(e+1)); quantum 2^(e - bits + 1)
    q = Fraction(2) ** (e - bits + 1)
    n = a / q
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * fl * q


def to_f32(v: Fraction) -> Fraction:
    return round_bits(v, 24)


def to_bf16(v: Fraction) -> Fraction:
    return round_bits(v, 8)


def bf16_bits(v: Fraction) -> int:
    f = float(v)
    return struct.unpack("<I", struct.pack("<f", f))[0] >> 16


def rint_even(v: Fraction) -> int:
    fl = v.numerator // v.denominator
    rem = v - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl


def case(M: int, N: int, K: int, seed: int, bias: str):
    rng = LCG(seed)
    G = K // 64
    codes = [[rng.next() >> 28 for _ in range(K)] for _ in range(N)]
    s = [[to_bf16(Fraction(5, 1000) + Fraction(15, 1000) * rng.uniform()) for _ in range(G)] for _ in range(N)]
    if bias == "minus8":
        b = [[to_bf16(-8 * s[n][g]) for g in range(G)] for n in range(N)]
    else:
        b = [[to_bf16(Fraction(5, 100) * (2 * rng.uniform() - 1)) for g in range(G)] for n in range(N)]
    # activations: bf16 of a symmetric triangular variate in (-2, 2)
    x = [[to_bf16(2 * (rng.uniform() + rng.uniform() - 1)) for _ in range(K)] for _ in range(M)]

    def w_exact(n, k):
        return s[n][k // 64] * codes[n][k] + b[n][k // 64]

    qmv = [[float(sum(w_exact(n, k) * x[m][k] for k in range(K))) for n in range(N)] for m in range(M)]
    qmm = [[float(sum(to_bf16(to_f32(w_exact(n, k))) * x[m][k] for k in range(K))) for n in range(N)]
           for m in range(M)]
    out = {"M": M, "N": N, "K": K, "bias": bias,
           "codes": codes,
           "s_bf16": [[bf16_bits(v) for v in row] for row in s],
           "b_bf16": [[bf16_bits(v) for v in row] for row in b],
           "x_bf16": [[bf16_bits(v) for v in row] for row in x],
           "qmv": qmv, "qmm": qmm}
    for per_token in (0, 1):
        xq = [[0] * K for _ in range(M)]
        sxs = [[Fraction(0)] * G for _ in range(M)]
        for m in range(M):
            row_amax = max(abs(v) for v in x[m])
            for g in range(G):
                amax = row_amax if per_token else max(abs(v) for v in x[m][g * 64:(g + 1) * 64])
                sx = to_f32(amax / 127) if amax > 0 else Fraction(1)
                sxs[m][g] = sx
                for k in range(g * 64, (g + 1) * 64):
                    xq[m][k] = rint_even(to_f32(x[m][k] / sx))
        y = []
        for m in range(M):
            row = []
            for n in range(N):
                acc = Fraction(0)
                for g in range(G):
                    P = sum(codes[n][k] * xq[m][k] for k in range(g * 64, (g + 1) * 64))
                    Q = sum(xq[m][k] for k in range(g * 64, (g + 1) * 64))
                    acc += s[n][g] * sxs[m][g] * P + b[n][g] * sxs[m][g] * Q
                row.append(float(acc))
            y.append(row)
        key = "a8_token" if per_token else "a8_group"
        out[key] = {"xq": xq, "sx": [[float(v) for v in row] for row in sxs], "y": y}
    return out


def main():
    cases = [case(2, 3, 128, 1, "minus8"), case(3, 2, 192, 7, "free")]
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py", "cases": cases}, f)


if __name__ == "__main__":
    main()
