"""Write the golden fixtures under tests/golden/ by exact-arithmetic brute force.

Why this exists: the reference ships no golden vectors for this path (its only kernel test,
tests/test_units.py:90-110, compares against MLX at run time, and MLX is not installed here).
These fixtures are therefore closed-form vectors, computed independently of oracle/qmm4_oracle.py:
  * codes are decoded from the little-endian BYTES of each word — byte j of word c holds
    k = 8c + 2j in its low nibble and k = 8c + 2j + 1 in its high nibble
    (src/mlx_tree_spec/qmm_packed.py:115-116) — not with the oracle's shifts;
  * bf16 and fp32 values are exact rationals (fractions.Fraction) decoded from their bit fields;
  * dequant is s*q + b in exact arithmetic, rounded to nearest-even fp32, then to nearest-even
    bf16, both with a rounding routine written here from the definition
    (the reference computes `T(float(q) * s + b)`: qmm_packed.py:200-201, 635-636);
  * the matmul reference is the exact rational sum of x * dequant(w) (tests/test_units.py:108
    defines it with fp32 accumulation; the exact sum is what fp32 accumulation approximates).

Run from the repository root:  python tests/golden/make_golden.py
Pure Python, seeded, deterministic; takes a few seconds.
"""

from __future__ import annotations

import os
import random
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


# ----------------------------------------------------------------------------- exact formats
def bits_value(bits: int, mant: int, expb: int):
    """Exact value of an IEEE-style binary float bit pattern (None for Inf/NaN)."""
    sign = -1 if (bits >> (mant + expb)) & 1 else 1
    e = (bits >> mant) & ((1 << expb) - 1)
    m = bits & ((1 << mant) - 1)
    bias = (1 << (expb - 1)) - 1
    if e == (1 << expb) - 1:
        return None
    if e == 0:
        return sign * Fraction(m, 1 << mant) * Fraction(2) ** (1 - bias)
    return sign * (1 + Fraction(m, 1 << mant)) * Fraction(2) ** (e - bias)


def floor_log2(a: Fraction) -> int:
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    return e


def round_even(q: Fraction) -> int:
    f = q.numerator // q.denominator
    r = q - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2 == 1):
        f += 1
    return f


def round_to_bits(v: Fraction, mant: int, expb: int) -> int:
    """Round an exact value to nearest-even in the format; returns the bit pattern."""
    bias = (1 << (expb - 1)) - 1
    sign_bit = 1 << (mant + expb)
    if v == 0:
        return 0
    sign = sign_bit if v < 0 else 0
    a = -v if v < 0 else v
    emin = 1 - bias
    e = max(floor_log2(a), emin)
    n = round_even(a / Fraction(2) ** (e - mant))
    if n >= (1 << (mant + 1)):
        n //= 2
        e += 1
    if e > bias:
        return sign | (((1 << expb) - 1) << mant)  # overflow to infinity
    if n < (1 << mant):
        return sign | n  # subnormal (e == emin)
    return sign | ((e + bias) << mant) | (n - (1 << mant))


def bf16v(bits: int):
    return bits_value(bits, 7, 8)


def f32v(bits: int):
    return bits_value(bits, 23, 8)


def dequant_one(sbits: int, bbits: int, q: int) -> int:
    """bf16 bits of bf16_rne(fp32_rne(s*q + b)) (an fp32 overflow stays infinite)."""
    v = bf16v(sbits) * q + bf16v(bbits)
    f = round_to_bits(v, 23, 8)
    fv = f32v(f)
    if fv is None:
        return ((f >> 16) & 0x8000) | 0x7F80
    return round_to_bits(fv, 7, 8)


def codes_from_bytes(word: int) -> list[int]:
    """The 8 codes of one word, decoded from its little-endian bytes."""
    out = []
    for byte in word.to_bytes(4, "little"):
        out.append(byte & 0xF)
        out.append(byte >> 4)
    return out


def bf16_bits_of(x: float) -> int:
    return round_to_bits(Fraction(x), 7, 8)


# ----------------------------------------------------------------------------- dequant table
def dequant_cases(rng: random.Random):
    """(s, b) bf16 pairs covering the arithmetic's corners; each used with all 16 codes."""
    pairs = []
    one, zero = bf16_bits_of(1.0), 0
    pairs += [(one, zero), (zero, bf16_bits_of(0.75)), (bf16_bits_of(-2.0), bf16_bits_of(3.0)),
              (bf16_bits_of(0.004), bf16_bits_of(-0.032)), (0x0001, 0x0001), (0x0080, 0x8001),
              (0x7F7F, 0x0000), (0x7F7F, 0xFF7F), (0x0040, 0x0000)]
    # Typical model groups: s = |N(0,1)|*0.004 + 1e-4, b = -8 s + N(0,1)*1e-3.
    for _ in range(160):
        s = abs(rng.gauss(0, 1)) * 0.004 + 1e-4
        sb = bf16_bits_of(s)
        b = -8 * float(bf16v(sb)) + rng.gauss(0, 1) * 1e-3
        pairs.append((sb, bf16_bits_of(b)))
    # Random bit patterns over wide exponent ranges (finite, both signs).
    while len(pairs) < 420:
        s = rng.getrandbits(16)
        b = rng.getrandbits(16)
        if ((s >> 7) & 0xFF) == 0xFF or ((b >> 7) & 0xFF) == 0xFF:
            continue
        pairs.append((s, b))
    # Double rounding: when s*q is exactly a bf16 midpoint and b is below half an fp32 ulp of
    # it, rounding to fp32 first lands on the tie and the bf16 result follows ties-to-even,
    # whereas rounding the exact value once would follow the sign of b.
    found = 0
    while found < 60:
        es = rng.randint(-40, 40)
        s = bf16_bits_of((1 + rng.getrandbits(7) / 128) * 2.0 ** es)
        q = rng.randint(1, 15)
        v = bf16v(s) * q
        e = floor_log2(v)
        t = v / Fraction(2) ** (e - 8)
        if t.denominator != 1 or t.numerator % 2 == 0:
            continue  # not a bf16 midpoint
        tiny = rng.choice([1, -1]) * (1 + rng.getrandbits(7) / 128) * 2.0 ** (e - 25 - rng.randint(0, 6))
        b = bf16_bits_of(tiny)
        if round_to_bits(bf16v(s) * q + bf16v(b), 7, 8) != dequant_one(s, b, q):
            pairs.append((s, b))
            found += 1
    return pairs


def write_dequant_table(rng: random.Random) -> None:
    pairs = dequant_cases(rng)
    s = np.array([p[0] for p in pairs], dtype=np.uint16)
    b = np.array([p[1] for p in pairs], dtype=np.uint16)
    out = np.zeros((len(pairs), 16), dtype=np.uint16)
    direct = np.zeros((len(pairs), 16), dtype=np.uint16)
    for i, (sb, bb) in enumerate(pairs):
        for q in range(16):
            out[i, q] = dequant_one(sb, bb, q)
            direct[i, q] = round_to_bits(bf16v(sb) * q + bf16v(bb), 7, 8)
    np.savez_compressed(os.path.join(HERE, "dequant_table.npz"), scales=s, biases=b, expected=out,
                        single_rounding=direct)
    print(f"dequant_table.npz: {len(pairs)} (s, b) pairs x 16 codes, "
          f"{int((out != direct).sum())} entries where fp32-then-bf16 differs from direct bf16")


# ----------------------------------------------------------------------------- matmul cases
# K % 128 == 0 and N % 16 == 0 except the last two, which only the oracle takes.
QMM_SHAPES = [(1, 128, 16), (3, 128, 32), (2, 256, 16), (16, 128, 48), (33, 128, 32), (5, 192, 32), (7, 64, 16)]


def write_qmm_cases(rng: random.Random) -> None:
    arrays = {}
    for ci, (m, k, n) in enumerate(QMM_SHAPES):
        x = np.array([[bf16_bits_of(rng.gauss(0, 1)) for _ in range(k)] for _ in range(m)], dtype=np.uint16)
        w = np.array([[rng.getrandbits(32) for _ in range(k // 8)] for _ in range(n)], dtype=np.uint32)
        s = np.zeros((n, k // 64), dtype=np.uint16)
        b = np.zeros((n, k // 64), dtype=np.uint16)
        for i in range(n):
            for g in range(k // 64):
                sv = abs(rng.gauss(0, 1)) * 0.004 + 1e-4
                s[i, g] = bf16_bits_of(sv)
                b[i, g] = bf16_bits_of(-8 * float(bf16v(int(s[i, g]))) + rng.gauss(0, 1) * 1e-3)
        deq = np.zeros((n, k), dtype=np.uint16)
        for i in range(n):
            for c in range(k // 8):
                codes = codes_from_bytes(int(w[i, c]))
                g = (8 * c) // 64
                for j in range(8):
                    deq[i, 8 * c + j] = dequant_one(int(s[i, g]), int(b[i, g]), codes[j])
        xv = [[bf16v(int(v)) for v in row] for row in x]
        wv = [[bf16v(int(v)) for v in row] for row in deq]
        exact = np.zeros((m, n), dtype=np.float64)
        ybf = np.zeros((m, n), dtype=np.uint16)
        for i in range(m):
            for j in range(n):
                acc = sum((xv[i][kk] * wv[j][kk] for kk in range(k)), Fraction(0))
                exact[i, j] = float(acc)
                ybf[i, j] = round_to_bits(acc, 7, 8)
        for name, arr in (("x", x), ("w", w), ("s", s), ("b", b), ("deq", deq), ("exact", exact), ("y", ybf)):
            arrays[f"c{ci}_{name}"] = arr
    arrays["shapes"] = np.array(QMM_SHAPES, dtype=np.int64)
    np.savez_compressed(os.path.join(HERE, "qmm_small.npz"), **arrays)
    print(f"qmm_small.npz: {len(QMM_SHAPES)} cases")


# ----------------------------------------------------------------------------- pack_nax indices
def write_pack_nax(rng: random.Random) -> None:
    """wq2[t][kb][r][j] = w[32t + r][2kb + j], sp2[t][g][r] = s[32t + r][g] (qmm_packed.py:224-231),
    with explicit index loops."""
    n, kw, g = 64, 8, 1
    w = np.array([[rng.getrandbits(32) for _ in range(kw)] for _ in range(n)], dtype=np.uint32)
    s = np.array([[rng.getrandbits(16) for _ in range(g)] for _ in range(n)], dtype=np.uint16)
    wq2 = []
    for t in range(n // 32):
        for kb in range(kw // 2):
            for r in range(32):
                for j in range(2):
                    wq2.append(int(w[32 * t + r, 2 * kb + j]))
    sp2 = []
    for t in range(n // 32):
        for gg in range(g):
            for r in range(32):
                sp2.append(int(s[32 * t + r, gg]))
    np.savez_compressed(os.path.join(HERE, "pack_nax.npz"), w=w, s=s,
                        wq2=np.array(wq2, dtype=np.uint32), sp2=np.array(sp2, dtype=np.uint16))
    print("pack_nax.npz written")


if __name__ == "__main__":
    write_dequant_table(random.Random(20261201))
    write_qmm_cases(random.Random(7))
    write_pack_nax(random.Random(11))
