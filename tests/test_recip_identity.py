"""The exact FP64 forms of fp_exp's squarings, of fp_div(ONE, r) and of a
softmax row's fp_div(e, sum) (csrc/q48_device.hpp: q48_exp_small, q48_recip,
q48_divisor_of / q48_div_by), restated step by step in Python with every FP64
operation rounded as the device rounds it (products and sums by Python floats,
fused multiply-adds through exact rationals), checked against integer
arithmetic (no GPU):

1. the first 12 of fp_exp's 14 squarings r_k = floor(r_{k-1}^2 / 2^48) of
   r_0 = ONE + (|x| >> 14), |x| <= 10 ONE, as f + floor(fma(r, r 2^-48, -f)),
   f = floor(r * (r 2^-48)), stay exact integers;
2. floor(2^96 / r) for 2^48 <= r < 2^63 from the reciprocal, two Newton steps,
   round(y 2^96) - 1 and one compare of the low remainder word, whatever
   first approximation within 2^-20 the hardware gives;
3. floor(e 2^48 / d) for 0 <= e <= min(d, 2^52 - 1), 1 <= d < 2^62, from 2^48 / d
   prepared once, the same way.

Each check also catches a plausible slip: one Newton step with a 2^-20 first
approximation, or the compare dropped, gives wrong quotients here.
"""
import math
import random
from fractions import Fraction

ONE = 1 << 48


def fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))


def word(x):   # the FP64 word of x as an unsigned integer
    import struct
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def round_m1(v):
    """The kernel's q48_round_m1: word(v + 2^52) - word(2^52) - 1 (mod 2^64)."""
    return (word(v + 2.0 ** 52) - 0x4330000000000001) & ((1 << 64) - 1)


def newton2(d, y0):
    y = y0
    for _ in range(2):
        y = fma(y, fma(-d, y, 1.0), y)
    return y


def recip(r, rel, steps=2, compare=True):
    u = r
    rd = float(u)                     # correctly rounded, as the device's conversion
    y = (1.0 / rd) * (1.0 + rel)      # a first approximation within |rel|
    for _ in range(steps):
        y = fma(y, fma(-rd, y, 1.0), y)
    q0 = round_m1(y * 2.0 ** 96)
    rem = (-q0 * u) & ((1 << 64) - 1)
    up = compare and rem >= u
    if rem - (u if up else 0) >= u:
        return None                   # the kernel's fallback to the general division
    return (q0 + up) & ((1 << 64) - 1)


def div_by(e, d, rel):
    dd = float(d)
    y48 = newton2(dd, (1.0 / dd) * (1.0 + rel)) * 2.0 ** 48
    ed = float(e)                     # exact: e < 2^52
    q0 = round_m1(ed * y48)
    rem = ((e << 48) - q0 * d) & ((1 << 64) - 1)
    up = rem >= d
    if rem - (d if up else 0) >= d:
        return None
    return (q0 + up) & ((1 << 64) - 1)


def test_fp64_squarings_are_exact():
    rng = random.Random(1)
    ms = [0, 1, 10 * ONE, 10 * ONE - 1, ONE, 5 * ONE] + [rng.randrange(0, 10 * ONE + 1)
                                                         for _ in range(3000)]
    for m in ms:
        r = ONE + (m >> 14)
        rd = float(r)
        for _ in range(12):
            ref = (r * r) >> 48
            rs = rd * 2.0 ** -48
            f = math.floor(rd * rs)
            rd = f + math.floor(fma(rd, rs, -f))
            assert rd == ref and rd < 2.0 ** 52, m
            r = ref


def test_recip_quotients():
    rng = random.Random(2)
    rs = [ONE, ONE + 1, (1 << 63) - 1, (1 << 62), int(22026.47 * ONE)]
    rs += [rng.randrange(ONE, 1 << 63) for _ in range(3000)]
    rs += [(1 << 96) // q + dd for q in (rng.randrange(1 << 33, 1 << 48) for _ in range(1000))
           for dd in (-1, 0, 1)]
    rs = [r for r in rs if ONE <= r < 1 << 63]
    for i, r in enumerate(rs):
        rel = (rng.random() - 0.5) * 2.0 ** -19   # up to 2^-20 either way
        assert recip(r, rel) == (1 << 96) // r, r
    # one Newton step from a 2^-20 approximation is not enough somewhere
    bad = sum(recip(r, 2.0 ** -20, steps=1) != (1 << 96) // r for r in rs[:800])
    assert bad > 0
    # without the final compare, about half the quotients come out one short
    short = sum(recip(r, 0.0, compare=False) != (1 << 96) // r for r in rs[:800])
    assert short > 100


def test_prepared_divisor_quotients():
    rng = random.Random(3)
    cases = []
    for _ in range(3000):
        d = max(1, rng.randrange(1, 1 << 62) >> rng.randrange(0, 62))
        lim = min(d, (1 << 52) - 1)
        cases.append((rng.randrange(0, lim + 1), d))
    for _ in range(1000):   # softmax rows: e <= ONE <= sum
        cases.append((rng.randrange(0, ONE + 1), rng.randrange(ONE, 4097 * ONE)))
    for _ in range(1000):   # next to exact quotients
        d = rng.randrange(1, 1 << 62)
        q = rng.randrange(0, ONE + 1)
        e = min((q * d) >> 48, min(d, (1 << 52) - 1))
        cases += [(max(e + dd, 0), d) for dd in (-1, 0, 1)]
    cases += [(0, 1), (1, 1), ((1 << 52) - 1, (1 << 52) - 1), (ONE, ONE), (0, (1 << 62) - 1),
              ((1 << 52) - 1, (1 << 62) - 1)]
    for e, d in cases:
        if e > min(d, (1 << 52) - 1):
            continue
        rel = (rng.random() - 0.5) * 2.0 ** -19
        assert div_by(e, d, rel) == (e << 48) // d, (e, d)
