"""The integer identity the int8 GEMM (k_gemm_i8 / k_gemm_i8_full) is built
on, and its digit-plane window, checked by brute force with Python integers
(no GPU):

1. nine signed digits: u = v + C mod 2^64 (C = 0x0080808080808080),
   d_i = byte_i(u) - 128 for i <= 6, d_7 = byte_7(u) as int8, d_8 = 1 when
   v + C overflowed int64; then v = sum_{i<=7} d_i 256^i + 2^64 d_8 exactly;
2. products: bits [48, 112) of sum_k x_k w_k equal those of
   sum_{a+b<=13} 256^(a+b) P_ab, P_ab = sum_k d_a(x_k) d_b(w_k), with no
   correction terms (every accumulator fits int32 for K <= 16320);
3. the window: for X digits in planes 0..6 and W digits in planes
   LO - 1 .. LO + 3, the pairs (a <= 6, b in the window) alone give the same
   bits, and the conservative overflow test of the window split (the high
   word >= 0x7F7F7F7F) catches every value that overflows;
4. the epilogue: the 128-bit sum of 256^d Q_d from four exact int64 group
   sums and one carry.

A plausible slip (d_7 offset like the others, a missing plane-8 term, the
plane-8 flag from the wrong sign test, a window one plane short) fails one of
these cases.
"""
import random

C = 0x0080808080808080
M64 = (1 << 64) - 1
EDGE = [0, 1, -1, C, -C, -(1 << 63), (1 << 63) - 1, (1 << 63) - C, (1 << 63) - C - 1,
        0x7F7F7F7F00000000, 0x7F7F7F7EFFFFFFFF, 1 << 48, -(1 << 48), 1 << 55, -(1 << 55),
        0x8080808080808080 - (1 << 64)]


def s64(x):
    x &= M64
    return x - (1 << 64) if x >> 63 else x


def digits9(v):
    """The kernel's split: nine digits of v (d_8 the overflow flag)."""
    u = (v + C) & M64
    d = [((u >> (8 * i)) & 0xFF) - 128 for i in range(7)]
    b7 = u >> 56
    d.append(b7 - 256 if b7 >= 128 else b7)
    d.append(1 if (v >= 0 and s64(u) < 0) else 0)
    return d


def bits48_112(x):
    return (x >> 48) & M64


def pairs_dot(xs, ws, pairs):
    q = [0] * 14
    for x, w in zip(xs, ws):
        dx, dw = digits9(x), digits9(w)
        for a, b in pairs:
            q[a + b] += dx[a] * dw[b]
    return q, sum(v * 256 ** d for d, v in enumerate(q))


ALL = [(a, b) for a in range(9) for b in range(9) if a + b <= 13]


def test_digits_reconstruct_and_fit_int8():
    rng = random.Random(3)
    vals = EDGE + [rng.randrange(-(1 << 63), 1 << 63) for _ in range(20000)]
    vals += [rng.randrange((1 << 63) - C - 64, 1 << 63) for _ in range(500)]
    for v in vals:
        d = digits9(v)
        assert all(-128 <= x <= 127 for x in d[:8]) and d[8] in (0, 1), v
        assert sum(x * 256 ** i for i, x in enumerate(d[:8])) + (d[8] << 64) == v, v
    assert digits9(0) == [0] * 9
    assert digits9((1 << 63) - C)[8] == 1 and digits9((1 << 63) - C - 1)[8] == 0


def test_every_pair_gives_the_product_bits():
    rng = random.Random(5)
    for trial in range(400):
        k = rng.randint(1, 24)
        pick = lambda: rng.choice([rng.randrange(-(1 << 63), 1 << 63), rng.choice(EDGE),
                                   rng.randrange((1 << 63) - C, 1 << 63),
                                   rng.randrange(-(1 << 40), 1 << 40)])
        xs = [pick() for _ in range(k)]
        ws = [pick() for _ in range(k)]
        q, tot = pairs_dot(xs, ws, ALL)
        assert bits48_112(tot) == bits48_112(sum(x * w for x, w in zip(xs, ws))), trial
    # dropping the plane-8 pairs breaks a dot product holding an overflowed value
    xs, ws = [3 << 40], [(1 << 63) - 1]
    _, tot = pairs_dot(xs, ws, [(a, b) for a, b in ALL if a < 8 and b < 8])
    assert bits48_112(tot) != bits48_112(xs[0] * ws[0])


def test_accumulators_fit_int32_at_the_run_limit():
    """|Q_d| <= (full pairs) 2^14 K + (plane-8 pairs) 2^7 K < 2^31 at K = 16320."""
    K = 16320
    worst = 0
    for d in range(14):
        full = sum(1 for a, b in ALL if a + b == d and a < 8 and b < 8)
        small = sum(1 for a, b in ALL if a + b == d and (a == 8 or b == 8))
        worst = max(worst, (full * (1 << 14) + small * (1 << 7)) * K)
    assert worst < 1 << 31


def bf16ish(rng, scale):
    m = rng.randrange(128, 256) << max(0, scale + rng.randrange(-6, 1) - 7)
    return -m if rng.random() < 0.5 else m


def window_of(top):
    return min(max(top - 3, 0), 4)


def test_window_pairs_give_the_product_bits():
    """Weights with 8 significant bits and activations below 2^55: the window
    chosen from the top W plane covers every nonzero pair."""
    rng = random.Random(7)
    for trial in range(300):
        scale = rng.choice([20, 27, 35, 42, 50, 58])
        k = rng.randint(1, 32)
        ws = [bf16ish(rng, scale) for _ in range(k)]
        xs = [rng.randrange(-(1 << 54), 1 << 54) for _ in range(k)]
        wplanes = {b for w in ws for b, x in enumerate(digits9(w)) if x}
        xplanes = {a for x in xs for a, y in enumerate(digits9(x)) if y}
        assert max(xplanes, default=0) <= 6
        lo = window_of(max(wplanes, default=3))
        if not wplanes <= set(range(max(lo - 1, 0), lo + 4)):
            continue   # the kernel redoes such a block with every pair
        pairs = [(a, b) for a in range(7) for b in range(max(lo - 1, 0), lo + 4)]
        assert all(a + b <= 13 for a, b in pairs)
        _, tot = pairs_dot(xs, ws, pairs)
        assert bits48_112(tot) == bits48_112(sum(x * w for x, w in zip(xs, ws))), trial
    # one plane short (no LO - 1) misses a weight that reaches it
    ws, xs = [(200 << 36), 3 << 10], [5 << 30, 7 << 41]   # top plane 5: LO = 2, W plane 1
    lo = window_of(max(b for w in ws for b, x in enumerate(digits9(w)) if x))
    assert lo == 2
    short = [(a, b) for a in range(7) for b in range(lo, lo + 4)]
    full = [(a, b) for a in range(7) for b in range(max(lo - 1, 0), lo + 4)]
    want = bits48_112(sum(x * w for x, w in zip(xs, ws)))
    assert bits48_112(pairs_dot(xs, ws, full)[1]) == want
    assert bits48_112(pairs_dot(xs, ws, short)[1]) != want


def test_overflow_test_is_conservative():
    """Every value whose v + C overflows has a high word >= 0x7F7F7F7F."""
    rng = random.Random(9)
    lo = (1 << 63) - C
    for v in [lo, lo + 1, (1 << 63) - 1] + [rng.randrange(lo, 1 << 63) for _ in range(5000)]:
        assert digits9(v)[8] == 1
        assert (v >> 32) >= 0x7F7F7F7F
    for v in [rng.randrange(-(1 << 63), lo) for _ in range(5000)]:
        assert digits9(v)[8] == 0


def sum128_grouped(acc, carry=True, arith=True):
    """The kernels' epilogue (acc_sum128): four exact int64 group sums of
    four digit sums each, then S = g0 + 2^32 g1 + 2^64 g2 + 2^96 g3 as two
    64-bit words with one carry, every operation wrapped to 64 bits."""
    def s64(x):
        x &= M64
        return x - (1 << 64) if x >> 63 else x
    g = []
    for j in range(4):
        v = 0
        for e in range(3, -1, -1):
            d = 4 * j + e
            v = (v << 8) & M64
            if d < 14:
                v = (v + (acc[d] & M64)) & M64
        g.append(s64(v))
    lo = ((g[0] & M64) + ((g[1] << 32) & M64)) & M64
    c = 1 if carry and lo < (g[0] & M64) else 0
    g1hi = (g[1] >> 32) & M64 if arith else ((g[1] & M64) >> 32)
    hi = (((g[0] >> 63) & M64) + g1hi + c + (g[2] & M64) + ((g[3] << 32) & M64)) & M64
    return lo, hi


def test_epilogue_grouped_sum_is_the_128_bit_sum():
    """S mod 2^128 and the output word bits 48..111 from the grouped form
    equal the direct sum of 256^d acc_d for int32 digit sums, extremes
    included; dropping the carry or shifting g1 logically fails."""
    rng = random.Random(13)
    lim = (1 << 31) - 1
    cases = [[lim] * 14, [-(1 << 31)] * 14, [0] * 14, [-1] * 14,
             [lim if d % 2 else -(1 << 31) for d in range(14)]]
    cases += [[rng.randint(-(1 << 31), lim) for _ in range(14)] for _ in range(3000)]
    cases += [[rng.choice([0, 1, -1, lim, -(1 << 31)]) for _ in range(14)] for _ in range(1000)]
    M128 = (1 << 128) - 1
    bad_carry = bad_arith = 0
    for acc in cases:
        want = sum(a << (8 * d) for d, a in enumerate(acc)) & M128
        lo, hi = sum128_grouped(acc)
        assert (hi << 64 | lo) == want, acc
        out = ((hi << 16) | (lo >> 48)) & M64
        assert out == (want >> 48) & M64
        l2, h2 = sum128_grouped(acc, carry=False)
        bad_carry += (h2 << 64 | l2) != want
        l3, h3 = sum128_grouped(acc, arith=False)
        bad_arith += (h3 << 64 | l3) != want
    assert bad_carry > 100 and bad_arith > 100
