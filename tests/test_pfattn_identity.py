"""The two integer identities the matrix-core prefill attention (k_pfa) is
built on, checked by brute force with Python integers (no GPU):

1. digits: sum_k x_k w_k = sum_{a+b<=13} 256^(a+b) P_ab + C sum x + C sum w - n C^2
   (mod 2^112), with S(v) the bytes of v ^ C as int8 except the top byte,
   also when some entries are the value C (all digits zero: pad positions
   and pad dims of the kernel);
2. truncated products: sum_j floor(p_j v_j / 2^48)
   = floor((sum_j p_j v_j - 2^24 sum_j t_j) / 2^48) (mod 2^64), t_j the
   24-bit limb term (a0 b1 + a1 b0 + floor(a0 b0 / 2^24)) mod 2^24 of
   a = p mod 2^48, b = v mod 2^48.

A plausible slip (the top byte offset like the others, a dropped carry
term, 2^24 t_j without the floor term) fails one of these cases.
"""
import random

C = 0x0080808080808080
M24 = (1 << 24) - 1
EDGE = [0, 1, -1, C, -(1 << 63), (1 << 63) - 1, 1 << 48, (1 << 48) - 1, -(1 << 48),
        1 << 24, (1 << 24) - 1, 0x7F7F7F7F7F7F7F7F, 0x8080808080808080 - (1 << 64)]


def s64(x):
    x &= (1 << 64) - 1
    return x - (1 << 64) if x >> 63 else x


def digits(v):
    """int8 digits s_0..s_7 of v: bytes of v ^ C, top byte v's own."""
    u = (v & ((1 << 64) - 1)) ^ C
    out = []
    for i in range(8):
        b = (u >> (8 * i)) & 0xFF
        out.append(b - 256 if b >= 128 else b)
    return out


def digit_dot(xs, ws):
    dx = [digits(x) for x in xs]
    dw = [digits(w) for w in ws]
    acc = [0] * 14
    for a in range(8):
        for b in range(8):
            if a + b <= 13:
                acc[a + b] += sum(p[a] * q[b] for p, q in zip(dx, dw))
    n = len(xs)
    tot = sum(acc[d] << (8 * d) for d in range(14)) + C * sum(xs) + C * sum(ws) - n * C * C
    return tot % (1 << 112)


def t_term(p, v):
    a, b = p & ((1 << 48) - 1), v & ((1 << 48) - 1)
    a0, a1, b0, b1 = a & M24, a >> 24, b & M24, b >> 24
    return (a0 * b1 + a1 * b0 + ((a0 * b0) >> 24)) & M24


def draw(rng, edge_share=0.3):
    if rng.random() < edge_share:
        return rng.choice(EDGE)
    return rng.choice([rng.randrange(-(1 << 63), 1 << 63), rng.randrange(-(1 << 50), 1 << 50)])


def test_digit_identity_with_pads():
    rng = random.Random(3)
    for trial in range(400):
        n = rng.choice([1, 2, 5, 16, 64, 200])
        xs = [draw(rng) for _ in range(n)]
        ws = [draw(rng) for _ in range(n)]
        # pads: the value C on either side (zero digits)
        for i in range(n):
            if rng.random() < 0.1:
                xs[i] = C
        exact = sum(x * w for x, w in zip(xs, ws)) % (1 << 112)
        assert digit_dot(xs, ws) == exact, trial


def test_digit_identity_all_min():
    """every digit -128: the accumulators' largest magnitudes"""
    xs = [-(1 << 63)] * 64
    assert digit_dot(xs, xs) == sum(x * x for x in xs) % (1 << 112)


def test_truncated_product_sum():
    rng = random.Random(1)
    for trial in range(600):
        n = rng.choice([1, 2, 3, 17, 64, 300])
        ps = [rng.choice([rng.randrange(0, 1 << 49), rng.randrange(0, 1 << 63), 0, 1 << 48,
                          (1 << 48) - 1, (1 << 24) - 1]) for _ in range(n)]
        vs = [draw(rng) for _ in range(n)]
        want = s64(sum((p * v) >> 48 for p, v in zip(ps, vs)))
        X = sum(p * v for p, v in zip(ps, vs)) % (1 << 112)
        lam = sum(t_term(p, v) for p, v in zip(ps, vs))
        assert s64((X - (lam << 24)) >> 48) == want, trial


def test_truncated_product_needs_the_carry_term():
    """dropping floor(a0 b0 / 2^24) from t_j gives a different sum"""
    p, v = (1 << 48) - 1, (1 << 48) - 1
    t_bad = (((p & M24) * (v >> 24 & M24)) + ((p >> 24 & M24) * (v & M24))) & M24
    X = p * v
    assert s64((X - (t_term(p, v) << 24)) >> 48) == s64((p * v) >> 48)
    assert s64((X - (t_bad << 24)) >> 48) != s64((p * v) >> 48)
