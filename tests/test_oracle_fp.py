"""The oracle's fp_math restatement against what pins it.

Pins: the reference's determinism golden hash (tests/determinism_golden.txt
of the reference, c0d933ea340452ec) and its 12 sub-hashes; per-function
vectors recorded from the compiled reference (tests/golden/fp.json); known
answers of the reference's fp_test.c; and closed forms (Python big-int
products and truncating quotients, trigonometric / exponential identities)
chosen so that a dropped term, a wrong sign or a floor-vs-truncate slip
fails one of them.
"""
import ctypes as C
import math
import random

import numpy as np

import oracle_lib as O
import spec
from conftest import GOLD, bf16_reference, golden

ONE = spec.ONE
SUB_ORDER = ["fp_mul", "fp_div", "fp_sqrt", "fp_sqrt_fast", "fp_inv_sqrt", "fp_exp", "fp_log",
             "fp_sincos_cos", "fp_sincos_sin", "fp_sigmoid", "fp_silu", "fp_rng"]


def test_determinism_gate_matches_reference_golden(oracle):
    g = golden("fp.json")
    subs = (C.c_uint64 * 12)()
    h = oracle.q48o_determinism(subs)
    assert "%016x" % h == g["determinism_golden"] == "c0d933ea340452ec"
    for i, name in enumerate(SUB_ORDER):
        assert "%016x" % subs[i] == g["sub_hashes"][name], name


def test_grid_restatements_agree(oracle):
    """C grid (oracle) == Python grid (spec) == 4230 values of build_grid."""
    buf = np.empty(5000, dtype=np.int64)
    n = oracle.q48o_det_grid(buf.ctypes.data, 5000)
    py = spec.det_grid()
    assert n == len(py) == golden("fp.json")["grid_inputs"] == 4230
    assert [int(v) for v in buf[:n]] == py


def _vec(oracle, name, x, y):
    f = lambda fn, arr: np.array([fn(int(a)) for a in arr], dtype=np.int64)  # noqa: E731
    if name == "mul":
        return np.array([oracle.q48o_fp_mul(int(a), int(b)) for a, b in zip(x, y)], dtype=np.int64)
    if name == "div":
        return np.array([oracle.q48o_fp_div(int(a), int(b)) if b != 0 else 0 for a, b in zip(x, y)],
                        dtype=np.int64)
    pos = [spec.pos_of(int(a)) for a in x]
    ex = [spec.exp_arg(int(a)) for a in x]
    if name in ("inv_sqrt", "sqrt", "log"):
        return f(getattr(oracle, "q48o_fp_" + name), pos)
    if name in ("exp", "safe_exp"):
        return f(getattr(oracle, "q48o_fp_" + name), ex)
    if name in ("sigmoid", "silu"):
        return f(getattr(oracle, "q48o_fp_" + name), x)
    c, s = C.c_int64(), C.c_int64()
    out = []
    for a in x:
        oracle.q48o_fp_sincos(int(a), C.byref(c), C.byref(s))
        out.append(c.value if name == "cos" else s.value)
    return np.array(out, dtype=np.int64)


def test_fp_vectors_match_reference(oracle):
    g = golden("fp.json")["vectors"]["fnv"]
    x, y = spec.fp_inputs()
    for name, want in g.items():
        assert O.fnv(_vec(oracle, name, x, y)) == want, name


def test_cordic_constants_match_reference(oracle):
    g = golden("fp.json")["consts"]
    pi, gain = C.c_int64(), C.c_int64()
    ang = np.empty(48, dtype=np.int64)
    oracle.q48o_fp_consts(C.byref(pi), C.byref(gain), ang.ctypes.data)
    assert pi.value == g["pi"] and gain.value == g["gain"]
    assert [int(a) for a in ang] == g["angles"]
    # fp_test.c:613: gain ~ 0.607252935 (170926505739103); pi to ~13 digits
    assert abs(gain.value - 170926505739103) < 1000
    assert abs(pi.value / ONE - math.pi) < 1e-12


def test_fp_test_known_answers(oracle):
    """Exact equalities of fp_test.c:298-299, 347-358."""
    assert oracle.q48o_fp_safe_exp(100 * ONE) == oracle.q48o_fp_exp(10 * ONE)
    assert oracle.q48o_fp_safe_exp(-11 * ONE) == 0
    assert oracle.q48o_fp_inv_sqrt(0) == 0 and oracle.q48o_fp_inv_sqrt(-ONE) == 0
    assert oracle.q48o_fp_exp(0) == ONE
    assert oracle.q48o_fp_log(0) == -50 * ONE


def _c_trunc_div(a: int, b: int) -> int:
    q = abs(a) // abs(b)
    return q if (a < 0) == (b < 0) else -q


def test_mul_div_closed_forms(oracle):
    """fp_mul = floor(a b / 2^48) and fp_div = trunc(a 2^48 / b), both cut
    to int64, on random and extreme operands (brute force, Python ints)."""
    rnd = random.Random(7)
    ext = [spec.INT64_MIN, spec.INT64_MAX, -1, 1, ONE, -ONE, 3, -3]
    vals = ext + [rnd.randrange(spec.INT64_MIN, spec.INT64_MAX) for _ in range(400)] + \
        [rnd.randrange(-40 * ONE, 40 * ONE) for _ in range(400)]
    for a in vals:
        b = rnd.choice(vals)
        assert oracle.q48o_fp_mul(a, b) == spec.wrap64((a * b) >> 48)
        if b != 0:
            assert oracle.q48o_fp_div(a, b) == spec.wrap64(_c_trunc_div(a << 48, b)), (a, b)


def test_math_identities(oracle):
    """cos^2 + sin^2 = 1, exp(log x) = x, sigmoid(x) + sigmoid(-x) = 1,
    inv_sqrt(x)^2 x = 1 — to the documented precision."""
    rnd = random.Random(3)
    c, s = C.c_int64(), C.c_int64()
    for _ in range(300):
        a = rnd.randrange(-100 * ONE, 100 * ONE)
        oracle.q48o_fp_sincos(a, C.byref(c), C.byref(s))
        assert abs(c.value / ONE - math.cos(a / ONE)) < 1e-9
        assert abs(s.value / ONE - math.sin(a / ONE)) < 1e-9
    for _ in range(200):
        x = rnd.randrange(ONE // 1000, 1000 * ONE)
        assert abs(oracle.q48o_fp_exp(oracle.q48o_fp_log(x)) / x - 1) < 1e-9
        r = oracle.q48o_fp_inv_sqrt(x) / ONE
        assert abs(r * r * x / ONE - 1) < 1e-9
        v = rnd.randrange(-10 * ONE, 10 * ONE)
        assert abs(oracle.q48o_fp_sigmoid(v) + oracle.q48o_fp_sigmoid(-v) - ONE) < 64
        # dyadic (1 + x/2^14)^(2^14): relative error ~ x^2 / 2^15
        t = v / ONE
        assert abs(oracle.q48o_fp_exp(v) / ONE / math.exp(t) - 1) < t * t / 2 ** 14 + 1e-9


def test_bf16_conversion_equals_reference_every_pattern(oracle):
    """The host's conversion (q48s_bf16_to_q48, used by the synthetic models
    and as the checker of the device expansion) equals the compiled
    reference's bfloat16_to_q1648 on all 65536 patterns: zero and subnormal
    exponents, the exponent-255 clamp, shifts of 64 bits or more and wrapping
    left shifts included."""
    want = bf16_reference()
    assert O.fnv(want) == golden("bf16_to_q48.json")["fnv"]
    got = np.array([oracle.q48s_bf16_to_q48(b) for b in range(1 << 16)], dtype=np.int64)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [hex(int(b)) for b in bad[:8]]


def test_f16_conversion_equals_reference_every_pattern(oracle):
    """The host's half-precision conversion (q48s_f16_to_q48) equals the
    compiled reference's float16_to_q1648 (safetensors.h:74-111) on all 65536
    patterns (tests/golden/f16_to_q48.npz), and the normal and subnormal
    ranges follow the closed form (1024 + m) 2^(e + 23), m 2^24 (wrapping at
    exponent 30, where the value reaches bit 63)."""
    import numpy as np
    meta = golden("f16_to_q48.json")
    with np.load(GOLD / meta["file"], allow_pickle=False) as z:
        want = z["v"]
    assert want.dtype == np.int64 and want.size == 65536 and O.fnv(want) == meta["fnv"]
    got = np.array([oracle.q48s_f16_to_q48(b) for b in range(1 << 16)], dtype=np.int64)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [hex(int(b)) for b in bad[:8]]
    for bits in range(0, 1 << 16, 5):
        e, m, sgn = (bits >> 10) & 0x1F, bits & 0x3FF, bits >> 15
        if e == 0x1F:
            continue
        v = (1024 + m) << (e + 23) if e else m << 24
        assert int(want[bits]) == spec.wrap64(-v if sgn else v), hex(bits)


def test_bf16_conversion(oracle):
    """bfloat16_to_q1648 (safetensors.h:115-152): every normal bf16 in range
    converts exactly (closed form), and q48 -> bf16 -> q48 rounds to nearest."""
    for bits in range(0, 1 << 16, 7):
        e, m, sgn = (bits >> 7) & 0xFF, bits & 0x7F, bits >> 15
        v = oracle.q48s_bf16_to_q48(bits)
        if e == 0:
            want = 0
        elif e == 0xFF:
            want = 32000 << 48
        else:
            sh = e - 86
            want = ((128 + m) << sh if sh >= 0 else (128 + m) >> -sh) if -64 < sh < 64 else 0
            want = spec.wrap64(want)
        assert v == spec.wrap64(-want if sgn else want), bits
    rnd = random.Random(11)
    for _ in range(2000):
        q = rnd.randrange(-ONE * 100, ONE * 100)
        r = oracle.q48s_bf16_to_q48(oracle.q48s_q48_to_bf16(q))
        if q == 0:
            assert r == 0
            continue
        ulp = 1 << max(0, abs(q).bit_length() - 8)
        assert abs(r - q) * 2 <= ulp
        assert r == 0 or (r >> max(0, abs(r).bit_length() - 8)) << max(0, abs(r).bit_length() - 8) == r
