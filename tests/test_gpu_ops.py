"""GPU parity of every op of libintllm_hip against the oracle and the
golden vectors recorded from the reference — bit-exact (integer work).

Each test prints the case it is about to run (flushed) before the device
call, so a failure names its case even from a truncated log.
"""
import ctypes as C

import numpy as np
import pytest

import intllm
import oracle_lib as O
import spec
from conftest import bf16_reference, golden

pytestmark = pytest.mark.gpu
ONE = spec.ONE
SUB_ORDER = ["fp_mul", "fp_div", "fp_sqrt", "fp_sqrt_fast", "fp_inv_sqrt", "fp_exp", "fp_log",
             "fp_sincos_cos", "fp_sincos_sin", "fp_sigmoid", "fp_silu", "fp_rng"]


def say(*a):
    print("[case]", *a, flush=True)


def dev_eval(ctx, func, x, y=None, two=False):
    n = len(x)
    dx = ctx.to_device(x)
    dy = ctx.to_device(y) if y is not None else None
    o0 = ctx.buffer(n)
    o1 = ctx.buffer(n) if two else None
    ctx.fp_eval(func, dx.ptr, dy.ptr if dy else None, o0.ptr, o1.ptr if o1 else None, n)
    r0 = o0.download()
    r1 = o1.download() if two else None
    for b in (dx, dy, o0, o1):
        if b is not None:
            b.free()
    return (r0, r1) if two else r0


def test_device_determinism_gate(ctx):
    """The gate of fp_determinism.c evaluated by the device fp_math: all 11
    function sub-hashes and the combined hash (the RNG sub-hash is host
    state, not device math) equal the reference golden."""
    g = golden("fp.json")
    grid = spec.det_grid()
    n = len(grid)
    x = np.array(grid, dtype=np.int64)
    y = np.array([grid[(i * 7 + 3) % n] for i in range(n)], dtype=np.int64)
    pos = np.array([spec.pos_of(int(v)) for v in grid], dtype=np.int64)
    ex = np.array([spec.exp_arg(int(v)) for v in grid], dtype=np.int64)
    say("determinism grid", n)
    got = {}
    got["fp_mul"] = O.fnv(dev_eval(ctx, intllm.FP_MUL, x, y))
    d = dev_eval(ctx, intllm.FP_DIV, x, y)
    got["fp_div"] = O.fnv(d[y != 0])
    got["fp_sqrt"] = O.fnv(dev_eval(ctx, intllm.FP_SQRT, pos))
    got["fp_sqrt_fast"] = O.fnv(dev_eval(ctx, intllm.FP_SQRT_FAST, pos))
    got["fp_inv_sqrt"] = O.fnv(dev_eval(ctx, intllm.FP_INV_SQRT, pos))
    got["fp_exp"] = O.fnv(dev_eval(ctx, intllm.FP_EXP, ex))
    got["fp_log"] = O.fnv(dev_eval(ctx, intllm.FP_LOG, pos))
    c, s = dev_eval(ctx, intllm.FP_SINCOS, x, two=True)
    got["fp_sincos_cos"], got["fp_sincos_sin"] = O.fnv(c), O.fnv(s)
    got["fp_sigmoid"] = O.fnv(dev_eval(ctx, intllm.FP_SIGMOID, x))
    got["fp_silu"] = O.fnv(dev_eval(ctx, intllm.FP_SILU, x))
    got["fp_rng"] = g["sub_hashes"]["fp_rng"]
    for k in SUB_ORDER:
        assert got[k] == g["sub_hashes"][k], k
    comb = np.array([int(got[k], 16) for k in SUB_ORDER], dtype=np.uint64).view(np.int64)
    assert O.fnv(comb) == g["determinism_golden"]


def test_device_fp_vectors_with_extremes(ctx):
    g = golden("fp.json")["vectors"]["fnv"]
    x, y = spec.fp_inputs()
    pos = np.array([spec.pos_of(int(v)) for v in x], dtype=np.int64)
    ex = np.array([spec.exp_arg(int(v)) for v in x], dtype=np.int64)
    say("fp vectors", len(x))
    assert O.fnv(dev_eval(ctx, intllm.FP_MUL, x, y)) == g["mul"]
    assert O.fnv(np.where(y != 0, dev_eval(ctx, intllm.FP_DIV, x, y), 0)) == g["div"]
    assert O.fnv(dev_eval(ctx, intllm.FP_INV_SQRT, pos)) == g["inv_sqrt"]
    assert O.fnv(dev_eval(ctx, intllm.FP_SQRT, pos)) == g["sqrt"]
    assert O.fnv(dev_eval(ctx, intllm.FP_LOG, pos)) == g["log"]
    assert O.fnv(dev_eval(ctx, intllm.FP_EXP, ex)) == g["exp"]
    assert O.fnv(dev_eval(ctx, intllm.FP_SAFE_EXP, ex)) == g["safe_exp"]
    c, s = dev_eval(ctx, intllm.FP_SINCOS, x, two=True)
    assert O.fnv(c) == g["cos"] and O.fnv(s) == g["sin"]
    assert O.fnv(dev_eval(ctx, intllm.FP_SIGMOID, x)) == g["sigmoid"]
    assert O.fnv(dev_eval(ctx, intllm.FP_SILU, x)) == g["silu"]


def test_device_div_random_vs_oracle(ctx, oracle):
    rng = np.random.default_rng(21)
    a = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=4096, dtype=np.int64)
    b = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=4096, dtype=np.int64)
    b[:64] = rng.integers(-1000, 1000, size=64)      # tiny divisors: quotient overflows
    b[64] = -1
    a[65] = spec.INT64_MIN
    b[65] = -1
    b[b == 0] = 7
    say("div random", a.size)
    d = dev_eval(ctx, intllm.FP_DIV, a, b)
    want = np.array([oracle.q48o_fp_div(int(p), int(q)) for p, q in zip(a, b)], dtype=np.int64)
    assert np.array_equal(d, want)
    # log-uniform magnitudes: every quotient size from 0 to 2^111 bits
    n = 8192
    ea, eb = rng.integers(0, 64, size=n), rng.integers(0, 64, size=n)
    a = np.array([spec.wrap64(int(rng.integers(0, 1 << 62)) >> (62 - min(int(e), 62))) for e in ea],
                 dtype=np.int64) * rng.choice([-1, 1], size=n)
    b = np.array([max(1, int(rng.integers(0, 1 << 62)) >> (62 - min(int(e), 62))) for e in eb],
                 dtype=np.int64) * rng.choice([-1, 1], size=n)
    say("div log-uniform", n)
    d = dev_eval(ctx, intllm.FP_DIV, a, b)
    want = np.array([oracle.q48o_fp_div(int(p), int(q)) for p, q in zip(a, b)], dtype=np.int64)
    assert np.array_equal(d, want)


def test_device_inv_sqrt_vs_oracle(ctx, oracle):
    """fp_inv_sqrt on the device (Newton steps on exact FP64 products) equals
    the oracle: every magnitude 2^0 .. 2^62 log-uniformly, the rmsnorm range
    around ONE, and one unit either side of each power of two, where the
    normalised argument crosses 2^48, 2^49 and 2^50."""
    rng = np.random.default_rng(29)
    n = 65536
    e = rng.integers(0, 63, size=n)
    x = [max(1, int(rng.integers(0, 1 << 62)) >> (62 - int(k))) for k in e]
    x += [int(v) for v in rng.integers(1 << 46, 1 << 51, size=16384)]
    for k in range(63):
        for d in (-1, 0, 1):
            v = (1 << k) + d
            if 0 < v < 1 << 63:
                x.append(v)
    x += [spec.INT64_MAX, spec.INT64_MAX - 1, 0, -1, spec.INT64_MIN]
    x = np.array(x, dtype=np.int64)
    say("inv_sqrt", x.size)
    got = dev_eval(ctx, intllm.FP_INV_SQRT, x)
    want = np.array([oracle.q48o_fp_inv_sqrt(int(v)) for v in x], dtype=np.int64)
    assert np.array_equal(got, want)


def test_device_safe_exp_sigmoid_silu_vs_oracle(ctx, oracle):
    """fp_safe_exp (squarings partly on exact FP64), fp_sigmoid and fp_silu
    on the device equal the oracle: uniform over [-11, 11] ONE, small
    magnitudes, and a few units either side of 0 and of the +-10 ONE clamps."""
    rng = np.random.default_rng(31)
    one, ten = 1 << 48, 10 << 48
    x = [int(v) for v in rng.integers(-11 * one, 11 * one, size=32768)]
    x += [int(v) >> int(s) for v, s in zip(rng.integers(-ten, ten, size=8192),
                                           rng.integers(0, 48, size=8192))]
    for c in (0, ten, -ten, one, -one):
        x += [c + d for d in range(-40, 41)]
    # within 0.05 ONE of the clamps: the largest squarings (e^|x| ONE near
    # 2^62.4) and the smallest reciprocals
    x += [int(v) for v in rng.integers(ten - one // 20, ten + 1, size=4096)]
    x += [int(v) for v in rng.integers(-ten, -ten + one // 20, size=4096)]
    x += [spec.INT64_MAX, spec.INT64_MIN]
    x = np.array(x, dtype=np.int64)
    say("safe_exp / sigmoid / silu", x.size)
    for fn, ref in ((intllm.FP_SAFE_EXP, oracle.q48o_fp_safe_exp),
                    (intllm.FP_SIGMOID, oracle.q48o_fp_sigmoid),
                    (intllm.FP_SILU, oracle.q48o_fp_silu)):
        got = dev_eval(ctx, fn, x)
        want = np.array([ref(int(v)) for v in x], dtype=np.int64)
        assert np.array_equal(got, want), fn


def test_device_div_quotients_at_integers(ctx, oracle):
    """Numerators at and one unit either side of exact multiples of the
    divisor (a 2^48 = q b): the quotient's estimate lands next to an integer,
    where an estimate off by one is caught only by the remainder steps; and
    softmax's e / sum, sigmoid's ONE / (ONE + e) shapes."""
    rng = np.random.default_rng(23)
    a, b = [], []
    for _ in range(2048):
        s = int(rng.integers(48, 62))
        c = int(rng.integers(1, 1 << (62 - s)))
        q = int(rng.integers(0, 1 << 52)) >> int(rng.integers(0, 52))
        base = q * c << (s - 48)
        if base >= 1 << 63:
            continue
        for d in (-1, 0, 1):
            v = base + d
            if 0 <= v < 1 << 63:
                sg = int(rng.choice([-1, 1]))
                a.append(sg * v)
                b.append(int(rng.choice([-1, 1])) * (c << s))
    one = 1 << 48
    for _ in range(2048):
        tot = int(rng.integers(one, 4096 * one))
        a.append(int(rng.integers(0, one + 1)))
        b.append(tot)
        a.append(one)
        b.append(one + int(rng.integers(0, 22027 * one)))
    a = np.array(a, dtype=np.int64)
    b = np.array(b, dtype=np.int64)
    say("div at integer quotients", a.size)
    d = dev_eval(ctx, intllm.FP_DIV, a, b)
    want = np.array([oracle.q48o_fp_div(int(p), int(q)) for p, q in zip(a, b)], dtype=np.int64)
    bad = np.nonzero(d != want)[0]
    assert bad.size == 0, [(int(a[i]), int(b[i]), int(d[i]), int(want[i])) for i in bad[:5]]


def test_device_div_prepared_divisor_vs_oracle(ctx, oracle):
    """The softmax rows' quotient (a reciprocal prepared once per divisor, one
    FP64 product and one remainder compare per element) equals fp_div: inside
    its range (0 <= e <= min(d, 2^52 - 1), 1 <= d < 2^62), at the range's
    edges (e = lim and lim + 1, d = 2^62 - 1 and 2^62, d = 1), near exact
    quotients, and outside it (negative or larger e, d < 1, d >= 2^62), where
    the general division answers."""
    rng = np.random.default_rng(37)
    one, top = 1 << 48, 1 << 62
    a, b = [], []

    def lim(d):
        return min(d, (1 << 52) - 1)

    for _ in range(8192):
        sh = int(rng.integers(0, 62))
        d = max(1, int(rng.integers(0, 1 << 62)) >> sh)
        a.append(int(rng.integers(0, lim(d) + 1)))
        b.append(d)
    for _ in range(4096):          # softmax shapes: e <= ONE <= sum
        a.append(int(rng.integers(0, one + 1)))
        b.append(int(rng.integers(one, 4097 * one)))
    for _ in range(2048):          # near exact quotients q = e 2^48 / d
        d = int(rng.integers(1, top))
        q = int(rng.integers(0, one + 1))
        e = (q * d) >> 48
        for dd in (-1, 0, 1):
            if 0 <= e + dd <= lim(d):
                a.append(e + dd)
                b.append(d)
    for d in (1, 2, 3, one - 1, one, one + 1, (1 << 52) - 1, 1 << 52, (1 << 52) + 1,
              top - 1, top, top + 1, spec.INT64_MAX):
        for e in (0, 1, lim(d) - 1, lim(d), lim(d) + 1, one, -1, -one, spec.INT64_MIN,
                  spec.INT64_MAX):
            a.append(e)
            b.append(d)
    for _ in range(2048):          # outside the range: negative e or d, e > d
        a.append(int(rng.integers(spec.INT64_MIN, spec.INT64_MAX)))
        b.append(int(rng.integers(spec.INT64_MIN, spec.INT64_MAX)) or 5)
    a = np.array([spec.wrap64(v) for v in a], dtype=np.int64)
    b = np.array(b, dtype=np.int64)
    say("div prepared divisor", a.size)
    got = dev_eval(ctx, intllm.FP_DIV_ROW, a, b)
    want = np.array([oracle.q48o_fp_div(int(p), int(q)) for p, q in zip(a, b)], dtype=np.int64)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(int(a[i]), int(b[i]), int(got[i]), int(want[i])) for i in bad[:5]]


def gemv_dev(ctx, W, x, M, K, w_offset=0):
    dW = ctx.buffer(M * K + w_offset)
    if w_offset:
        pad = np.zeros(w_offset, dtype=np.int64)
        dW.upload(np.concatenate([pad, np.asarray(W, dtype=np.int64)]))
    else:
        dW.upload(W)
    dx = ctx.to_device(x)
    dy = ctx.buffer(M)
    ctx.gemv(dy.ptr, dW.at(w_offset), dx.ptr, M, K)
    y = dy.download()
    for b in (dW, dx, dy):
        b.free()
    return y


def test_gemv_edges(ctx):
    g = golden("gemv.json")["edges"]
    for (M, K, W, x), e in zip(spec.gemv_edge_cases(), g):
        for off in (0, 1):
            say("gemv edge", M, K, "offset", off)
            y = gemv_dev(ctx, W, x, M, K, off)
            assert [int(v) for v in y] == e["y"], (M, K, off)


@pytest.mark.parametrize("M,K", spec.GEMV_SHAPES)
def test_gemv_tinyllama_shapes(ctx, M, K):
    W, x = spec.gemv_inputs_ref(O.synth, M, K)
    g = golden("gemv.json")["shapes"][f"{M}x{K}"]
    say("gemv shape", M, K)
    y = gemv_dev(ctx, W, x, M, K)
    assert O.fnv(y) == g["fnv"]


@pytest.mark.parametrize("M,K", [(1, 2), (1, 3), (63, 130), (64, 4096), (33, 4098), (3, 12288),
                                 (17, 8200), (1000, 688), (2500, 256), (5, 12289)])
def test_gemv_random_vs_oracle(ctx, M, K):
    rng = np.random.default_rng(M * 7919 + K)
    W = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=M * K, dtype=np.int64)
    x = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=K, dtype=np.int64)
    want = O.gemv(W, x, M, K)
    for off in (0, 1):
        say("gemv random", M, K, "offset", off)
        assert np.array_equal(gemv_dev(ctx, W, x, M, K, off), want), (M, K, off)


GEMM_KERNELS = [pytest.param(intllm.GEMM_VALU, id="valu"), pytest.param(intllm.GEMM_I8, id="i8"),
                pytest.param(intllm.GEMM_I8_PLANES, id="i8planes")]


@pytest.mark.parametrize("kernel", GEMM_KERNELS)
@pytest.mark.parametrize("T,N,K", [(1, 1, 1), (3, 5, 7), (64, 64, 16), (65, 70, 33),
                                   (130, 129, 688), (128, 256, 2048), (64, 64, 8192),
                                   (70, 33, 1031), (200, 96, 96), (3, 5, 20000),
                                   (1030, 37, 1031), (1024, 64, 8192)])
def test_gemm_random_vs_oracle(ctx, oracle, T, N, K, kernel):
    """Full-range int64 operands.  The cases cover partial tiles, a k tail
    (K not a multiple of 32), odd K (8-byte loads), K split across blocks
    (64x64x8192: one tile, many splits), K past one int32 accumulation run of
    the int8 kernel (20000), and T >= 1024 (alone and with K splits).  Full-range
    operands leave the int8 kernel's digit window in the first step, so these
    run its every-pair pass."""
    rng = np.random.default_rng(T * 31 + N * 7 + K)
    W = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=N * K, dtype=np.int64)
    X = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=T * K, dtype=np.int64)
    want = np.empty(T * N, dtype=np.int64)
    oracle.q48o_gemm(want.ctypes.data, W.ctypes.data, X.ctypes.data, T, N, K)
    dW, dX, dY = ctx.to_device(W), ctx.to_device(X), ctx.buffer(T * N)
    say("gemm", T, N, K, "kernel", kernel)
    ctx.gemm(dY.ptr, dW.ptr, dX.ptr, T, N, K, kernel)
    assert np.array_equal(dY.download(), want)
    for b in (dW, dX, dY):
        b.free()


def _bf16ish(rng, n, scale):
    """Values with 8 significant bits around `scale` (a bfloat16 weight in
    Q16.48), both signs, and a few zeros."""
    m = rng.integers(128, 256, size=n).astype(np.int64)
    e = rng.integers(-6, 1, size=n)
    v = np.array([int(a) << max(0, int(scale) + int(b) - 7) for a, b in zip(m, e)], dtype=np.int64)
    v *= rng.choice([-1, 1], size=n)
    v[rng.random(n) < 0.01] = 0
    return v


@pytest.mark.parametrize("tokens,kernel", [pytest.param(96, intllm.GEMM_I8_FUSED, id="fused"),
                                           pytest.param(300, intllm.GEMM_I8_PLANES, id="planes")])
@pytest.mark.parametrize("case", ["plain", "ext", "late_w", "late_x", "big_w", "ovf_w",
                                  "lo0", "lo4", "zero_w", "split"])
def test_gemm_digit_windows(ctx, oracle, case, tokens, kernel):
    """The int8 GEMM's digit-plane window (X digits 0..6 against four W
    planes chosen from the block's first W tile, plus the plane below in the
    steps that reach it; blocks leaving it redone with every pair) against the
    oracle: weights with 8 significant bits (bfloat16-like) and activations
    below 2^55, a W plane below the window in one step ("ext"), a step late
    in K whose W or X digits leave the window ("late_w", "late_x"), W values
    at the high-word bound that is treated as a possible overflow ("big_w")
    and values that do overflow v + C ("ovf_w"), windows at both ends of the
    plane range ("lo0", "lo4"), an all-zero W tile, and K split across blocks
    with some splits redone ("split").  Both int8 kernels run each case: the
    one that splits tiles into digits inside its k loop (96 tokens) and the
    one fed digit planes split beforehand (300: a ragged last token tile)."""
    rng = np.random.default_rng(sum(map(ord, case)))
    T, N, K = (tokens - 32, 64, 8192) if case == "split" else (tokens, 130, 1000)
    scale = {"lo0": 27, "lo4": 58}.get(case, 42)
    W = _bf16ish(rng, N * K, scale)
    X = rng.integers(-(1 << 52), 1 << 52, size=T * K, dtype=np.int64)
    if case == "ext":
        W[5 * K + 100] = 3 << 10            # digit 1, below a window of planes 2..5
    elif case == "late_w":
        W[7 * K + 900] = 1 << 60            # plane 7 in the 29th step
    elif case == "late_x":
        X[3 * K + 950] = -(1 << 58)
    elif case == "big_w":
        W[2 * K + 40] = 0x7F7F7F7F00000000  # high word at the bound, no overflow
    elif case == "ovf_w":
        W[K + 17] = spec.INT64_MAX
        W[9 * K + 500] = 0x7F7F7F7F7F7F7F80  # 2^63 - C: the first value that overflows
        X[11 * K + 500] = 0x7F7F7F7F7F7F7F90
    elif case == "zero_w":
        W[:64 * K] = 0
    elif case == "split":
        W[30 * K + 7000] = -(1 << 62)        # one k range of one row tile leaves the window
    want = np.empty(T * N, dtype=np.int64)
    oracle.q48o_gemm(want.ctypes.data, W.ctypes.data, X.ctypes.data, T, N, K)
    dW, dX, dY = ctx.to_device(W), ctx.to_device(X), ctx.buffer(T * N)
    say("gemm window", case, T, N, K)
    ctx.gemm(dY.ptr, dW.ptr, dX.ptr, T, N, K, kernel)
    got = dY.download()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (case, bad[:5])
    for b in (dW, dX, dY):
        b.free()


def test_gemm_prepared_planes(ctx, oracle):
    """q48_gemm_prepared: W's digit planes prepared once (q48_gemm_prepare),
    then GEMMs of 1, 3, 17, 64, 128 and 300 tokens (the GEMV for one token,
    else the planes path with W's planes read from the prepared buffer) over
    bfloat16-like weights with one row tile leaving the digit window (its
    blocks redone from W itself), against the oracle; then the buffer
    re-prepared from other weights.  Misaligned buffers are refused."""
    N, K = 1030, 1000
    rng = np.random.default_rng(99)
    W = _bf16ish(rng, N * K, 42)
    W[40 * K + 333] = 1 << 61
    need = intllm.Context.gemm_planes_bytes(N, K)
    assert need >= N * K * 8
    dW, dP = ctx.to_device(W), ctx.buffer(need // 8 + 2)
    ctx.gemm_prepare(dP.ptr, dW.ptr, N, K)
    for T in (1, 3, 17, 64, 128, 300):
        X = rng.integers(-(1 << 52), 1 << 52, size=T * K, dtype=np.int64)
        want = np.empty(T * N, dtype=np.int64)
        oracle.q48o_gemm(want.ctypes.data, W.ctypes.data, X.ctypes.data, T, N, K)
        dX, dY = ctx.to_device(X), ctx.buffer(T * N)
        say("gemm prepared", T, N, K)
        ctx.gemm_prepared(dY.ptr, dW.ptr, dP.ptr, dX.ptr, T, N, K)
        assert np.array_equal(dY.download(), want), T
        dX.free()
        dY.free()
    W2 = _bf16ish(rng, N * K, 35)
    dW2 = ctx.to_device(W2)
    ctx.gemm_prepare(dP.ptr, dW2.ptr, N, K)
    T = 256
    X = rng.integers(-(1 << 52), 1 << 52, size=T * K, dtype=np.int64)
    want = np.empty(T * N, dtype=np.int64)
    oracle.q48o_gemm(want.ctypes.data, W2.ctypes.data, X.ctypes.data, T, N, K)
    dX, dY = ctx.to_device(X), ctx.buffer(T * N)
    say("gemm prepared again", T, N, K)
    ctx.gemm_prepared(dY.ptr, dW2.ptr, dP.ptr, dX.ptr, T, N, K)
    assert np.array_equal(dY.download(), want)
    with pytest.raises(intllm.Q48Error):
        ctx.gemm_prepare(dP.ptr + 8, dW2.ptr, N, K)
    with pytest.raises(intllm.Q48Error):
        ctx.gemm_prepared(dY.ptr, dW2.ptr, dP.ptr + 8, dX.ptr, T, N, K)
    for b in (dW, dW2, dP, dX, dY):
        b.free()


@pytest.mark.parametrize("kernel", GEMM_KERNELS)
def test_gemm_extreme_digits(ctx, oracle, kernel):
    """INT64_MIN has every int8 digit at -128 (the largest digit products);
    with K = 16352 + 8 one block accumulates the longest int32 run the int8
    kernel allows, then more.  Mixed INT64_MIN / INT64_MAX / 0 / -1 / C
    operands exercise the digit offsets, and the unaligned views (one
    element in) the 8-byte load path."""
    T, N, K = 40, 36, 16360
    rng = np.random.default_rng(11)
    pool = np.array([spec.INT64_MIN, spec.INT64_MAX, 0, -1, 0x0080808080808080], dtype=np.int64)
    for name, W, X in (
        ("all-min", np.full(N * K, spec.INT64_MIN, np.int64), np.full(T * K, spec.INT64_MIN, np.int64)),
        ("mixed", pool[rng.integers(0, 5, N * K)], pool[rng.integers(0, 5, T * K)]),
    ):
        want = np.empty(T * N, dtype=np.int64)
        oracle.q48o_gemm(want.ctypes.data, W.ctypes.data, X.ctypes.data, T, N, K)
        for off in (0, 1):
            pad = np.zeros(off, dtype=np.int64)
            dW = ctx.to_device(np.concatenate([pad, W]))
            dX = ctx.to_device(np.concatenate([pad, X]))
            dY = ctx.buffer(T * N + off)
            say("gemm extreme", name, "offset", off, "kernel", kernel)
            ctx.gemm(dY.at(off), dW.at(off), dX.at(off), T, N, K, kernel)
            assert np.array_equal(dY.download()[off:], want), (name, off)
            for b in (dW, dX, dY):
                b.free()


def test_rmsnorm(ctx, oracle):
    g = golden("ops.json")["rmsnorm"]
    for dim, want in g.items():
        dim = int(dim)
        x, w = spec.rmsnorm_inputs(O.synth, dim)
        dx, dw, do = ctx.to_device(x), ctx.to_device(w), ctx.buffer(dim)
        say("rmsnorm", dim)
        ctx.rmsnorm(do.ptr, dx.ptr, dw.ptr, dim)
        assert O.fnv(do.download()) == want, dim
    # extremes: sum of squares wraps int128, mean < 0 -> inv_sqrt 0
    rng = np.random.default_rng(2)
    for dim in (1, 3, 4096, 5000):
        x = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=dim, dtype=np.int64)
        w = rng.integers(-ONE, ONE, size=dim, dtype=np.int64)
        want = np.empty(dim, dtype=np.int64)
        oracle.q48o_rmsnorm(want.ctypes.data, x.ctypes.data, w.ctypes.data, dim)
        dx, dw, do = ctx.to_device(x), ctx.to_device(w), ctx.buffer(dim)
        say("rmsnorm extreme", dim)
        ctx.rmsnorm(do.ptr, dx.ptr, dw.ptr, dim)
        assert np.array_equal(do.download(), want), dim


def test_rope_tables_and_apply(ctx):
    g = golden("ops.json")["rope"]
    for (hd, ms, th) in spec.ROPE_TABLES:
        say("rope tables", hd, ms, th)
        ctx.rope_init(hd, ms, th)
        cp, sp = ctx.rope_tables()
        n = ms * hd // 2
        c = np.empty(n, dtype=np.int64)
        s = np.empty(n, dtype=np.int64)
        intllm.check("d2h", intllm.hip_lib().q48_memcpy_d2h(ctx.h, c.ctypes.data, cp, n * 8))
        intllm.check("d2h", intllm.hip_lib().q48_memcpy_d2h(ctx.h, s.ctypes.data, sp, n * 8))
        e = g[f"{hd}x{ms}x{th}"]
        assert O.fnv(c) == e["cos"] and O.fnv(s) == e["sin"], (hd, ms)
        if "apply" in e:
            v0 = O.synth("rope.vec", 1, hd, spec.SEED_OPS, spec.SIGMA_ACT, 0)
            dv = ctx.buffer(hd)
            for pos, want in enumerate(e["apply"]):
                dv.upload(v0)
                ctx.rope(dv.ptr, 1, hd, pos)
                assert O.fnv(dv.download()) == want, pos


def test_rope_errors(ctx):
    ctx.rope_init(32, 64, 10000)
    d = ctx.buffer(64)
    with pytest.raises(intllm.Q48Error) as e:
        ctx.rope(d.ptr, 2, 32, 64)
    assert e.value.code == intllm.Q48_ERANGE
    with pytest.raises(intllm.Q48Error) as e:
        ctx.rope(d.ptr, 1, 64, 0)
    assert e.value.code == intllm.Q48_ESTATE


@pytest.mark.parametrize("nh,nkv,hd,max_seq,positions", [
    (8, 2, 32, 64, [0, 1, 5, 63]),
    (32, 4, 64, 600, [0, 130, 200, 257, 300, 599]),
    (4, 4, 64, 40, [0, 39]),
    (6, 1, 128, 300, [257]),
])
def test_attention_vs_oracle(ctx, oracle, nh, nkv, hd, max_seq, positions):
    rng = np.random.default_rng(nh * 100 + hd)
    L = 2
    kvd = nkv * hd
    kc = (rng.standard_normal(L * max_seq * kvd) * ONE).astype(np.int64)
    vc = (rng.standard_normal(L * max_seq * kvd) * ONE).astype(np.int64)
    dk, dv = ctx.to_device(kc), ctx.to_device(vc)
    for pos in positions:
        for layer in range(L):
            q = (rng.standard_normal(nh * hd) * 3 * ONE).astype(np.int64)
            kn = (rng.standard_normal(kvd) * ONE).astype(np.int64)
            vn = (rng.standard_normal(kvd) * ONE).astype(np.int64)
            out = np.empty(nh * hd, dtype=np.int64)
            oracle.q48o_attn_decode(out.ctypes.data, q.ctypes.data, kc.ctypes.data, vc.ctypes.data,
                                    kn.ctypes.data, vn.ctypes.data, layer, pos, nh, nkv, hd, max_seq)
            dq, dkn, dvn, do = ctx.to_device(q), ctx.to_device(kn), ctx.to_device(vn), ctx.buffer(nh * hd)
            say("attention", nh, nkv, hd, max_seq, "pos", pos, "layer", layer)
            ctx.attn_decode(do.ptr, dq.ptr, dk.ptr, dv.ptr, dkn.ptr, dvn.ptr, layer, pos, nh, nkv, hd, max_seq)
            assert np.array_equal(do.download(), out), (pos, layer)
            # the cache write at [layer][pos] happened exactly like the oracle's
            assert np.array_equal(dk.download(), kc) and np.array_equal(dv.download(), vc)
            for b in (dq, dkn, dvn, do):
                b.free()
    dk.free()
    dv.free()


def test_silu_mul_vs_oracle(ctx, oracle):
    x, y = spec.fp_inputs()
    rng = np.random.default_rng(4)
    g = np.concatenate([x, (rng.standard_normal(5632) * 4 * ONE).astype(np.int64)])
    u = np.concatenate([y, (rng.standard_normal(5632) * ONE).astype(np.int64)])
    n = g.size
    want = np.empty(n, dtype=np.int64)
    oracle.q48o_silu_mul(want.ctypes.data, g.ctypes.data, u.ctypes.data, n)
    dg, du, do = ctx.to_device(g), ctx.to_device(u), ctx.buffer(n)
    say("silu_mul", n)
    ctx.silu_mul(do.ptr, dg.ptr, du.ptr, n)
    assert np.array_equal(do.download(), want)


def test_add_embed_argmax(ctx):
    rng = np.random.default_rng(8)
    a = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=3001, dtype=np.int64)
    b = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=3001, dtype=np.int64)
    da, db = ctx.to_device(a), ctx.to_device(b)
    say("add")
    ctx.add(da.ptr, db.ptr, a.size)
    assert np.array_equal(da.download(), (a.view(np.uint64) + b.view(np.uint64)).view(np.int64))
    table = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=7 * 300, dtype=np.int64)
    dt, do = ctx.to_device(table), ctx.buffer(300)
    say("embed")
    ctx.embed(do.ptr, dt.ptr, 5, 300)
    assert np.array_equal(do.download(), table[1500:1800])
    # argmax: first index of the maximum, ties included
    for n in (1, 2, 1023, 1025, 32000):
        v = rng.integers(-1000, 1000, size=n, dtype=np.int64)
        if n > 10:
            v[n // 3] = v[n - 2] = v.max() + 5
        dvv = ctx.to_device(v)
        say("argmax", n)
        assert ctx.argmax(dvv.ptr, n) == int(np.argmax(v))
        dvv.free()


@pytest.mark.parametrize("n", [1, 1000, 8191, 8192, 9001, 32000])
def test_argmax_step_and_record(ctx, n):
    """q48_argmax_step and q48_argmax_record_step (the decode step's token
    choice, llama_int.c:2888-2893: the first maximum) against numpy over
    several steps in a row, with ties across the blocks' chunks, INT64_MIN
    and INT64_MAX entries, and the state (token, pos + 1, count + 1), the
    tokens array and the recorded rows checked after every step; the record
    stops at its capacity and the tokens at theirs."""
    lib = intllm.hip_lib()
    rng = np.random.default_rng(n)
    steps, rec_cap, tok_cap = 5, 3, 4
    rows = []
    for s in range(steps):
        v = rng.integers(-(1 << 40), 1 << 40, size=n, dtype=np.int64)
        if s == 1:
            v[:] = spec.INT64_MIN                       # all equal: index 0
        if s == 2 and n > 10:
            v[n // 3] = v[n - 1] = v[2 * n // 3] = spec.INT64_MAX   # first of three
        if s == 3:
            v[rng.integers(0, n, size=min(n, 7))] = v.max()      # repeated maximum
        rows.append(v)
    dv = ctx.buffer(n)
    tokens = ctx.buffer(tok_cap // 2)   # int32 tokens in int64 words
    rec = ctx.buffer(rec_cap * n)
    rec.upload(np.zeros(rec_cap * n, dtype=np.int64))
    for fused in (False, True):
        assert lib.q48_step_mode(ctx.h, 1) == 0
        assert lib.q48_step_set(ctx.h, 11, 40) == 0
        tokens.upload(np.full(tok_cap // 2, -1, dtype=np.int64))
        want_tok = []
        for s, v in enumerate(rows):
            dv.upload(v)
            if fused:
                rc = lib.q48_argmax_record_step(ctx.h, dv.ptr, n, tokens.ptr, tok_cap, rec.ptr,
                                                rec_cap)
            else:
                rc = lib.q48_argmax_step(ctx.h, dv.ptr, n, tokens.ptr, tok_cap)
            assert rc == 0
            want_tok.append(int(np.argmax(v)))
            tok, pos, cnt = C.c_int(), C.c_int(), C.c_int()
            assert lib.q48_step_get(ctx.h, C.byref(tok), C.byref(pos), C.byref(cnt)) == 0
            assert (tok.value, pos.value, cnt.value) == (want_tok[-1], 41 + s, s + 1), (fused, s)
        got = tokens.download().view(np.int32)[:tok_cap]
        assert list(got) == want_tok[:tok_cap]
        if fused:
            r = rec.download().reshape(rec_cap, n)
            for s in range(rec_cap):
                assert np.array_equal(r[s], rows[s])
        assert lib.q48_step_mode(ctx.h, 0) == 0
    for b in (dv, tokens, rec):
        b.free()


def test_abi_rejects_bad_arguments(ctx):
    lib = intllm.hip_lib()
    assert lib.q48_gemv(ctx.h, None, None, None, 4, 4) == intllm.Q48_EINVAL
    d = ctx.buffer(16)
    assert lib.q48_gemv(ctx.h, d.ptr, d.ptr, d.ptr, 0, 4) == intllm.Q48_EINVAL
    assert lib.q48_gemv(ctx.h, d.ptr, d.ptr + 4, d.ptr, 1, 1) == intllm.Q48_EINVAL
    assert lib.q48_attn_decode(ctx.h, d.ptr, d.ptr, d.ptr, d.ptr, d.ptr, d.ptr, 0, 5, 2, 1, 8,
                               4) == intllm.Q48_ERANGE
    assert lib.q48_attn_decode(ctx.h, d.ptr, d.ptr, d.ptr, d.ptr, d.ptr, d.ptr, 0, 0, 3, 2, 8,
                               4) == intllm.Q48_EINVAL
    assert lib.q48_embed(ctx.h, d.ptr, d.ptr, -1, 4) == intllm.Q48_ERANGE


# ---------------------------------------------------------------------------
# fused decode ops: each equals the composition of the separate reference ops
# ---------------------------------------------------------------------------

def _rms(oracle, x, w):
    out = np.empty(x.size, dtype=np.int64)
    oracle.q48o_rmsnorm(out.ctypes.data, x.ctypes.data, w.ctypes.data, x.size)
    return out


@pytest.mark.parametrize("M,K", [(2560, 2048), (32000, 2048), (64, 256), (17, 688), (9, 7681),
                                 (5, 129)])
def test_rmsnorm_gemv_fused(ctx, oracle, M, K):
    rng = np.random.default_rng(M + K)
    W = (rng.standard_normal(M * K) * spec.SIGMA_W).astype(np.int64)
    x = (rng.standard_normal(K) * 3 * ONE).astype(np.int64)
    w = (rng.standard_normal(K) * ONE).astype(np.int64)
    want = O.gemv(W, _rms(oracle, x, w), M, K)
    dW, dx, dw, dy = ctx.to_device(W), ctx.to_device(x), ctx.to_device(w), ctx.buffer(M)
    say("rmsnorm_gemv", M, K)
    ctx.rmsnorm_gemv(dy.ptr, dW.ptr, dx.ptr, dw.ptr, M, K)
    assert np.array_equal(dy.download(), want)
    for b in (dW, dx, dw, dy):
        b.free()


@pytest.mark.parametrize("M,K", [(2048, 2048), (2048, 5632), (256, 688), (3, 7681), (7, 33),
                                 (4616, 2048)])
def test_gemv_residual_fused(ctx, M, K):
    rng = np.random.default_rng(M * 3 + K)
    W = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=M * K, dtype=np.int64)
    x = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=K, dtype=np.int64)
    h = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=M, dtype=np.int64)
    want = (h.view(np.uint64) + O.gemv(W, x, M, K).view(np.uint64)).view(np.int64)
    dW, dx, dh = ctx.to_device(W), ctx.to_device(x), ctx.to_device(h)
    say("gemv_residual", M, K)
    ctx.gemv_residual(dh.ptr, dW.ptr, dx.ptr, M, K)
    assert np.array_equal(dh.download(), want)
    for b in (dW, dx, dh):
        b.free()


@pytest.mark.parametrize("ffn,K", [(5632, 2048), (688, 256), (13, 64), (6, 7681)])
def test_rmsnorm_gemv_swiglu_fused(ctx, oracle, ffn, K):
    rng = np.random.default_rng(ffn + 7 * K)
    W = (rng.standard_normal(2 * ffn * K) * spec.SIGMA_W * 20).astype(np.int64)
    x = (rng.standard_normal(K) * ONE).astype(np.int64)
    w = (rng.standard_normal(K) * ONE).astype(np.int64)
    t = O.gemv(W, _rms(oracle, x, w), 2 * ffn, K)
    want = np.empty(ffn, dtype=np.int64)
    g, u = t[:ffn].copy(), t[ffn:].copy()
    oracle.q48o_silu_mul(want.ctypes.data, g.ctypes.data, u.ctypes.data, ffn)
    dW, dx, dw, do = ctx.to_device(W), ctx.to_device(x), ctx.to_device(w), ctx.buffer(ffn)
    say("swiglu", ffn, K)
    ctx.rmsnorm_gemv_swiglu(do.ptr, dW.ptr, dx.ptr, dw.ptr, ffn, K)
    assert np.array_equal(do.download(), want)
    for b in (dW, dx, dw, do):
        b.free()


@pytest.mark.parametrize("one_launch", [(True, True), (True, False), (False, True)],
                         ids=["one_launch", "one_launch_valu_scores", "three_launches"])
@pytest.mark.parametrize("nh,nkv,hd,max_seq,positions", [
    (8, 2, 32, 64, [0, 1, 63]),
    (32, 4, 64, 300, [0, 7, 299]),
    # from q48_attn_split_min() (256) on, the split (chunked) kernels; chunk
    # edges 767/768 of the three-launch form
    (32, 4, 64, 1300, [255, 256, 511, 512, 767, 768, 1299]),
    (8, 2, 32, 600, [513, 599]),
    # a group of 3 query heads: rows 3..15 of the matrix-core scores are padding
    (12, 4, 64, 600, [520, 599]),
    # head_dim 128: chunks of 128 positions
    (16, 4, 128, 700, [512, 639, 640, 699]),
    # the largest one-launch grid of the TinyLlama heads: 16 chunks x 32 heads
    (32, 4, 64, 4096, [2047, 2048, 4095]),
])
def test_attention_rope_fused(ctx, oracle, nh, nkv, hd, max_seq, positions, one_launch):
    """one_launch = (one-launch split form, its scores on the matrix cores
    for head_dim 64): every form against the oracle."""
    ctx.set_attn_one_launch(one_launch[0])
    ctx.set_attn_g_mfma(one_launch[1])
    try:
        _attention_rope_case(ctx, oracle, nh, nkv, hd, max_seq, positions)
        assert ctx.attn_status() == 0
    finally:
        ctx.set_attn_one_launch(True)
        ctx.set_attn_g_mfma(True)


@pytest.mark.parametrize("full_keys", [False, True], ids=["normal_keys", "full_range_keys"])
def test_attention_full_range_values(ctx, oracle, full_keys):
    """Values spread over the whole int64 range (and, in one case, keys too,
    so that scores wrap and the softmax weights take their extremes): the
    single-block and split kernels' value products against the oracle."""
    _attention_rope_case(ctx, oracle, 32, 4, 64, 1400, [40, 200, 300, 1300],
                         full_values=True, full_keys=full_keys)
    assert ctx.attn_status() == 0


def _attention_rope_case(ctx, oracle, nh, nkv, hd, max_seq, positions, full_values=False,
                         full_keys=False):
    rng = np.random.default_rng(nh + hd + max_seq)
    kvd = nkv * hd
    kc = (rng.standard_normal(2 * max_seq * kvd) * ONE).astype(np.int64)
    vc = (rng.standard_normal(2 * max_seq * kvd) * ONE).astype(np.int64)
    if full_keys:
        kc = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=kc.size, dtype=np.int64,
                          endpoint=True)
    if full_values:
        vc = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=vc.size, dtype=np.int64,
                          endpoint=True)
        vc[::97] = spec.INT64_MIN
        vc[1::89] = spec.INT64_MAX
    cos_t = np.empty(max_seq * hd // 2, dtype=np.int64)
    sin_t = np.empty(max_seq * hd // 2, dtype=np.int64)
    oracle.q48o_rope_tables(cos_t.ctypes.data, sin_t.ctypes.data, hd, max_seq, 10000)
    ctx.rope_init(hd, max_seq, 10000)
    dk, dv = ctx.to_device(kc), ctx.to_device(vc)
    for pos in positions:
        q = (rng.standard_normal(nh * hd) * 3 * ONE).astype(np.int64)
        kn = (rng.standard_normal(kvd) * ONE).astype(np.int64)
        vn = (rng.standard_normal(kvd) * ONE).astype(np.int64)
        qr, kr = q.copy(), kn.copy()
        for h in range(nh):
            oracle.q48o_rope_apply(cos_t.ctypes.data, sin_t.ctypes.data, hd // 2,
                                   qr[h * hd:].ctypes.data, pos)
        for h in range(nkv):
            oracle.q48o_rope_apply(cos_t.ctypes.data, sin_t.ctypes.data, hd // 2,
                                   kr[h * hd:].ctypes.data, pos)
        out = np.empty(nh * hd, dtype=np.int64)
        oracle.q48o_attn_decode(out.ctypes.data, qr.ctypes.data, kc.ctypes.data, vc.ctypes.data,
                                kr.ctypes.data, vn.ctypes.data, 1, pos, nh, nkv, hd, max_seq)
        dq, dkn, dvn, do = ctx.to_device(q), ctx.to_device(kn), ctx.to_device(vn), ctx.buffer(nh * hd)
        say("attention+rope", nh, nkv, hd, "max_seq", max_seq, "pos", pos)
        ctx.attn_decode_rope(do.ptr, dq.ptr, dk.ptr, dv.ptr, dkn.ptr, dvn.ptr, 1, pos, nh, nkv, hd,
                             max_seq)
        assert np.array_equal(do.download(), out), pos
        assert np.array_equal(dk.download(), kc) and np.array_equal(dv.download(), vc)
        # the same with the idle compute units reading another buffer meanwhile
        do2 = ctx.buffer(nh * hd)
        ctx.attn_decode_rope_prefetch(do2.ptr, dq.ptr, dk.ptr, dv.ptr, dkn.ptr, dvn.ptr, 1, pos, nh,
                                      nkv, hd, max_seq, dv.ptr, (vc.size * 8) // 16 * 16)
        assert np.array_equal(do2.download(), out), pos
        assert np.array_equal(dk.download(), kc) and np.array_equal(dv.download(), vc)
        do2.free()
        for b in (dq, dkn, dvn, do):
            b.free()


def rms_inv_exact(oracle, x):
    """The scalar of rmsnorm (llama_int.c:1049-1055) with Python integers:
    int128-wrapped sum of squares, floor shift, truncating division."""
    ss = sum(int(v) * int(v) for v in x)
    ss = ((ss + (1 << 127)) % (1 << 128)) - (1 << 127)
    q = ss >> 48
    ms = abs(q) // len(x) * (1 if q >= 0 else -1)
    ms = spec.wrap64(spec.wrap64(ms) + 2814749767)
    return oracle.q48o_fp_inv_sqrt(ms)


@pytest.mark.parametrize("dim", [1, 7, 256, 2048, 5000])
def test_rms_inv_and_embed_rms(ctx, oracle, dim):
    rng = np.random.default_rng(dim)
    table = (rng.standard_normal(3 * dim) * 2 * ONE).astype(np.int64)
    dt, do, dr = ctx.to_device(table), ctx.buffer(dim), ctx.buffer(1)
    say("embed_rms", dim)
    ctx.embed_rms(do.ptr, dt.ptr, 2, dim, dr.ptr)
    row = table[2 * dim:3 * dim]
    assert np.array_equal(do.download(), row)
    assert int(dr.download()[0]) == rms_inv_exact(oracle, row)
    ctx.rms_inv(dr.ptr, dt.ptr, dim)
    assert int(dr.download()[0]) == rms_inv_exact(oracle, table[:dim])


@pytest.mark.parametrize("M,K", [(2560, 2048), (32000, 2048), (64, 256), (9, 7681)])
def test_norm_gemv_with_r(ctx, oracle, M, K):
    rng = np.random.default_rng(M * 5 + K)
    W = (rng.standard_normal(M * K) * spec.SIGMA_W).astype(np.int64)
    x = (rng.standard_normal(K) * 3 * ONE).astype(np.int64)
    w = (rng.standard_normal(K) * ONE).astype(np.int64)
    want = O.gemv(W, _rms(oracle, x, w), M, K)
    dW, dx, dw, dy, dr = ctx.to_device(W), ctx.to_device(x), ctx.to_device(w), ctx.buffer(M), ctx.buffer(1)
    say("norm_gemv", M, K)
    ctx.rms_inv(dr.ptr, dx.ptr, K)
    ctx.norm_gemv(dy.ptr, dW.ptr, dx.ptr, dw.ptr, dr.ptr, M, K)
    assert np.array_equal(dy.download(), want)
    for b in (dW, dx, dw, dy, dr):
        b.free()


@pytest.mark.parametrize("ffn,K", [(5632, 2048), (688, 256), (6, 7681)])
def test_norm_gemv_swiglu_with_r(ctx, oracle, ffn, K):
    rng = np.random.default_rng(ffn + 3 * K)
    W = (rng.standard_normal(2 * ffn * K) * spec.SIGMA_W * 20).astype(np.int64)
    x = (rng.standard_normal(K) * ONE).astype(np.int64)
    w = (rng.standard_normal(K) * ONE).astype(np.int64)
    t = O.gemv(W, _rms(oracle, x, w), 2 * ffn, K)
    want = np.empty(ffn, dtype=np.int64)
    g, u = t[:ffn].copy(), t[ffn:].copy()
    oracle.q48o_silu_mul(want.ctypes.data, g.ctypes.data, u.ctypes.data, ffn)
    dW, dx, dw, do, dr = ctx.to_device(W), ctx.to_device(x), ctx.to_device(w), ctx.buffer(ffn), ctx.buffer(1)
    say("norm_gemv_swiglu", ffn, K)
    ctx.rms_inv(dr.ptr, dx.ptr, K)
    ctx.norm_gemv_swiglu(do.ptr, dW.ptr, dx.ptr, dw.ptr, dr.ptr, ffn, K)
    assert np.array_equal(do.download(), want)
    for b in (dW, dx, dw, do, dr):
        b.free()


@pytest.mark.parametrize("M,K", [(2048, 2048), (2048, 5632), (256, 688), (13, 40), (3, 7681)])
def test_gemv_residual_rms(ctx, oracle, M, K):
    """acc += W x and r_out = statistics of the new acc; three calls in a row
    (the last-block counter must reset itself)."""
    rng = np.random.default_rng(M + 11 * K)
    h = (rng.standard_normal(M) * ONE).astype(np.int64)
    dh, dr = ctx.to_device(h), ctx.buffer(1)
    for it in range(3):
        W = (rng.standard_normal(M * K) * spec.SIGMA_W).astype(np.int64)
        x = (rng.standard_normal(K) * ONE).astype(np.int64)
        h = (h.view(np.uint64) + O.gemv(W, x, M, K).view(np.uint64)).view(np.int64)
        dW, dx = ctx.to_device(W), ctx.to_device(x)
        say("gemv_residual_rms", M, K, "call", it)
        ctx.gemv_residual_rms(dh.ptr, dW.ptr, dx.ptr, M, K, dr.ptr)
        assert np.array_equal(dh.download(), h), it
        assert int(dr.download()[0]) == rms_inv_exact(oracle, h), it
        dW.free()
        dx.free()


# ---------------------------------------------------------------------------
# statistics as per-8-row partial sums (producer) finished by the consumer
# ---------------------------------------------------------------------------

def stats_exact(x):
    """Partial sums of squares of rows 8i..8i+7 as 128-bit (lo, hi) words,
    computed with Python integers (the wrap of an int128 sum)."""
    x = [int(v) for v in x]
    out = []
    for i in range(0, len(x), 8):
        s = sum(v * v for v in x[i:i + 8]) % (1 << 128)
        out += [spec.wrap64(s & ((1 << 64) - 1)), spec.wrap64(s >> 64)]
    return np.array(out, dtype=np.int64)


@pytest.mark.parametrize("dim", [1, 7, 256, 2048, 5000])
def test_rms_stats_and_embed_stats(ctx, dim):
    rng = np.random.default_rng(dim + 1)
    table = (rng.standard_normal(3 * dim) * 2 * ONE).astype(np.int64)
    table[0] = spec.INT64_MIN          # extreme squares wrap like the reference's int128
    sw = intllm.stats_words(dim)
    dt, do, ds = ctx.to_device(table), ctx.buffer(dim), ctx.buffer(sw)
    say("embed_stats", dim)
    ctx.embed_stats(do.ptr, dt.ptr, 2, dim, ds.ptr)
    row = table[2 * dim:3 * dim]
    assert np.array_equal(do.download(), row)
    assert np.array_equal(ds.download(), stats_exact(row))
    ctx.rms_stats(ds.ptr, dt.ptr, dim)
    assert np.array_equal(ds.download(), stats_exact(table[:dim]))


@pytest.mark.parametrize("M,K", [(2560, 2048), (32000, 2048), (64, 256), (9, 7681), (5, 129)])
def test_norm_gemv_with_stats(ctx, oracle, M, K):
    rng = np.random.default_rng(M * 7 + K)
    W = (rng.standard_normal(M * K) * spec.SIGMA_W).astype(np.int64)
    x = (rng.standard_normal(K) * 3 * ONE).astype(np.int64)
    w = (rng.standard_normal(K) * ONE).astype(np.int64)
    want = O.gemv(W, _rms(oracle, x, w), M, K)
    dW, dx, dw, dy = ctx.to_device(W), ctx.to_device(x), ctx.to_device(w), ctx.buffer(M)
    ds = ctx.buffer(intllm.stats_words(K))
    say("norm_gemv_stats", M, K)
    ctx.rms_stats(ds.ptr, dx.ptr, K)
    ctx.norm_gemv_stats(dy.ptr, dW.ptr, dx.ptr, dw.ptr, ds.ptr, M, K)
    assert np.array_equal(dy.download(), want)
    for b in (dW, dx, dw, dy, ds):
        b.free()


@pytest.mark.parametrize("K", [2048, 7681])
def test_norm_gemv_stats_wrapped_sum(ctx, oracle, K):
    """Sums of squares past 2^127 wrap negative in the reference's int128:
    the normalised vector (and so the product) is then exactly zero."""
    rng = np.random.default_rng(K)
    M = 16
    W = (rng.standard_normal(M * K) * spec.SIGMA_W).astype(np.int64)
    x = (rng.standard_normal(K) * ONE).astype(np.int64)
    x[:3] = spec.INT64_MIN
    w = (rng.standard_normal(K) * ONE).astype(np.int64)
    want = O.gemv(W, _rms(oracle, x, w), M, K)
    dW, dx, dw, dy = ctx.to_device(W), ctx.to_device(x), ctx.to_device(w), ctx.buffer(M)
    ds = ctx.buffer(intllm.stats_words(K))
    say("norm_gemv_stats wrapped", M, K)
    ctx.rms_stats(ds.ptr, dx.ptr, K)
    ctx.norm_gemv_stats(dy.ptr, dW.ptr, dx.ptr, dw.ptr, ds.ptr, M, K)
    assert np.array_equal(dy.download(), want)
    for b in (dW, dx, dw, dy, ds):
        b.free()


@pytest.mark.parametrize("ffn,K", [(5632, 2048), (688, 256), (6, 7681)])
def test_norm_gemv_swiglu_with_stats(ctx, oracle, ffn, K):
    rng = np.random.default_rng(ffn + 5 * K)
    W = (rng.standard_normal(2 * ffn * K) * spec.SIGMA_W * 20).astype(np.int64)
    x = (rng.standard_normal(K) * ONE).astype(np.int64)
    w = (rng.standard_normal(K) * ONE).astype(np.int64)
    t = O.gemv(W, _rms(oracle, x, w), 2 * ffn, K)
    want = np.empty(ffn, dtype=np.int64)
    g, u = t[:ffn].copy(), t[ffn:].copy()
    oracle.q48o_silu_mul(want.ctypes.data, g.ctypes.data, u.ctypes.data, ffn)
    dW, dx, dw, do = ctx.to_device(W), ctx.to_device(x), ctx.to_device(w), ctx.buffer(ffn)
    ds = ctx.buffer(intllm.stats_words(K))
    say("norm_gemv_swiglu_stats", ffn, K)
    ctx.rms_stats(ds.ptr, dx.ptr, K)
    ctx.norm_gemv_swiglu_stats(do.ptr, dW.ptr, dx.ptr, dw.ptr, ds.ptr, ffn, K)
    assert np.array_equal(do.download(), want)
    for b in (dW, dx, dw, do, ds):
        b.free()


@pytest.mark.parametrize("persistent", [True, False])
@pytest.mark.parametrize("M,ffn", [(32000, 0), (9001, 0), (0, 5632), (0, 4097)])
def test_long_normed_gemv_persistent(ctx, oracle, M, ffn, persistent):
    """The normed lm_head / gate|up shapes with more row groups than two rounds
    of blocks: persistent blocks looping over row groups (the default) and one
    block per group both give the oracle's bits, with a partial last group
    (9001 rows, ffn 4097)."""
    K = 2048
    rows = M or 2 * ffn
    rng = np.random.default_rng(rows + 3 * K + persistent)
    W = (rng.standard_normal(rows * K) * spec.SIGMA_W * 20).astype(np.int64)
    x = (rng.standard_normal(K) * ONE).astype(np.int64)
    w = (rng.standard_normal(K) * ONE).astype(np.int64)
    t = O.gemv(W, _rms(oracle, x, w), rows, K)
    if ffn:
        want = np.empty(ffn, dtype=np.int64)
        g, u = t[:ffn].copy(), t[ffn:].copy()
        oracle.q48o_silu_mul(want.ctypes.data, g.ctypes.data, u.ctypes.data, ffn)
    else:
        want = t
    dW, dx, dw = ctx.to_device(W), ctx.to_device(x), ctx.to_device(w)
    dy, ds = ctx.buffer(want.size), ctx.buffer(intllm.stats_words(K))
    ctx.set_gemv_persistent(persistent)
    try:
        say("long normed gemv", M, ffn, "persistent", persistent)
        ctx.rms_stats(ds.ptr, dx.ptr, K)
        if ffn:
            ctx.norm_gemv_swiglu_stats(dy.ptr, dW.ptr, dx.ptr, dw.ptr, ds.ptr, ffn, K)
        else:
            ctx.norm_gemv_stats(dy.ptr, dW.ptr, dx.ptr, dw.ptr, ds.ptr, M, K)
        assert np.array_equal(dy.download(), want)
    finally:
        ctx.set_gemv_persistent(True)
    for b in (dW, dx, dw, dy, ds):
        b.free()


@pytest.mark.parametrize("M,K", [(2048, 2048), (2048, 5632), (256, 688), (13, 40), (3, 7681),
                                 (5128, 2048)])
def test_gemv_residual_stats(ctx, oracle, M, K):
    """acc += W x and the partial sums of the new acc, three calls in a row,
    then a consumer GEMV normalising acc with them."""
    rng = np.random.default_rng(M + 13 * K)
    h = (rng.standard_normal(M) * ONE).astype(np.int64)
    dh, ds = ctx.to_device(h), ctx.buffer(intllm.stats_words(M))
    for it in range(3):
        W = (rng.standard_normal(M * K) * spec.SIGMA_W).astype(np.int64)
        x = (rng.standard_normal(K) * ONE).astype(np.int64)
        h = (h.view(np.uint64) + O.gemv(W, x, M, K).view(np.uint64)).view(np.int64)
        dW, dx = ctx.to_device(W), ctx.to_device(x)
        say("gemv_residual_stats", M, K, "call", it)
        ctx.gemv_residual_stats(dh.ptr, dW.ptr, dx.ptr, M, K, ds.ptr)
        assert np.array_equal(dh.download(), h), it
        assert np.array_equal(ds.download(), stats_exact(h)), it
        dW.free()
        dx.free()
    # the consumer side: the same r as rmsnorm of the updated vector
    N = 24
    Wn = (rng.standard_normal(N * M) * spec.SIGMA_W).astype(np.int64)
    nw = (rng.standard_normal(M) * ONE).astype(np.int64)
    dWn, dnw, dy = ctx.to_device(Wn), ctx.to_device(nw), ctx.buffer(N)
    ctx.norm_gemv_stats(dy.ptr, dWn.ptr, dh.ptr, dnw.ptr, ds.ptr, N, M)
    assert np.array_equal(dy.download(), O.gemv(Wn, _rms(oracle, h, nw), N, M))
    for b in (dWn, dnw, dy, dh, ds):
        b.free()


# ---- bfloat16-resident weights ----------------------------------------------

def _bf16_values(oracle, bits):
    """bfloat16_to_q1648 of each pattern, from the compiled reference's
    table of all 65536 (tests/golden/bf16_to_q48.npz)."""
    return bf16_reference()[np.asarray(bits, dtype=np.uint16).astype(np.int64)]


def test_bf16_pack_every_pattern(ctx, oracle):
    """Every one of the 65536 bfloat16 patterns, converted as the compiled
    reference converts it (safetensors.h:115-152), packs back to bits that convert to the same
    int64; a value with more than 8 significant bits is reported inexact."""
    bits = np.arange(1 << 16, dtype=np.uint16)
    vals = _bf16_values(oracle, bits)
    dv = ctx.to_device(vals)
    db = ctx.buffer(vals.size // 4)   # 2 bytes per element
    say("bf16 pack, all patterns")
    assert ctx.bf16_pack(db.ptr, dv.ptr, vals.size)
    packed = db.download().view(np.uint16)
    assert np.array_equal(_bf16_values(oracle, packed), vals)
    bad = ctx.to_device(np.array([0, ONE, 0x123456789, -ONE], dtype=np.int64))
    assert not ctx.bf16_pack(db.ptr, bad.ptr, 4)
    for b in (dv, db, bad):
        b.free()


def test_bf16_gemv_every_pattern(ctx, oracle):
    """The in-kernel expansion on every bfloat16 pattern (zero, subnormal,
    wrapping left shifts, truncating right shifts, shifts past 64, +-Inf/NaN
    clamps): a 128 x 512 matrix holding all 65536 patterns against random x,
    equal to the int64 GEMV of the expanded matrix and to the oracle."""
    M, K = 128, 512
    rng = np.random.default_rng(5)
    bits = rng.permutation(np.arange(1 << 16, dtype=np.uint16))
    W = _bf16_values(oracle, bits)
    x = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=K, dtype=np.int64)
    want = O.gemv(W, x, M, K)
    dWb = ctx.buffer(M * K // 4)
    dWb.upload(bits.view(np.int64))
    dx, dy = ctx.to_device(x), ctx.buffer(M)
    say("bf16 gemv, all patterns")
    ctx.gemv_bf16(dy.ptr, dWb.ptr, dx.ptr, M, K)
    assert np.array_equal(dy.download(), want)
    for b in (dWb, dx, dy):
        b.free()


def _bf16_matrix(rng, rows, cols, mode="wide"):
    """bfloat16 bits of model-like weights: sign, exponents around 2^-6 (N(0,
    0.02)-sized), any mantissa.  The kernels take a fast path for exponents
    103..126 (2^-24 <= |w| < 1) and recompute a wave's tiles exactly when any
    weight lies outside:
      wide:   exponents 1..140, spread 4 (most waves see an outlier);
      window: exponents 103..126 only (every wave fast);
      mixed:  window, plus an outlier (zero, subnormal, tiny, |w| >= 1,
              inf/NaN) at about 1 in 20000 weights, so fast and recomputed
              waves meet in one launch."""
    n = rows * cols
    if mode == "wide":
        e = np.clip(rng.normal(121, 4, n).round(), 1, 140)
    else:
        e = np.clip(rng.normal(119, 3, n).round(), 103, 126)
    e = e.astype(np.uint16)
    m = rng.integers(0, 128, n, dtype=np.uint16)
    s = rng.integers(0, 2, n, dtype=np.uint16)
    bits = (s << 15) | (e << 7) | m
    if mode == "mixed":
        at = rng.choice(n, size=max(1, n // 20000), replace=False)
        bits[at] = rng.choice(np.array([0x0000, 0x8000, 0x0011, 0x3300, 0xb380, 0x3f80,
                                        0xbfc0, 0x4500, 0x7f80, 0xffc1, 0x3f7f, 0xbf7f], np.uint16), at.size)
    return bits


@pytest.mark.parametrize("mode", ["wide", "window", "mixed"])
@pytest.mark.parametrize("persistent", [True, False])
@pytest.mark.parametrize("M,K", [(2560, 2048), (2048, 5632), (9001, 2048), (32000, 2048),
                                 (100, 512), (1030, 1024)])
def test_bf16_gemv_forms_equal_int64(ctx, oracle, M, K, persistent, mode):
    """Every fused form on bfloat16 weights (plain, normed with partial-sum
    statistics, residual add with the next statistics, gate|up + SwiGLU)
    gives the bits of the same form on the expanded int64 weights, with the
    persistent row-group loop on and off, on the fast path, the exact
    recomputation and a mixture of both."""
    rng = np.random.default_rng(M * 3 + K + 7 * len(mode))
    bits = _bf16_matrix(rng, M, K, mode)
    lut = _bf16_values(oracle, np.arange(1 << 16, dtype=np.uint16))
    W = lut[bits]
    x = (rng.standard_normal(K) * ONE).astype(np.int64)
    nw = (rng.standard_normal(K) * ONE).astype(np.int64)
    h0 = (rng.standard_normal(M) * ONE).astype(np.int64)
    dW, dWb = ctx.to_device(W), ctx.buffer((M * K + 3) // 4)
    dWb.upload(np.concatenate([bits, np.zeros((-M * K) % 4, np.uint16)]).view(np.int64))
    dx, dnw = ctx.to_device(x), ctx.to_device(nw)
    ds = ctx.buffer(intllm.stats_words(K) + 2)
    ctx.rms_stats(ds.ptr, dx.ptr, K)
    ya, yb = ctx.buffer(M), ctx.buffer(M)
    ctx.set_gemv_persistent(persistent)
    try:
        say("bf16 forms", M, K, "persistent", persistent, mode)
        ctx.gemv(ya.ptr, dW.ptr, dx.ptr, M, K)
        ctx.gemv_bf16(yb.ptr, dWb.ptr, dx.ptr, M, K)
        assert np.array_equal(ya.download(), yb.download()), "plain"
        ctx.norm_gemv_stats(ya.ptr, dW.ptr, dx.ptr, dnw.ptr, ds.ptr, M, K)
        ctx.norm_gemv_stats_bf16(yb.ptr, dWb.ptr, dx.ptr, dnw.ptr, ds.ptr, M, K)
        assert np.array_equal(ya.download(), yb.download()), "normed"
        if M % 2 == 0:
            ffn = M // 2
            ctx.norm_gemv_swiglu_stats(ya.ptr, dW.ptr, dx.ptr, dnw.ptr, ds.ptr, ffn, K)
            ctx.norm_gemv_swiglu_stats_bf16(yb.ptr, dWb.ptr, dx.ptr, dnw.ptr, ds.ptr, ffn, K)
            assert np.array_equal(ya.download(ffn), yb.download(ffn)), "swiglu"
        sa, sb = ctx.buffer(intllm.stats_words(M) + 2), ctx.buffer(intllm.stats_words(M) + 2)
        ya.upload(h0)
        yb.upload(h0)
        ctx.gemv_residual_stats(ya.ptr, dW.ptr, dx.ptr, M, K, sa.ptr)
        ctx.gemv_residual_stats_bf16(yb.ptr, dWb.ptr, dx.ptr, M, K, sb.ptr)
        assert np.array_equal(ya.download(), yb.download()), "residual"
        n = intllm.stats_words(M)
        assert np.array_equal(sa.download(n), sb.download(n)), "residual stats"
        for b in (sa, sb):
            b.free()
    finally:
        ctx.set_gemv_persistent(True)
    for b in (dW, dWb, dx, dnw, ds, ya, yb):
        b.free()


def test_graph_drop_and_replace_while_in_flight(ctx):
    """q48_graph_drop, and q48_graph_begin replacing a graph, right after
    q48_graph_launch with no synchronisation between: the launches in flight
    finish before the executable graph is destroyed, and the captured GEMV's
    output equals the eager one's."""
    rng = np.random.default_rng(11)
    M, K = 2048, 2048
    W = rng.integers(-(1 << 46), 1 << 46, M * K, dtype=np.int64)
    x = rng.integers(-(1 << 50), 1 << 50, K, dtype=np.int64)
    dW, dx = ctx.buffer(M * K), ctx.to_device(x)
    dW.upload(W)
    ya, yb = ctx.buffer(M), ctx.buffer(M)
    L = intllm.hip_lib()
    try:
        ctx.gemv(ya.ptr, dW.ptr, dx.ptr, M, K)
        want = ya.download()
        def capture():
            assert L.q48_graph_begin(ctx.h) == 0
            ctx.gemv(yb.ptr, dW.ptr, dx.ptr, M, K)
            assert L.q48_graph_end(ctx.h) == 0

        say("graph drop while in flight")
        capture()
        assert L.q48_graph_launch(ctx.h, 16) == 0
        assert L.q48_graph_drop(ctx.h) == 0
        assert np.array_equal(yb.download(), want), "drop"
        say("graph replaced while in flight")
        capture()
        assert L.q48_graph_launch(ctx.h, 16) == 0
        capture()                                   # replaces the graph in flight
        assert L.q48_graph_launch(ctx.h, 1) == 0
        assert np.array_equal(yb.download(), want), "replace"
        assert L.q48_graph_drop(ctx.h) == 0
    finally:
        for b in (dW, dx, ya, yb):
            b.free()
