"""The oracle's llama_int.c ops and forward pass against what pins them.

Pins: vectors recorded from the compiled reference (tests/golden/*.json:
matmul_vec, rmsnorm, rope_init / rope_apply, softmax,
transformer_layer_forward, generate); a Python big-int restatement of the
GEMV definition on the int64 extremes; and structural properties (the
GEMM is the GEMV per token, softmax sums to one).
"""
import ctypes as C
import random

import numpy as np
import pytest

import oracle_lib as O
import spec
from conftest import golden

ONE = spec.ONE


def test_gemv_edges_bigint_and_reference(oracle):
    """Extreme operands: oracle == Python int128 definition == reference."""
    g = golden("gemv.json")["edges"]
    cases = spec.gemv_edge_cases()
    assert len(cases) == len(g)
    for (M, K, W, x), e in zip(cases, g):
        assert [int(v) for v in W] == e["W"] and [int(v) for v in x] == e["x"]
        y = O.gemv(W, x, M, K)
        assert [int(v) for v in y] == e["y"], (M, K)
        assert np.array_equal(y, spec.gemv_exact(W, x, M, K)), (M, K)


def test_gemv_random_bigint(oracle):
    rng = np.random.default_rng(5)
    for (M, K) in [(3, 5), (8, 64), (2, 300)]:
        W = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=M * K, dtype=np.int64)
        x = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=K, dtype=np.int64)
        assert np.array_equal(O.gemv(W, x, M, K), spec.gemv_exact(W, x, M, K))


@pytest.mark.parametrize("M,K", spec.GEMV_SHAPES)
def test_gemv_tinyllama_shapes_match_reference(oracle, M, K):
    W, x = spec.gemv_inputs_ref(O.synth, M, K)
    g = golden("gemv.json")["shapes"][f"{M}x{K}"]
    y = O.gemv(W, x, M, K)
    assert O.fnv(y) == g["fnv"]
    assert [int(v) for v in y[:4]] == g["head"]


def test_gemm_is_gemv_per_token(oracle):
    rng = np.random.default_rng(9)
    T, N, K = 5, 7, 33
    W = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=N * K, dtype=np.int64)
    X = rng.integers(spec.INT64_MIN, spec.INT64_MAX, size=T * K, dtype=np.int64)
    Y = np.empty(T * N, dtype=np.int64)
    oracle.q48o_gemm(Y.ctypes.data, W.ctypes.data, X.ctypes.data, T, N, K)
    for t in range(T):
        assert np.array_equal(Y[t * N:(t + 1) * N], spec.gemv_exact(W, X[t * K:(t + 1) * K], N, K))


def test_rmsnorm_matches_reference(oracle):
    g = golden("ops.json")["rmsnorm"]
    for dim, want in g.items():
        dim = int(dim)
        x, w = spec.rmsnorm_inputs(O.synth, dim)
        out = np.empty(dim, dtype=np.int64)
        oracle.q48o_rmsnorm(out.ctypes.data, x.ctypes.data, w.ctypes.data, dim)
        assert O.fnv(out) == want, dim


def test_rope_tables_and_apply_match_reference(oracle):
    g = golden("ops.json")["rope"]
    for (hd, ms, th) in spec.ROPE_TABLES:
        n = ms * hd // 2
        c = np.empty(n, dtype=np.int64)
        s = np.empty(n, dtype=np.int64)
        oracle.q48o_rope_tables(c.ctypes.data, s.ctypes.data, hd, ms, th)
        e = g[f"{hd}x{ms}x{th}"]
        assert O.fnv(c) == e["cos"] and O.fnv(s) == e["sin"], (hd, ms)
        # invariants: every (cos, sin) pair lies on the unit circle, position 0
        # is the identity rotation, and frequency 0 turns by exactly pos radians
        cf, sf = c / 2.0**48, s / 2.0**48
        assert np.abs(cf * cf + sf * sf - 1.0).max() < 1e-9, (hd, ms)
        assert np.abs(cf[: hd // 2] - 1.0).max() < 1e-9 and np.abs(sf[: hd // 2]).max() < 1e-9
        pos = np.arange(ms)
        ang = np.arctan2(sf.reshape(ms, hd // 2)[:, 0], cf.reshape(ms, hd // 2)[:, 0])
        assert np.abs(np.angle(np.exp(1j * (ang - pos)))).max() < 1e-9, (hd, ms)
        if "apply" in e:
            v0 = O.synth("rope.vec", 1, hd, spec.SEED_OPS, spec.SIGMA_ACT, 0)
            for pos, want in enumerate(e["apply"]):
                v = v0.copy()
                oracle.q48o_rope_apply(c.ctypes.data, s.ctypes.data, hd // 2, v.ctypes.data, pos)
                assert O.fnv(v) == want, pos


def test_softmax_matches_reference_and_sums_to_one(oracle):
    g = golden("ops.json")["softmax"]
    for n, want in g.items():
        n = int(n)
        x = spec.softmax_inputs(O.synth, n)
        oracle.q48o_softmax(x.ctypes.data, n)
        assert O.fnv(x) == want, n
        # each p_t is truncated, so the sum is at most n ulps below ONE
        assert ONE - n <= int(x.sum()) <= ONE


def test_layer_forward_matches_reference(oracle):
    g = golden("layer.json")
    m = O.Model(spec.TINY, g["seed"])
    try:
        h = O.synth("layer.hidden", 1, spec.TINY[0], spec.SEED_OPS, spec.SIGMA_W, 1)
        for pos, want in enumerate(g["hidden_fnv_per_pos"]):
            oracle.q48o_layer_forward(m.h, 0, pos, h.ctypes.data)
            assert O.fnv(h) == want, pos
    finally:
        m.free()


def test_tiny_generate_matches_reference(oracle):
    g = golden("tiny_generate.json")
    m = O.Model(spec.TINY, g["seed"])
    try:
        assert g["prompt"] == spec.prompt(g["seed"], 16, spec.TINY[6])
        toks, hs = m.generate(g["prompt"], g["max_new"])
        assert toks == g["tokens"]
        assert hs == g["step_fnv"]
    finally:
        m.free()


def test_forward_range_checks(oracle):
    """llama_forward returns NULL for token/pos out of range (llama_int.c:2813-2820)."""
    m = O.Model(spec.TINY, 1)
    try:
        assert m.forward(spec.TINY[6], 0)[0] == -1
        assert m.forward(-1, 0)[0] == -1
        assert m.forward(5, spec.TINY[7])[0] == -1
        assert m.forward(5, 0)[0] == 0
    finally:
        m.free()


def test_generate_stops_at_max_seq(oracle):
    """generate breaks when pos reaches max_seq (llama_forward's NULL)."""
    cfg = list(spec.TINY)
    cfg[7] = 20
    m = O.Model(tuple(cfg), 2)
    try:
        toks, hs = m.generate(spec.prompt(2, 16, cfg[6]), 32)
        assert len(hs) <= 20 and len(toks) <= 21
    finally:
        m.free()


def test_rng_matches_reference(oracle):
    """rng_seed (SplitMix64) and rng_next (xoroshiro128+), llama_int.c:2909-2929,
    against the reference's own streams."""
    g = golden("sample.json")["rng"]
    for seed, v in g.items():
        st = O.rng_seed(int(seed))
        assert ["%016x" % w for w in st] == v["state"]
        s = (C.c_uint64 * 2)(*st)
        assert ["%016x" % O.load().q48o_rng_next(s) for _ in range(8)] == v["next"]


def test_sample_token_matches_reference(oracle):
    """sample_token (llama_int.c:2958-3039) on 1176 cases: four logit kinds
    (spread, runs of ties, one dominant logit, extreme magnitudes that wrap in
    the temperature division) x temperatures on both sides of the 0.01
    greedy floor x top-k (off, 1, 2, 10, 50, n - 1) x top-p (off, 0.05, 0.5,
    0.9, 0.999, 1.0): the token and the rng state after it equal the
    reference's."""
    for c in golden("sample.json")["cases"]:
        x = spec.sample_logits(c["kind"], c["seed"], c["n"])
        st = [int(v, 16) for v in c["rng_in"]]
        tok, st2 = O.sample(x, c["T"], c["top_k"], c["top_p"], st)
        assert tok == c["token"], c
        assert ["%016x" % v for v in st2] == c["rng_out"], c


def test_sample_token_properties(oracle):
    """Closed forms the reference fixes, on fresh logits: below the 0.01
    floor it is argmax and draws nothing; top_k = 1 always gives the first
    maximum (every other logit is masked to exp(-inf) = 0); with top_p under
    the largest probability only that entry survives."""
    rng = np.random.default_rng(99)
    for _ in range(50):
        n = int(rng.integers(2, 700))
        x = rng.integers(-8 * ONE, 8 * ONE, size=n, dtype=np.int64)
        st = O.rng_seed(int(rng.integers(0, 2**63)))
        am = int(np.argmax(x))
        assert O.sample(x, ONE // 100 - 1, 0, ONE, st) == (am, st)
        assert O.sample(x, ONE // 2, 1, ONE, st)[0] == am
        assert O.sample(x, ONE, 0, 1, st)[0] == am


def test_generate_sampled_matches_reference(oracle):
    """generate() with sampling parameters (llama_int.c:3067-3135) on the tiny
    model: four (temperature, top-k, top-p, seed) settings, 32 new tokens."""
    g = golden("sample.json")["generate_tiny"]
    m = O.Model(spec.TINY, g["seed"])
    try:
        for r in g["runs"]:
            toks, _ = m.generate_sampled(g["prompt"], g["max_new"], r["T"], r["top_k"],
                                         r["top_p"], r["seed"])
            assert toks == r["tokens"], r
    finally:
        m.free()
