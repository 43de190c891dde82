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
